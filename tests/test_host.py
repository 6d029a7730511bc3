"""Host-side logic of the drop-in surface (CPU only)."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

import mimansm1_v1_amd as mm
from mimansm1_v1_amd import attention as A
from mimansm1_v1_amd import tuned

ROOT = Path(__file__).resolve().parent.parent

# Public names of attention_tilelang (AT) that are on the attention path.
MIRRORED = ["DTYPE", "AUTOTUNE", "FWD_TILES", "BWD_TILES", "fwd_configs", "bwd_configs",
            "get_kernel", "warmup", "_kernels", "flash_delta", "FlashAttention",
            "flash_attention", "AttnConfig", "RMSNorm", "Rotary", "rotate_half", "apply_rope",
            "Attention", "reference", "rope_reference", "check_math", "check_gpu", "benchmark",
            "tune"]


def test_surface_mirrors_reference_module():
    for name in MIRRORED:
        assert hasattr(A, name), name


def test_check_math_passes():
    assert A.check_math()


def test_attn_config_asserts():
    assert A.AttnConfig().groups == 5
    with pytest.raises(AssertionError):
        A.AttnConfig(n_heads=10, n_kv_heads=3)
    with pytest.raises(AssertionError):
        A.AttnConfig(d_model=1024)
    with pytest.raises(AssertionError):
        A.AttnConfig(head_dim=96, d_model=960, n_heads=10)


def test_get_kernel_cache_keys_and_handles():
    A._kernels.clear()
    shape = (2, 10, 256, 128, True, 5)
    k1 = A.get_kernel("fwd", *shape)
    assert A.get_kernel("fwd", *shape) is k1
    kb = A.get_kernel("bwd", *shape)
    kinds = {kind for kind, *_ in A._kernels}
    assert kinds == {"fwd", "bwd"}          # what preflight.py:191-194 checks
    assert ("fwd", shape, A.AUTOTUNE) in A._kernels
    assert kb.kv_heads == 2 and abs(kb.sm_scale - 128 ** -0.5) < 1e-15
    with pytest.raises(ValueError):
        A.get_kernel("swizzle", *shape)
    with pytest.raises(ValueError):
        A.get_kernel("fwd", 2, 10, 256, 128, True, 3)


def test_kernels_reject_cpu_tensors_before_any_device_call():
    k = A.get_kernel("fwd", 1, 10, 64, 128, True, 5)
    q = torch.zeros(1, 64, 10, 128, dtype=torch.bfloat16)
    kv = torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA"):
        k(q, kv, kv)
    with pytest.raises(ValueError, match="CUDA"):
        mm.flash_attention(q, kv, kv, True, 5)
    with pytest.raises(ValueError, match="groups"):
        mm.flash_attention(q, kv, kv, True, 4)


def test_hip_backend_fails_loudly_without_device():
    cfg = A.AttnConfig()
    attn = A.Attention(cfg, A.Rotary(cfg.head_dim, 64, cfg.rope_theta))
    x = torch.randn(1, 16, cfg.d_model)
    for backend in ("hip", "tilelang"):
        with pytest.raises(ValueError, match="CUDA"):
            attn(x, backend=backend)
    with pytest.raises(ValueError, match="unknown backend"):
        attn(x, backend="triton")


def test_math_backend_matches_reference_function():
    torch.manual_seed(0)
    cfg = A.AttnConfig(backend="math")
    attn = A.Attention(cfg, A.Rotary(cfg.head_dim, 64, cfg.rope_theta))
    x = torch.randn(2, 24, cfg.d_model)
    q, k, v = attn.project(x)
    want = attn.wo(A.reference(q, k, v, True, cfg.groups).reshape(2, 24, -1))
    assert (attn(x) - want).abs().max() < 1e-5


def test_attention_flops():
    fwd, bwd = A.attention_flops(2, 8192)
    assert fwd == 2 * 2 * 10 * 8192 ** 2 * 128 and abs((fwd + bwd) - 1202.59e9) < 0.01e9


def test_tuned_store_roundtrip(tmp_path, monkeypatch):
    monkeypatch.setattr(tuned, "STORE", tmp_path / "tiles.json")
    assert tuned.lookup("attention_fwd", (1, 10, 64, 128, True, 5)) is None
    tuned.record("attention_fwd", (1, 10, 64, 128, True, 5), {"rows_per_wave": 32})
    assert tuned.lookup("attention_fwd", (1, 10, 64, 128, True, 5)) == {"rows_per_wave": 32}
    assert json.loads((tmp_path / "tiles.json").read_text())


def test_bench_refuses_multi_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_profsum_tables(tmp_path, capsys):
    """profsum reads rocprofv3 outputs: trace view and calibrated PMC means."""
    import sqlite3
    from mimansm1_v1_amd import profsum
    db = tmp_path / "t.db"
    con = sqlite3.connect(db)
    con.execute("create table top_kernels (name, total_calls, total_duration, average, percentage)")
    con.execute("insert into top_kernels values ('void mm1::attn_fwd_kernel<4, 2, true>(int)', 3, 30.0, 10.0, 100.0)")
    con.commit()
    con.close()
    hdr = "Kernel_Name,Counter_Name,Counter_Value\n"
    (tmp_path / "f.csv").write_text(hdr + '"void mm1::attn_fwd_kernel<4, 2, true>(int)",FETCH_SIZE,10\n'
                                    '"void mm1::attn_fwd_kernel<4, 2, true>(int)",FETCH_SIZE,30\n')
    (tmp_path / "w.csv").write_text(hdr + '"void mm1::attn_fwd_kernel<4, 2, true>(int)",WRITE_SIZE,4\n')
    (tmp_path / "cf.csv").write_text(hdr + '"copyBuffer",FETCH_SIZE,512\n"copyBuffer",FETCH_SIZE,2\n')
    (tmp_path / "cw.csv").write_text(hdr + '"copyBuffer",WRITE_SIZE,1024\n')
    out = tmp_path / "traffic.json"
    profsum.main(["--trace", str(db), "--fetch", str(tmp_path / "f.csv"), "--write", str(tmp_path / "w.csv"),
                  "--copy-fetch", str(tmp_path / "cf.csv"), "--copy-write", str(tmp_path / "cw.csv"),
                  "--copy-bytes", str(1 << 20), "--json", str(out)])
    text = capsys.readouterr().out
    assert "attn_fwd_kernel<4, 2, true>" in text and "| 3 | 10.0 |" in text
    # mean fetch 20 KiB x 2 (copy read 512 KiB for 1 MiB) + 4 KiB writes x 1
    assert json.loads(out.read_text())["fwd"] == (20 * 2 + 4) * 1024
