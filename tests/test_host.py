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
    """The drop-in modules' CPU harnesses (the reference's check()) hold."""
    from mimansm1_v1_amd import lm_head, swiglu
    for module in (A, swiglu, lm_head):
        report = module.check_math(quiet=True)
        assert report.ok and len(report.outcomes) >= 8, (module.__name__, report.failures())


def test_harness_cli(capsys):
    """`python -m mimansm1_v1_amd.attention [check|tune|...]`, also with the
    reference's --flags; an unknown action is an error."""
    from mimansm1_v1_amd import harness
    calls = []
    actions = {"check": lambda: calls.append("check"), "tune": lambda: calls.append("tune")}
    assert harness.main("m", actions, []) == 0 and calls == ["check"]
    calls.clear()
    assert harness.main("m", actions, ["tune", "--check"]) == 0 and calls == ["check", "tune"]
    failing = harness.Report("x", quiet=True)
    failing.expect("never", False)
    assert harness.main("m", {"check": lambda: failing}, []) == 1
    with pytest.raises(SystemExit):
        harness.main("m", actions, ["bogus"])


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


def test_tuned_store_roundtrip_and_precedence(tmp_path, monkeypatch):
    """Nested device -> "kernel:shape" -> config records (tuned.py:45-74); the
    machine's own store wins over the shipped table; other devices miss."""
    monkeypatch.setattr(tuned, "STORE", tmp_path / "store.json")
    monkeypatch.setattr(tuned, "TABLE", tmp_path / "table.json")
    shape = (1, 10, 64, 128, True, 5)
    assert tuned.lookup("attention_fwd", shape, device="gfx950-256cu") is None
    tuned.record("attention_fwd", shape, dict(A.FWD_TILES), device="gfx950-256cu",
                 store=tmp_path / "table.json")
    assert tuned.lookup("attention_fwd", shape, device="gfx950-256cu") == A.FWD_TILES
    other = dict(A.FWD_TILES, waves=8)
    tuned.record("attention_fwd", shape, other, device="gfx950-256cu")
    assert tuned.lookup("attention_fwd", shape, device="gfx950-256cu") == other
    assert tuned.lookup("attention_fwd", shape, device="gfx942-304cu") is None
    tuned.record("attention_fwd", (2,), {}, device="gfx950-256cu")      # empty: ignored
    data = json.loads((tmp_path / "store.json").read_text())
    assert list(data) == ["gfx950-256cu"]
    assert list(data["gfx950-256cu"]) == ["attention_fwd:1,10,64,128,True,5"]
    text = tuned.summary()
    line = [ln for ln in text.splitlines() if "attention_fwd" in ln and "store.json" in ln]
    assert len(line) == 1 and "gfx950-256cu" in line[0] and "(1,10,64,128,True,5)" in line[0]
    assert "waves=8" in line[0]
    assert "(no records)" in tuned.summary([tmp_path / "missing.json"])
    assert tuned.config_of(A.FwdKernel(shape, A.FWD_TILES)) == A.FWD_TILES
    assert tuned.device_key() == "no-hip"


def test_tile_space_matches_library_and_defaults():
    """The configs are the library's own descriptions; index 0 is the default
    and every config maps back to its index."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    fwd, bwd = A.fwd_configs(), A.bwd_configs()
    assert A.FWD_TILES == fwd[0] and A.BWD_TILES == bwd[0]
    assert len(fwd) == lib.mm1_attn_tile_count(0) >= 2
    assert len(bwd) == lib.mm1_attn_tile_count(1) * lib.mm1_attn_tile_count(2)
    assert [A.tile_index("fwd", c) for c in fwd] == list(range(len(fwd)))
    pairs = [A.tile_index("bwd", c) for c in bwd]
    assert sorted(pairs) == [(i, j) for i in range(lib.mm1_attn_tile_count(1))
                             for j in range(lib.mm1_attn_tile_count(2))]
    assert all(c["block_N"] == 64 and c["waves"] in (4, 8) for c in fwd)
    # a config naming no compiled tiling: rejected by the handle, index None
    assert A.tile_index("fwd", dict(A.FWD_TILES, block_M=96)) is None
    assert A.tile_index("bwd", dict(A.BWD_TILES, extra=1)) is None
    assert A.tile_index("bwd", {k: v for k, v in A.BWD_TILES.items() if k != "dq_waves"}) is None
    with pytest.raises(ValueError, match="not a tiling"):
        A.FwdKernel((1, 10, 64, 128, True, 5), dict(A.FWD_TILES, stages=9))
    assert A.get_kernel("bwd", 1, 10, 64, 128, True, 5).tiles == (0, 0)


def test_get_kernel_uses_record_and_ignores_stale_one(tmp_path, monkeypatch):
    monkeypatch.setattr(tuned, "STORE", tmp_path / "store.json")
    monkeypatch.setattr(tuned, "TABLE", tmp_path / "none.json")
    monkeypatch.setattr(tuned, "device_key", lambda: "gfx950-256cu")
    monkeypatch.setattr(A, "_kernels", {})
    shape = (3, 10, 96, 128, True, 5)
    tuned.record("attention_fwd", shape, A.fwd_configs()[2])
    tuned.record("attention_bwd", shape, dict(A.BWD_TILES, dq_stages=11))   # not compiled
    assert A.get_kernel("fwd", *shape).tiles == 2
    assert A.get_kernel("bwd", *shape).config == A.BWD_TILES     # no GPU: defaults


def test_shipped_tile_table_names_compiled_tilings():
    """The measured gfx950 table covers both run shapes, fwd and bwd, and every
    entry is a tiling this build has."""
    from mimansm1_v1_amd import tune as T
    data = json.loads(tuned.TABLE.read_text())
    assert data, "empty shipped table"
    cfg = A.AttnConfig()
    for device, entries in data.items():
        assert device.startswith("gfx950-"), device
        for _, micro, seq in T.stage_shapes():
            for name, kind, shape in T.jobs(micro, seq, cfg):
                key = f"{name}:{','.join(str(x) for x in shape)}"
                assert key in entries, (device, key)
                assert A.tile_index(kind, entries[key]) is not None, (key, entries[key])


def test_backward_record_overlap_entry():
    """A backward tile record may carry "overlap_dq" (how its two launches
    share the device) beside its tilings; anything but a bool there, or an
    unknown key, names no tiling."""
    base = dict(A.BWD_TILES)
    assert A.tile_index("bwd", dict(base, overlap_dq=True)) == A.tile_index("bwd", base) == (0, 0)
    assert A.tile_index("bwd", dict(base, overlap_dq=False)) == (0, 0)
    assert A.tile_index("bwd", dict(base, overlap_dq="yes")) is None
    assert A.tile_index("bwd", dict(base, overlap=True)) is None
    assert A.tile_index("fwd", dict(A.FWD_TILES, overlap_dq=True)) is None


def test_tune_cli_shapes_and_control_flow():
    """stage_shapes follows the stage switch (tune.py:30-46): 8 x 2048 then
    2 x 8192; tune_all skips known entries unless forced, records each
    winner, and carries on past a failing job."""
    from mimansm1_v1_amd import tune as T
    assert T.stage_shapes() == [("foundation", 8, 2048), ("long_ctx", 2, 8192)]
    assert T.stage_shapes(4, 4096) == [("foundation", 8, 2048), ("long_ctx", 2, 8192)]
    cfg = A.AttnConfig()
    known, recorded, lines = {}, [], []

    def search(kind, shape):
        if kind == "bwd" and shape[2] == 8192:
            raise RuntimeError("boom")
        return (A.FWD_TILES if kind == "fwd" else A.BWD_TILES), 1.5

    def record(name, shape, config):
        recorded.append((name, shape))
        known[(name, shape)] = config

    hooks = dict(lookup=lambda n, s: known.get((n, s)), search=search, record=record,
                 out=lines.append)
    done = T.tune_all(8, 2048, cfg, **hooks)
    assert set(done) == {"attention_fwd", "attention_bwd"} and all(done.values())
    assert recorded == [("attention_fwd", (8, 10, 2048, 128, True, 5)),
                        ("attention_bwd", (8, 10, 2048, 128, True, 5))]
    assert T.tune_all(8, 2048, cfg, **hooks) == {"attention_fwd": None, "attention_bwd": None}
    assert sum("already known" in x for x in lines) == 2
    T.tune_all(8, 2048, cfg, force=True, **hooks)
    assert len(recorded) == 4
    done = T.tune_all(2, 8192, cfg, **hooks)
    assert done["attention_fwd"] and done["attention_bwd"] is None
    assert any("FAILED" in x and "boom" in x for x in lines)


def test_tune_cli_refuses_without_gpu():
    r = subprocess.run([sys.executable, "-m", "mimansm1_v1_amd.tune"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "needs the gpu" in r.stderr


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
    con.execute("create table kernels (name, start, end)")
    for start, end in ((0, 8_000), (10_000, 20_000), (30_000, 42_000)):
        con.execute("insert into kernels values ('void mm1::attn_fwd_kernel<4, 2, true>(int)', ?, ?)",
                    (start, end))
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
    assert "attn_fwd_kernel<4, 2, true>" in text and "| 3 | 10.0 | 10.0 | 100.0% | 3 | 10.0 | 10.0 |" in text
    # mean fetch 20 KiB x 2 (copy read 512 KiB for 1 MiB) + 4 KiB writes x 1
    assert json.loads(out.read_text())["fwd"] == (20 * 2 + 4) * 1024


@pytest.mark.parametrize("t,chunks", [(512, 2), (4096, 8), (1000, 8), (100, 2), (256, 1)])
def test_wgrad_chunking_equals_one_product(monkeypatch, t, chunks):
    """wgrad's token chunking (reshape per chunk, transpose of the left
    operand, fp32 sum) equals the one product a^T b; uneven or short token
    counts take the single product.  Run in fp32 on the CPU, where the
    fp32-output GEMM forms are stood in by plain fp32 products."""
    import torch
    from mimansm1_v1_amd import wgrad as W
    calls = []
    bmm, mm = torch.bmm, torch.mm

    def bmm32(x, y, out_dtype=None):
        calls.append("bmm")
        return bmm(x.double(), y.double()).float()

    def mm32(x, y, out_dtype=None):
        calls.append("mm")
        return mm(x.double(), y.double()).float()

    monkeypatch.setattr(W.torch, "bmm", bmm32)
    monkeypatch.setattr(W.torch, "mm", mm32)
    gen = torch.Generator().manual_seed(t)
    a, b = torch.randn(t, 7, generator=gen), torch.randn(t, 5, generator=gen)
    got = W.wgrad(a, b, chunks)
    want = (a.double().t() @ b.double()).float()
    assert got.shape == (7, 5)
    assert torch.allclose(got, want, atol=1e-4, rtol=1e-5)
    chunked = chunks > 1 and t % chunks == 0 and t >= 64 * chunks
    assert calls == (["bmm"] if chunked else ["mm"])


def test_profsum_separates_dispatches_that_ran_alone():
    """profsum's per-dispatch split: a dispatch counts as alone only when no
    other dispatch of the trace overlapped it (touching ends do not)."""
    from mimansm1_v1_amd.profsum import dispatch_stats
    spans = [("a", 0, 10_000), ("b", 5_000, 15_000),          # overlap each other
             ("c", 20_000, 30_000), ("c", 30_000, 40_000),    # touch only
             ("d", 41_000, 100_000), ("e", 42_000, 45_000),   # e inside d
             ("c", 60_000, 70_000),                           # inside d too
             ("a", 200_000, 210_000)]
    st = dispatch_stats(spans)
    assert st["a"] == ([10.0, 10.0], [10.0])
    assert st["b"] == ([10.0], [])
    assert st["c"] == ([10.0, 10.0, 10.0], [10.0, 10.0])
    assert st["d"] == ([59.0], []) and st["e"] == ([3.0], [])


def test_bench_select_tiles_follows_the_record(monkeypatch):
    """bench.py launches what the tile record names, including the dQ
    side-stream switch; an explicit --tiles override runs on one stream."""
    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench
    records = {"attention_fwd": dict(A.FWD_TILES),
               "attention_bwd": dict(A.BWD_TILES, dq_block_M=256, dq_waves=8, dq_stages=3,
                                     overlap_dq=True)}
    monkeypatch.setattr(tuned, "lookup", lambda name, shape: records.get(name))
    assert bench.select_tiles(2, 8192) == {"fwd": 0, "dkdv": 0, "dq": 1, "overlap": True}
    records["attention_bwd"].pop("overlap_dq")
    monkeypatch.setattr(A, "OVERLAP_DQ", True)
    assert bench.select_tiles(2, 8192)["overlap"] is True       # the module default
    monkeypatch.setattr(A, "OVERLAP_DQ", False)
    assert bench.select_tiles(2, 8192)["overlap"] is False
    assert bench.select_tiles(2, 8192, "1,5,0") == {"fwd": 1, "dkdv": 5, "dq": 0, "overlap": False}
