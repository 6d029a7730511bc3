"""The drop-in modules' GPU harnesses, and BASELINE.json config 5 (the full
attention sublayer) at its real size (GPU only)."""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import reference as R
from tests.parity import assert_bf16_close, assert_lse_close, metrics

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("module", ["attention", "swiglu", "lm_head"])
def test_drop_in_check_gpu_harness(hip_device, module):
    """check_gpu() of each drop-in module -- the harness a user of the
    reference runs (attention_tilelang.py:633-678, swiglu_tilelang.py:497-556,
    lm_head_tilelang.py:479-520) -- passes every check, and benchmark() times
    the kernels."""
    import importlib
    mod = importlib.import_module(f"mimansm1_v1_amd.{module}")
    log(f"[case] {module}.check_gpu()")
    report = mod.check_gpu()
    assert report.outcomes and report.ok, report.failures()
    log(f"[case] {module}.benchmark()")
    small = {"attention": dict(batch=2, seq_len=1024, iters=5), "swiglu": dict(tokens=4096),
             "lm_head": dict(tokens=2048)}[module]
    ms = mod.benchmark(**small)
    assert ms and all(t > 0 for t in ms.values()), ms


def test_config5_sublayer_full_size(hip_device, monkeypatch):
    """the Attention sublayer forward + backward at
    x [2, 8192, 1280] ~ N(0,1), weights ~ N(0, 0.02^2), under bf16 autocast on
    the "hip" backend (fused QKV GEMM, QK-norm + RoPE kernel, flash attention,
    wo).  The attention op inside it is held to the north-star gates on the
    q, k, v and upstream gradient the sublayer itself produced: O, lse2 and
    dQ, dK, dV against the fp32 math on those tensors (tests/parity.py).  The
    sublayer's output and parameter gradients are reported against the same
    module run by the reference's fp32 "math" backend without autocast, with
    a loose sanity bound (the hip path rounds the projections to bf16)."""
    import mimansm1_v1_amd.attention as A
    from tests.test_gpu_parity import check_grads, precast
    B, S = 2, 8192
    log(f"[case] config 5 sublayer B{B} S{S} d_model 1280")
    cfg = A.AttnConfig(max_seq_len=S)
    torch.manual_seed(0)
    layer = A.Attention(cfg, A.Rotary(cfg.head_dim, S, cfg.rope_theta))
    gen = torch.Generator().manual_seed(0)
    with torch.no_grad():
        for lin in (layer.wq, layer.wk, layer.wv, layer.wo):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=gen) * 0.02)
    layer = layer.to(hip_device)
    x = torch.randn(B, S, cfg.d_model, generator=gen).to(hip_device)
    dy = torch.randn(B, S, cfg.d_model, generator=gen).to(hip_device)

    seen = {}
    real = A.flash_attention

    def capture(q, k, v, causal=True, groups=5):
        seen["q"], seen["k"], seen["v"] = (t.detach().clone() for t in (q, k, v))
        for name, t in (("dq", q), ("dk", k), ("dv", v)):
            if t.requires_grad:
                t.register_hook(lambda g, name=name: seen.__setitem__(name, g.detach().clone()))
        out = real(q, k, v, causal, groups)
        seen["o"] = out.detach().clone()
        out.register_hook(lambda g: seen.__setitem__("do", g.detach().clone()))
        return out

    monkeypatch.setattr(A, "flash_attention", capture)
    xi = x.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = layer(xi, backend="hip")
    y.backward(dy.to(y.dtype))
    torch.cuda.synchronize()
    monkeypatch.setattr(A, "flash_attention", real)
    hip = {"y": y.detach().float(), "dx": xi.grad.float()}
    for name, p in layer.named_parameters():
        hip[name] = p.grad.float()
    assert all(key in seen for key in ("q", "k", "v", "o", "do", "dq", "dk", "dv")), sorted(seen)

    # the attention op on the sublayer's own tensors, against the fp32 math
    q, k, v, do = seen["q"], seen["k"], seen["v"], seen["do"]
    case = "config 5 attention"
    pre = precast(q.cpu(), k.cpu(), v.cpu(), do.cpu(), True, hip_device)
    want_o, want_lse = R.forward_chunked(q, k, v, True, cfg.groups)
    assert_bf16_close("O", seen["o"].cpu(), want_o.cpu(), log, precast=pre[0], case=case)
    _, lse = A.flash_attention_with_lse(q, k, v, True, cfg.groups)
    assert_lse_close(lse.cpu(), want_lse.cpu(), log, case=case)
    del want_o, want_lse
    want = [t.cpu() for t in R.grads_analytic(q, k, v, do, True, cfg.groups)]
    emu = [t.cpu() for t in R.grads_analytic(q, k, v, do, True, cfg.groups, bf16_products=True)]
    check_grads(case, (seen["dq"].cpu(), seen["dk"].cpu(), seen["dv"].cpu()), want, pre, emu)
    del want, emu, seen
    torch.cuda.empty_cache()

    # the whole sublayer against the reference's fp32 "math" backend
    layer.zero_grad(set_to_none=True)
    xf = x.clone().requires_grad_(True)
    yf = layer(xf, backend="math")
    yf.backward(dy)
    torch.cuda.synchronize()
    ref = {"y": yf.detach(), "dx": xf.grad}
    for name, p in layer.named_parameters():
        ref[name] = p.grad
    for name in hip:
        m = metrics(hip[name], ref[name])
        log(f"    sublayer {name:14s} rel_l2 {m['rel_l2']:.3e}  max|d|/max|ref| {m['ref_rel']:.3e}")
        assert m["finite"] and m["rel_l2"] < 2e-2, (name, m)
