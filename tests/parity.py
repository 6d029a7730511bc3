"""Parity metrics and gates shared by the GPU tests.

Gates, all against the fp32 reference math on the
same bf16 inputs:
  * bf16 outputs O, dQ, dK, dV: relative L2 <= 5e-3 and
    max-abs <= 2e-2 + floor, where floor = max|bf16(ref) - ref| is the error
    that rounding the exact answer to bf16 already costs (dK/dV sum over up to
    G*S query rows, so at large magnitude one bf16 half-ulp exceeds 2e-2);
  * fp32 lse2: max-abs <= 1e-3;
    plus, where given, the error of the reference kernel's own arithmetic:
    alg = max|emulated - ref| (and alg_rel = relative L2 of emulated - ref) for
    the backward, whose P and dS are rounded to bf16 before their products
    exactly as the reference's TileLang kernel does (AT:306, :310-314).  With
    peaky softmax (config 4, logits std up to ~9) that rounding alone exceeds
    2e-2 max-abs on dQ/dK, and on tiny peaky cases 5e-3 relative L2; the gates
    then read max_abs <= 2e-2 + floor + alg and rel_l2 <= 5e-3 + alg_rel;
  * the reference harness's own metric max|d| / max|ref| < 2e-2 (AT:664-669),
    applied where max|ref| >= 1e-3 (it is undefined for an exactly-zero
    reference such as dQ at S = 1, where the max-abs gate still holds).
"""
from __future__ import annotations

import torch

REL_L2 = 5e-3
MAX_ABS = 2e-2
LSE_ABS = 1e-3
REF_REL = 2e-2


def metrics(got: torch.Tensor, want: torch.Tensor) -> dict:
    g = got.detach().float().cpu()
    w = want.detach().float().cpu()
    diff = (g - w)
    max_abs = diff.abs().max().item() if diff.numel() else 0.0
    wn = w.norm().item()
    rel_l2 = diff.norm().item() / wn if wn > 0 else diff.norm().item()
    floor = (w.to(torch.bfloat16).float() - w).abs().max().item() if w.numel() else 0.0
    ref_max = w.abs().max().item() if w.numel() else 0.0
    ref_rel = max_abs / max(ref_max, 1e-12)
    finite = bool(torch.isfinite(g).all())
    return dict(max_abs=max_abs, rel_l2=rel_l2, floor=floor, ref_rel=ref_rel, ref_max=ref_max,
                finite=finite)


def assert_bf16_close(name: str, got, want, log=print, emulated=None):
    m = metrics(got, want)
    alg = alg_rel = 0.0
    if emulated is not None:
        e = metrics(emulated, want)
        alg, alg_rel = e["max_abs"], e["rel_l2"]
    m["alg_floor"], m["alg_rel"] = alg, alg_rel
    log(f"    {name:4s} max_abs {m['max_abs']:.3e} (floor {m['floor']:.3e}, alg {alg:.3e})  "
        f"rel_l2 {m['rel_l2']:.3e} (alg {alg_rel:.3e})  ref_rel {m['ref_rel']:.3e}")
    assert m["finite"], f"{name}: non-finite values"
    assert m["rel_l2"] <= REL_L2 + alg_rel, (
        f"{name}: rel L2 {m['rel_l2']:.3e} > {REL_L2} + alg {alg_rel:.3e}")
    assert m["max_abs"] <= MAX_ABS + m["floor"] + alg, (
        f"{name}: max abs {m['max_abs']:.3e} > {MAX_ABS} + floor {m['floor']:.3e} + alg {alg:.3e}")
    if m["ref_max"] >= 1e-3:
        assert m["ref_rel"] < REF_REL, f"{name}: max|d|/max|ref| {m['ref_rel']:.3e} >= {REF_REL}"
    return m


def assert_lse_close(got, want, log=print):
    m = metrics(got, want)
    log(f"    lse2 max_abs {m['max_abs']:.3e}")
    assert m["finite"], "lse2: non-finite values"
    assert m["max_abs"] <= LSE_ABS, f"lse2: max abs {m['max_abs']:.3e} > {LSE_ABS}"
    return m
