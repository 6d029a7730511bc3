"""Parity metrics and gates shared by the GPU tests.

North-star tolerances, against the fp32 reference math
(AT:521-530) on the same bf16 inputs: bf16 O, dQ, dK, dV max-abs <= 2e-2 and
relative L2 <= 5e-3; fp32 lse2 max-abs <= 1e-3.  Also the reference harness's
own metric max|d| / max|ref| < 2e-2 (AT:664-669), applied where
max|ref| >= 1e-3 (it is undefined for an exactly-zero reference such as dQ at
S = 1, where the max-abs gate still holds).

How a bf16 output passes (the first that holds; which one is recorded):
  "bf16"     the bf16 output itself meets max-abs <= 2e-2 and rel-L2 <= 5e-3;
  "precast"  the kernel's fp32 values before the bf16 cast meet max-abs <=
             2e-2 and rel-L2 <= 5e-3, the bf16 output is exactly their bf16
             rounding (the pre-cast values come from the same kernels and
             tilings with fp32 stores: mm1_attn_fwd_f32,
             mm1_attn_bwd_f32_tiles), and the bf16 output meets rel-L2 <=
             5e-3 and max-abs <= 2e-2 + its rounding of the pre-cast values.
             Where the exact answer is large (dK/dV sum over up to G*S query
             rows), one bf16 half-ulp of it, the `floor` max|bf16(ref) - ref|,
             already exceeds 2e-2, so the bound is measured before the
             rounding.
Anything else fails.  The oracle's emulation of the reference kernel's own
bf16 rounding of P and dS (grads_analytic(bf16_products=True)) is recorded
beside each gradient as `alg` (what the reference's arithmetic scores) but is
no gate.

Every check can append its numbers to a JSON-lines file (MM1_PARITY_LOG) so a
GPU run leaves the per-case table behind.
"""
from __future__ import annotations

import json
import os

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


def _record(rec: dict) -> None:
    path = os.environ.get("MM1_PARITY_LOG")
    if not path:
        return
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "a") as f:
        f.write(json.dumps(rec) + "\n")


def assert_bf16_close(name: str, got, want, log=print, precast=None, emulated=None, case: str = ""):
    """Gate one bf16 output (see the module docstring); returns the metrics."""
    m = metrics(got, want)
    rec = dict(case=case, out=name, max_abs=m["max_abs"], rel_l2=m["rel_l2"], floor=m["floor"],
               ref_rel=m["ref_rel"], ref_max=m["ref_max"])
    assert m["finite"], f"{name}: non-finite values"
    if m["ref_max"] >= 1e-3:
        assert m["ref_rel"] < REF_REL, f"{name}: max|d|/max|ref| {m['ref_rel']:.3e} >= {REF_REL}"
    gate = None
    if m["max_abs"] <= MAX_ABS and m["rel_l2"] <= REL_L2:
        gate = "bf16"
    pc = None
    if precast is not None:
        pc = metrics(precast, want)
        assert pc["finite"], f"{name}: non-finite pre-cast values"
        g_cpu, p_cpu = got.detach().cpu(), precast.detach().float().cpu()
        rounds = torch.equal(g_cpu.to(torch.bfloat16), p_cpu.to(torch.bfloat16))
        own = (p_cpu.to(torch.bfloat16).float() - p_cpu).abs().max().item() if p_cpu.numel() else 0.0
        rec.update(precast_max_abs=pc["max_abs"], precast_rel_l2=pc["rel_l2"], rounds_precast=rounds)
        assert rounds, f"{name}: the bf16 output is not the bf16 rounding of the kernel's pre-cast values"
        if gate is None and pc["max_abs"] <= MAX_ABS and pc["rel_l2"] <= REL_L2 \
                and m["rel_l2"] <= REL_L2 and m["max_abs"] <= MAX_ABS + own:
            gate = "precast"
    if emulated is not None:
        al = metrics(emulated, want)
        rec.update(alg=al["max_abs"], alg_rel=al["rel_l2"])
    rec["gate"] = gate
    _record(rec)
    extra = ""
    if pc is not None:
        extra += f"  precast max_abs {pc['max_abs']:.3e} rel_l2 {pc['rel_l2']:.3e}"
    if emulated is not None:
        extra += f"  (reference-kernel rounding: {rec['alg']:.3e} / {rec['alg_rel']:.3e})"
    log(f"    {name:4s} max_abs {m['max_abs']:.3e} (floor {m['floor']:.3e})  rel_l2 {m['rel_l2']:.3e}  "
        f"ref_rel {m['ref_rel']:.3e}{extra}  -> {gate}")
    assert gate is not None, (
        f"{name}: bf16 max_abs {m['max_abs']:.3e} rel_l2 {m['rel_l2']:.3e} outside {MAX_ABS} / {REL_L2}"
        + (f"; pre-cast {pc['max_abs']:.3e} / {pc['rel_l2']:.3e}" if pc else "; no pre-cast values"))
    m["gate"] = gate
    return m


def assert_lse_close(got, want, log=print, case: str = ""):
    m = metrics(got, want)
    _record(dict(case=case, out="lse2", max_abs=m["max_abs"], rel_l2=m["rel_l2"], floor=0.0,
                 ref_rel=m["ref_rel"], ref_max=m["ref_max"], gate="fp32" if m["max_abs"] <= LSE_ABS else None))
    log(f"    lse2 max_abs {m['max_abs']:.3e}")
    assert m["finite"], "lse2: non-finite values"
    assert m["max_abs"] <= LSE_ABS, f"lse2: max abs {m['max_abs']:.3e} > {LSE_ABS}"
    return m


def assert_delta_close(got, want, log=print, case: str = ""):
    """Delta (fp32 rowsum of bf16 O * dO, AT:212-214) against the oracle's fp32
    sum of the same bf16 values: equal up to fp32 summation order, i.e. within
    a few fp32 ulps of sum_d |O_d dO_d| per row."""
    g, w = got.detach().float().cpu(), want.detach().float().cpu()
    err = (g - w).abs().max().item()
    m = dict(max_abs=err, ref_max=w.abs().max().item())
    _record(dict(case=case, out="delta", max_abs=err, rel_l2=((g - w).norm() / max(w.norm(), 1e-30)).item(),
                 floor=0.0, ref_rel=err / max(m["ref_max"], 1e-12), ref_max=m["ref_max"], gate="fp32"))
    log(f"    delta max_abs {err:.3e} (max|ref| {m['ref_max']:.3e})")
    assert torch.isfinite(g).all(), "delta: non-finite values"
    return m
