"""HIP kernels vs the oracle on identical seeded bf16 inputs (GPU only).

Small shapes are checked against the CPU oracle (fp32 autograd through the
restated reference attention).  The BASELINE.json configs 2-4 are checked at
full size against the oracle's chunked closed-form fp32 math run on the GPU
(itself pinned to the CPU oracle in test_gpu_oracle_device_agrees).  Every
check also takes the kernels' pre-cast fp32 outputs (mm1_attn_fwd_f32,
mm1_attn_bwd_f32_tiles: the same kernels and tilings as the bf16 outputs, so
the bf16 outputs must equal their rounding bitwise) and, for the gradients,
the oracle's emulation of the reference kernel's bf16 rounding points
(grads_analytic(bf16_products=True)) as a reported column: tests/parity.py
says how an output passes."""
from __future__ import annotations

import ctypes
import math
import sys

import pytest
import torch
import torch.nn.functional as F

from oracle import reference as R
from tests.parity import assert_bf16_close, assert_delta_close, assert_lse_close

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def hip_run(q, k, v, do, causal, groups, device, backward=True):
    """Runs the drop-in op on the GPU; returns CPU tensors (o, lse2, dq, dk, dv)."""
    import mimansm1_v1_amd as mm
    qd, kd, vd = (t.to(device).requires_grad_(backward) for t in (q, k, v))
    out, lse = mm.flash_attention_with_lse(qd.detach(), kd.detach(), vd.detach(), causal, groups)
    grads = (None, None, None)
    if backward:
        o2 = mm.flash_attention(qd, kd, vd, causal, groups)
        o2.backward(do.to(device))
        grads = (qd.grad, kd.grad, vd.grad)
        assert torch.equal(o2.detach(), out), "autograd forward differs from the kernel handle"
    torch.cuda.synchronize()
    cpu = lambda t: None if t is None else t.detach().cpu()
    return cpu(out), cpu(lse), *(cpu(g) for g in grads)


def _tiles_of(B, S, H, D, causal, G):
    """(forward tiling, (dK/dV tiling, dQ tiling)) of the kernel handles the
    drop-in op runs for this shape (the tile record or the autotuner's pick)."""
    import mimansm1_v1_amd as mm
    return (mm.get_kernel("fwd", B, H, S, D, causal, G).tiles,
            mm.get_kernel("bwd", B, H, S, D, causal, G).tiles)


def precast(q, k, v, do, causal, device, tiles=None):
    """The kernels' fp32 values before their bf16 casts, from the tilings the
    drop-in op runs for this shape (or `tiles` = (fwd, (dkdv, dq))): O
    (mm1_attn_fwd_f32) and dQ, dK, dV (mm1_attn_bwd_f32_tiles on the state of
    that forward and its O rounded to bf16, which is the bf16 forward's O);
    CPU fp32 tensors (o, dq, dk, dv), the gradients None when do is None."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    qd, kd, vd = (t.to(device).contiguous() for t in (q, k, v))
    B, S, H, D = qd.shape
    Hkv = kd.shape[2]
    ft, (dkt, dqt) = tiles if tiles is not None else _tiles_of(B, S, H, D, causal, H // Hkv)
    sp = torch.cuda.current_stream(device).cuda_stream
    p = lambda t: t.data_ptr()
    o32 = torch.empty(qd.shape, dtype=torch.float32, device=device)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=device)
    st = torch.empty(lib.mm1_attn_fwd_state_size(B, S, H, Hkv, D), dtype=torch.uint8, device=device)
    args = (B, S, H, Hkv, D, int(causal), D ** -0.5)
    _lib.check(lib.mm1_attn_fwd_f32(p(qd), p(kd), p(vd), p(o32), p(lse), p(st), st.numel(), *args, ft, sp),
               "fwd_f32")
    if do is None:
        torch.cuda.synchronize()
        return o32.cpu(), None, None, None
    dod = do.to(device).contiguous()
    ob = o32.to(torch.bfloat16)
    ws = torch.empty(lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, D), dtype=torch.uint8, device=device)
    dq = torch.empty(qd.shape, dtype=torch.float32, device=device)
    dk = torch.empty(kd.shape, dtype=torch.float32, device=device)
    dv = torch.empty(vd.shape, dtype=torch.float32, device=device)
    _lib.check(lib.mm1_attn_bwd_f32_tiles(p(ob), p(dod), p(lse), p(st), st.numel(), p(dq), p(dk), p(dv),
                                          p(ws), ws.numel(), *args, dkt, dqt, sp), "bwd_f32")
    torch.cuda.synchronize()
    out = (o32.cpu(), dq.cpu(), dk.cpu(), dv.cpu())
    del ws, dq, dk, dv, o32, st
    return out


def check_grads(case, got, want, pre, emu):
    """dQ, dK, dV; `pre` is precast()'s (o, dq, dk, dv)."""
    for name, g, w, pc, e in zip(("dQ", "dK", "dV"), got, want, pre[1:], emu):
        assert_bf16_close(name, g, w, log, precast=pc, emulated=e, case=case)


SMALL = [
    # (B, S, H, Hkv)
    (1, 1, 10, 2),
    (1, 17, 10, 2),
    (2, 64, 10, 2),
    (1, 100, 10, 2),
    (1, 255, 4, 4),
    (2, 130, 6, 3),
    (1, 320, 8, 1),
    (2, 512, 10, 2),
]


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("shape", SMALL, ids=[f"B{b}S{s}H{h}K{kv}" for b, s, h, kv in SMALL])
def test_small_shapes_vs_cpu_oracle(hip_device, shape, causal):
    B, S, H, Hkv = shape
    G = H // Hkv
    case = f"small B{B} S{S} H{H} Hkv{Hkv} {'causal' if causal else 'full'}"
    log(f"[case] {case}")
    q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=S + 7 * H)
    o, lse, dq, dk, dv = hip_run(q, k, v, do, causal, G, hip_device)
    pre = precast(q, k, v, do, causal, hip_device)
    assert_bf16_close("O", o, R.attention(q, k, v, causal, G, cast=False), log, precast=pre[0], case=case)
    assert_lse_close(lse, R.lse2(q, k, causal, G), log, case=case)
    check_grads(case, (dq, dk, dv), R.grads(q, k, v, do, causal, G), pre,
                R.grads_analytic(q, k, v, do, causal, G, bf16_products=True))


def _tilings():
    from mimansm1_v1_amd import attention as A
    return ([("fwd", i) for i in range(1, len(A.fwd_configs()))]
            + [("bwd", i) for i in range(1, len(A.bwd_configs()))])


TILINGS = _tilings()


@pytest.mark.parametrize("kind,index", TILINGS, ids=[f"{k}{i}" for k, i in TILINGS])
def test_tilings_vs_cpu_oracle(hip_device, monkeypatch, kind, index):
    """Every compiled tiling other than the defaults, launched through a kernel
    handle that carries it (as a tuned record would), meets the same gates as
    the defaults: causal and full, ragged S, GQA and MHA."""
    from mimansm1_v1_amd import attention as A
    config = (A.fwd_configs() if kind == "fwd" else A.bwd_configs())[index]
    monkeypatch.setattr(A, "_kernels", {})
    for (B, S, H, Hkv), causal in [((2, 300, 10, 2), True), ((1, 200, 6, 3), False), ((1, 77, 4, 4), True)]:
        G = H // Hkv
        case = f"tiling {kind}{index} B{B} S{S} H{H} Hkv{Hkv} {'causal' if causal else 'full'}"
        log(f"[case] {case} {config}")
        shape = (B, H, S, 128, causal, G)
        for k in ("fwd", "bwd"):
            tiles = config if k == kind else (A.FWD_TILES if k == "fwd" else A.BWD_TILES)
            A._kernels[(k, shape, A.AUTOTUNE)] = (A.FwdKernel if k == "fwd" else A.BwdKernel)(shape, tiles)
        q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=3 * S + H)
        o, lse, dq, dk, dv = hip_run(q, k, v, do, causal, G, hip_device)
        pre = precast(q, k, v, do, causal, hip_device)
        assert_bf16_close("O", o, R.attention(q, k, v, causal, G, cast=False), log, precast=pre[0], case=case)
        assert_lse_close(lse, R.lse2(q, k, causal, G), log, case=case)
        check_grads(case, (dq, dk, dv), R.grads(q, k, v, do, causal, G), pre,
                    R.grads_analytic(q, k, v, do, causal, G, bf16_products=True))


def _fwd_state(lib, q, k, v, causal, device, tiles=-1):
    """Forward through the C ABI: (o, lse2, state)."""
    B, S, H = q.shape[0], q.shape[1], q.shape[2]
    Hkv = k.shape[2]
    o, lse = torch.empty_like(q), torch.empty(B, H, S, dtype=torch.float32, device=device)
    st = torch.empty(lib.mm1_attn_fwd_state_size(B, S, H, Hkv, 128), dtype=torch.uint8, device=device)
    sp = torch.cuda.current_stream(device).cuda_stream
    assert lib.mm1_attn_fwd_tiles(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                                  st.data_ptr(), st.numel(), B, S, H, Hkv, 128, int(causal), 128 ** -0.5,
                                  tiles, sp) == 0
    return o, lse, st


def _workspace(lib, B, S, H, Hkv, device):
    return torch.empty(lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, 128), dtype=torch.uint8, device=device)


@pytest.mark.parametrize("dkdv_tiles", [0, 1])
def test_staged_tiling_calls_and_layout_check(hip_device, dkdv_tiles):
    """The staged calls with an explicit tiling (prep; dK/dV, then the
    separate sum, then dQ; and dK/dV, then dQ with the sum in its tail) give
    the combined mm1_attn_bwd_tiles result bitwise.  A summing call that
    names another dK/dV tiling, shape or `causal` than the dK/dV call that
    filled the workspace returns MM1_E_LAYOUT and launches nothing: dk/dv
    keep their contents."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    E_LAYOUT = -8
    B, S, H, Hkv, causal = 2, 1111, 10, 2, True
    log(f"[case] staged calls, dK/dV tiling {dkdv_tiles}, B={B} S={S}")
    q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=17))
    o, lse, st = _fwd_state(lib, q, k, v, causal, hip_device)
    ws = _workspace(lib, B, S, H, Hkv, hip_device)
    sp = torch.cuda.current_stream(hip_device).cuda_stream
    p = lambda t: t.data_ptr()
    args = (B, S, H, Hkv, 128, int(causal), 128 ** -0.5)
    S_ = (p(st), st.numel())
    W_ = (p(ws), ws.numel())
    ref = [torch.empty_like(t) for t in (q, k, v)]
    assert lib.mm1_attn_bwd_tiles(p(o), p(do), p(lse), *S_, *(p(t) for t in ref), *W_, *args, dkdv_tiles, 1,
                                  sp) == 0
    for tail in (False, True):
        dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
        assert lib.mm1_attn_bwd_prep(p(o), p(do), p(lse), *S_, *W_, *args[:5], args[6], sp) == 0
        assert lib.mm1_attn_bwd_dkdv_tiles(*S_, p(dk), p(dv), *W_, *args, dkdv_tiles, sp) == 0
        if tail:
            assert lib.mm1_attn_bwd_dq_reduce_tiles(*S_, p(dq), p(dk), p(dv), *W_, *args, dkdv_tiles, 1, sp) == 0
        else:
            assert lib.mm1_attn_bwd_dkdv_reduce_tiles(*W_, p(dk), p(dv), B, S, H, Hkv, 128, int(causal),
                                                      dkdv_tiles, sp) == 0
            assert lib.mm1_attn_bwd_dq_tiles(*S_, p(dq), *W_, *args, 1, sp) == 0
        torch.cuda.synchronize()
        for name, x, y in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
            assert torch.equal(x, y), (name, tail)
    # a summing call that disagrees with the layout in the workspace
    grouped = dkdv_tiles == 0
    other = 1 if grouped else 0
    sk, sv = torch.full_like(k, 7.0), torch.full_like(v, 7.0)
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(*W_, p(sk), p(sv), B, S, H, Hkv, 128, int(causal), other,
                                              sp) == E_LAYOUT
    sq = torch.full_like(q, 7.0)
    assert lib.mm1_attn_bwd_dq_reduce_tiles(*S_, p(sq), p(sk), p(sv), *W_, *args, other, 1, sp) == E_LAYOUT
    if grouped:   # the chunk plan of the grouped tiling depends on `causal` too
        assert lib.mm1_attn_bwd_dkdv_reduce_tiles(*W_, p(sk), p(sv), B, S, H, Hkv, 128, 0, dkdv_tiles,
                                                  sp) == E_LAYOUT
    # another shape (fewer positions, same workspace address)
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(*W_, p(sk), p(sv), B, S - 100, H, Hkv, 128, int(causal),
                                              dkdv_tiles, sp) == E_LAYOUT
    torch.cuda.synchronize()
    assert bool((sk == 7.0).all()) and bool((sv == 7.0).all()) and bool((sq == 7.0).all()), \
        "a refused call wrote its outputs"


@pytest.mark.parametrize("B,S,H,Hkv", [(2, 1111, 10, 2), (8, 2048, 10, 2), (1, 77, 4, 4)],
                         ids=["B2S1111", "config2", "B1S77mha"])
def test_backward_dq_overlap_matches_single_stream(hip_device, monkeypatch, B, S, H, Hkv):
    """The backward handle with dQ on a second stream beside dK/dV and the
    separate partial sum (a tile record's "overlap_dq", or the OVERLAP_DQ
    default) gives the single-stream mm1_attn_bwd_tiles result bitwise."""
    from mimansm1_v1_amd import attention as A
    log(f"[case] dQ overlap vs one stream B{B} S{S} H{H} Hkv{Hkv}")
    q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=S + 1))
    shape = (B, H, S, 128, True, H // Hkv)
    o, lse, state = A.FwdKernel(shape, A.FWD_TILES).run(q, k, v)
    delta = A.DeltaKernel(B, H, S, 128)(o, do)
    outs = []
    for config, default in ((dict(A.BWD_TILES, overlap_dq=False), True),
                            (dict(A.BWD_TILES, overlap_dq=True), False),
                            (dict(A.BWD_TILES), True)):
        monkeypatch.setattr(A, "OVERLAP_DQ", default)   # the record's entry wins
        for saved in (True, False):   # the autograd op's call, and the reference signature's
            grads = [torch.full_like(t, 3.0) for t in (q, k, v)]
            if saved:
                A.BwdKernel(shape, config).run_saved(o, do, lse, state, *grads)
            else:
                A.BwdKernel(shape, config)(q, k, v, do, lse, delta, *grads)
            torch.cuda.synchronize()
            outs.append(grads)
    outs = outs[0::2] + outs[1::2]
    for other in outs[1:3]:
        for name, x, y in zip(("dq", "dk", "dv"), outs[0], other):
            assert torch.equal(x, y), name
    outs = outs[3:]
    for other in outs[1:]:
        for name, x, y in zip(("dq", "dk", "dv"), outs[0], other):
            assert torch.equal(x, y), name


@pytest.mark.parametrize("B,S,H,Hkv", [(8, 2048, 10, 2), (2, 8192, 10, 2), (4, 4096, 10, 2), (3, 2999, 10, 2),
                                       (1, 77, 4, 4), (2, 1, 6, 3)],
                         ids=["config2", "config3", "config4", "B3S2999", "B1S77", "B2S1"])
def test_delta_kernel_vs_oracle(hip_device, B, S, H, Hkv):
    """mm1_attn_delta (flash_delta, AT:192-217) against the oracle's
    R.delta (rowsum(O * dO) in fp32, AT:212-214, itself pinned by the identity
    rowsum(O * dO) = sum_j P_ij dP_ij) on the same bf16 O and dO: equal up to
    the order of the 128-term fp32 sums."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    case = f"delta B{B} S{S} H{H} Hkv{Hkv}"
    log(f"[case] {case}")
    gen = torch.Generator().manual_seed(B * S + H)
    o = torch.randn(B, S, H, 128, generator=gen).to(torch.bfloat16)
    do = torch.randn(B, S, H, 128, generator=gen).to(torch.bfloat16)
    if S >= 4096:   # config-4-like magnitudes too
        o[:, :, 0] *= 8
    od, dod = o.to(hip_device), do.to(hip_device)
    delta = torch.empty(B, H, S, dtype=torch.float32, device=hip_device)
    _lib.check(lib.mm1_attn_delta(od.data_ptr(), dod.data_ptr(), delta.data_ptr(), B, S, H, 128,
                                  torch.cuda.current_stream(hip_device).cuda_stream), "delta")
    torch.cuda.synchronize()
    want = R.delta(o, do)
    m = assert_delta_close(delta, want, log, case=case)
    # fp32 sums of 128 products: a few ulps of the sum of |terms|
    bound = 4 * 2 ** -23 * 128 * (o.float() * do.float()).abs().sum(-1).max().item()
    assert m["max_abs"] <= bound, (m["max_abs"], bound)


def _ws_regions(lib, B, S, H, Hkv):
    """Byte offsets of the backward workspace's regions (the layout
    include/mm1_attn.h describes): fp16 dO, -2^E Delta, lse2 - log2(sm_scale),
    the scale."""
    up = lambda x: (x + 255) // 256 * 256
    do16 = 0
    delta = up(2 * B * S * H * 128)
    lse = delta + up(4 * B * H * S)
    dmax = lse + up(4 * B * H * S)
    scale = dmax + up(1024 * 4)
    return do16, delta, lse, scale


@pytest.mark.parametrize("B,S,H,Hkv,dscale", [(2, 1000, 10, 2, 1.0), (1, 333, 6, 3, 2.0 ** -20),
                                               (1, 77, 4, 4, 2.0 ** 12), (8, 2048, 10, 2, 1.0)],
                         ids=["B2S1000", "B1S333tiny", "B1S77huge", "config2"])
def test_bwd_prep_delta_and_scaled_do(hip_device, B, S, H, Hkv, dscale):
    """mm1_attn_bwd_prep leaves in the workspace: 2^E with E from max|dO| and
    max|V| by the rule of the library's do_scale_exp (E = 0 for dO of
    ordinary size, a power of two that brings tiny or huge dO back into
    fp16's range otherwise); do16 = fp16(2^E dO) exactly; -2^E Delta, with
    Delta = rowsum(O dO) from the forward's fp32 O (mm1_attn_fwd_f32, the
    values the bf16 O rounds): within 2^-14 of sum_d |O_d dO_d| (15
    significant bits of O), where the bf16 O alone is about 2^-9 away; and
    lse2 - log2(sm_scale), the fp32 difference."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    case = f"bwd prep B{B} S{S} H{H} Hkv{Hkv} dO x {dscale:g}"
    log(f"[case] {case}")
    q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=S + 3))
    do = (do.float() * dscale).to(torch.bfloat16)
    o, lse, st = _fwd_state(lib, q, k, v, True, hip_device)
    ws = _workspace(lib, B, S, H, Hkv, hip_device)
    sp = torch.cuda.current_stream(hip_device).cuda_stream
    o32 = torch.empty(q.shape, dtype=torch.float32, device=hip_device)
    st2 = torch.empty_like(st)
    l2 = torch.empty_like(lse)
    assert lib.mm1_attn_fwd_f32(q.data_ptr(), k.data_ptr(), v.data_ptr(), o32.data_ptr(), l2.data_ptr(),
                                st2.data_ptr(), st2.numel(), B, S, H, Hkv, 128, 1, 128 ** -0.5, -1, sp) == 0
    assert lib.mm1_attn_bwd_prep(o.data_ptr(), do.data_ptr(), lse.data_ptr(), st.data_ptr(), st.numel(),
                                 ws.data_ptr(), ws.numel(), B, S, H, Hkv, 128, 128 ** -0.5, sp) == 0
    torch.cuda.synchronize()
    r_do, r_delta, r_lse, r_scale = _ws_regions(lib, B, S, H, Hkv)
    do16 = ws[r_do:r_do + 2 * do.numel()].view(torch.float16).view(do.shape).cpu()
    delta = -ws[r_delta:r_delta + 4 * B * H * S].view(torch.float32).view(B, H, S).cpu()
    lse_ws = ws[r_lse:r_lse + 4 * B * H * S].view(torch.float32).view(B, H, S).cpu()
    l2sm = torch.tensor(128 ** -0.5, dtype=torch.float32).log2()
    assert torch.allclose(lse_ws, lse.cpu() - l2sm, rtol=0, atol=4e-6 * (1 + lse.abs().max().item()))
    scale = ws[r_scale:r_scale + 8].view(torch.float32).cpu()
    # the rule, on the host
    mdo, mv = do.float().abs().max().item(), v.float().abs().max().item()
    bound = 2 * 128 * 128 ** -0.5 * mdo * mv
    if 2 ** -8 <= mdo <= 2 ** 8 and bound < 2 ** 15:
        e = 0
    else:
        e = -(math.frexp(mdo)[1] - 1)
        e = min(e, 14 - (math.frexp(bound)[1] - 1))
    log(f"    max|dO| {mdo:.3e} max|V| {mv:.3e} -> E = {e}; scale cells {scale.tolist()}")
    assert scale[0].item() == 2.0 ** -e and scale[1].item() == 2.0 ** e
    assert torch.equal(do16, (do.float().cpu() * 2.0 ** e).to(torch.float16))
    o32c, doc = o32.cpu(), do.float().cpu()
    want = (o32c * doc).sum(-1).permute(0, 2, 1) * 2.0 ** e
    mag = (o32c * doc).abs().sum(-1).permute(0, 2, 1) * 2.0 ** e
    err = (delta - want).abs()
    log(f"    Delta max err {err.max().item():.3e}, relative to sum|O dO| "
        f"{(err / mag.clamp_min(1e-30)).max().item():.3e}")
    assert bool((err <= 2 ** -14 * mag + 1e-30).all())
    # the bf16 O alone: several times further off
    err_bf = ((o.float().cpu() * doc).sum(-1).permute(0, 2, 1) * 2.0 ** e - want).abs()
    assert err_bf.max().item() > 4 * err.max().item()


@pytest.mark.parametrize("s1,s2", [(2.0 ** -20, 2.0 ** -24), (2.0 ** 10, 2.0 ** 14), (1.0, 2.0 ** -20),
                                   (1.0, 2.0 ** -130)], ids=["tiny", "huge", "ordinary-tiny", "subnormal"])
def test_backward_is_linear_in_do(hip_device, s1, s2):
    """The gradients are linear in dO.  dO outside [2^-8, 2^8] is brought to
    max|2^E dO| in [1, 2) before its fp16 rounding, so two such dO that differ
    by a power of two have the same fp16 copy and every intermediate is the
    same: dQ, dK, dV differ by exactly that power of two, bitwise.  Against
    dO of ordinary size (E = 0) the fp16 roundings of the smallest dS values
    (fp16 subnormals) differ, and with them a few bf16 roundings of the
    outputs: equal up to rel-L2 1e-3.  For dO of 2^-130 (bf16 subnormals,
    compared with the same values scaled back to 1) the gradients are bf16
    subnormals too: within one bf16 step (2^-133) of the linear answer."""
    import mimansm1_v1_amd as mm
    B, S, H, Hkv = 2, 640, 10, 2
    log(f"[case] backward with dO x {s1:g} and x {s2:g}")
    q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=31))
    # the same bf16 values up to the power of two (a bf16 subnormal dO has
    # lost bits: the first input is the second one's values scaled back)
    do2 = (do.double() * s2).to(torch.bfloat16)
    do1 = (do2.double() * (s1 / s2)).to(torch.bfloat16)
    assert torch.equal(do1.double() * (s2 / s1), do2.double())
    outs = []
    for d in (do1, do2):
        qd, kd, vd = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = mm.flash_attention(qd, kd, vd, True, 5)
        out.backward(d)
        torch.cuda.synchronize()
        outs.append([t.grad.float().cpu() for t in (qd, kd, vd)])
    for name, a, b in zip(("dq", "dk", "dv"), *outs):
        assert torch.isfinite(b).all(), name
        # in float64 and back in a's units: (s2 / s1) a may not be a normal float32
        rel = ((b.double() * (s1 / s2) - a.double()).norm() / a.double().norm()).item()
        log(f"    {name}: rel-L2 vs linear {rel:.2e}")
        if s1 != 1.0:
            assert torch.equal(b, a * (s2 / s1)), name
        elif s2 >= 2.0 ** -100:
            assert rel <= 1e-3, name     # fp16 subnormal dS, then a bf16 rounding flipped here and there
        else:
            # bf16 outputs of this size are subnormal (spacing 2^-133): within one
            # step of the linear answer rounded to bf16
            want = (a.double() * (s2 / s1)).to(torch.bfloat16).double()
            err = (b.double() - want).abs().max().item()
            log(f"    {name}: max |dx - bf16(linear)| = {err / 2.0 ** -133:.1f} x 2^-133")
            assert err <= 2.0 ** -133, name


@pytest.mark.parametrize("dkdv_tiles,dq_tiles", [(0, 0), (1, 1), (0, 1)], ids=["t00", "t11", "t01"])
@pytest.mark.parametrize("B,S", [(8, 2048), (4, 4096)])
def test_dispatch_order_is_bitwise_neutral(hip_device, monkeypatch, B, S, dkdv_tiles, dq_tiles):
    """The dispatch order only changes which workgroup runs which item: every
    output is bitwise the one of the default (longest-first) order, which the
    full-size parity tests check against the oracle."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    H, Hkv = 10, 2
    for fwd_tiles in (0, 2):
        tables = [lib.mm1_attn_dispatch_order(0, fwd_tiles, B, S, H, Hkv, 1, 256, None, 0),
                  lib.mm1_attn_dispatch_order(1, dkdv_tiles, B, S, H, Hkv, 1, 256, None, 0),
                  lib.mm1_attn_dispatch_order(2, dq_tiles, B, S, H, Hkv, 1, 256, None, 0)]
        log(f"[case] dispatch order B={B} S={S} tiles=({fwd_tiles},{dkdv_tiles},{dq_tiles}) "
            f"table sizes {tables}")
        q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=B + S))
        sp = torch.cuda.current_stream(hip_device).cuda_stream
        p = lambda t: t.data_ptr()
        ws = _workspace(lib, B, S, H, Hkv, hip_device)

        def run(order):
            monkeypatch.setenv("MM1_DISPATCH_ORDER", "1" if order else "0")
            o, lse, st = _fwd_state(lib, q, k, v, True, hip_device, fwd_tiles)
            dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            assert lib.mm1_attn_bwd_tiles(p(o), p(do), p(lse), p(st), st.numel(), p(dq), p(dk), p(dv),
                                          p(ws), ws.numel(), B, S, H, Hkv, 128, 1, 128 ** -0.5, dkdv_tiles,
                                          dq_tiles, sp) == 0
            torch.cuda.synchronize()
            monkeypatch.delenv("MM1_DISPATCH_ORDER")
            return [x.cpu() for x in (o, lse, dq, dk, dv)]

        base, packed = run(False), run(True)
        for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), base, packed):
            assert torch.equal(x, y), name


def test_fp32_outputs_round_to_the_bf16_outputs(hip_device):
    """mm1_attn_fwd_f32 / mm1_attn_bwd_f32_tiles run the kernels of the bf16
    calls with fp32 stores: for every tiling, bf16 of their O, dQ, dK, dV is
    the bf16 call's output bitwise, with the same lse2 and forward state."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    for (B, S, H, Hkv, causal) in [(2, 1500, 10, 2, True), (1, 333, 6, 3, False), (4, 4096, 10, 2, True)]:
        log(f"[case] fp32 outputs B={B} S={S} H={H} Hkv={Hkv} causal={causal}")
        q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=S, rope_sigma=S == 4096))
        sp = torch.cuda.current_stream(hip_device).cuda_stream
        p = lambda t: t.data_ptr()
        args = (B, S, H, Hkv, 128, int(causal), 128 ** -0.5)
        ws = _workspace(lib, B, S, H, Hkv, hip_device)
        for t in range(lib.mm1_attn_tile_count(0)):
            o32 = torch.empty(q.shape, dtype=torch.float32, device=hip_device)
            l32 = torch.empty(B, H, S, dtype=torch.float32, device=hip_device)
            st32 = torch.empty(lib.mm1_attn_fwd_state_size(B, S, H, Hkv, 128), dtype=torch.uint8,
                               device=hip_device)
            assert lib.mm1_attn_fwd_f32(p(q), p(k), p(v), p(o32), p(l32), p(st32), st32.numel(), *args, t,
                                        sp) == 0
            o, lse, st = _fwd_state(lib, q, k, v, causal, hip_device, t)
            torch.cuda.synchronize()
            assert torch.equal(o, o32.to(torch.bfloat16)) and torch.equal(lse, l32), t
            assert torch.equal(st, st32), t            # the same state, residual bytes included
        for dkt in range(lib.mm1_attn_tile_count(1)):
            for dqt in range(lib.mm1_attn_tile_count(2)):
                g = [torch.empty_like(x) for x in (q, k, v)]
                g32 = [torch.empty(x.shape, dtype=torch.float32, device=hip_device) for x in (q, k, v)]
                assert lib.mm1_attn_bwd_tiles(p(o), p(do), p(lse), p(st), st.numel(), *(p(x) for x in g),
                                              p(ws), ws.numel(), *args, dkt, dqt, sp) == 0
                assert lib.mm1_attn_bwd_f32_tiles(p(o), p(do), p(lse), p(st), st.numel(),
                                                  *(p(x) for x in g32), p(ws), ws.numel(), *args, dkt, dqt,
                                                  sp) == 0
                torch.cuda.synchronize()
                for name, x, y in zip(("dq", "dk", "dv"), g, g32):
                    assert torch.equal(x, y.to(torch.bfloat16)), (dkt, dqt, name)


def test_autotune_records_a_compiled_winner(hip_device, monkeypatch, tmp_path):
    """get_kernel with AUTOTUNE and no record: every tiling is timed, the
    fastest is recorded under (device, kernel, shape) and the handle uses it;
    a second lookup is served from the record without a search."""
    from mimansm1_v1_amd import attention as A
    from mimansm1_v1_amd import tuned
    monkeypatch.setattr(tuned, "STORE", tmp_path / "store.json")
    monkeypatch.setattr(tuned, "TABLE", tmp_path / "none.json")
    monkeypatch.setattr(A, "_kernels", {})
    monkeypatch.setattr(A, "AUTOTUNE", True)
    shape = (1, 10, 640, 128, True, 5)
    log(f"[case] autotune {shape}")
    best, ms, results = A.autotune("bwd", shape)
    assert len(results) == len(A.bwd_configs()) and ms == min(r[0] for r in results) > 0
    assert A.tile_index("bwd", best) is not None
    for kind in ("fwd", "bwd"):
        handle = A.get_kernel(kind, *shape)
        assert handle.latency is not None and handle.latency > 0
        assert tuned.lookup(f"attention_{kind}", shape) == handle.config
    calls = []
    monkeypatch.setattr(A, "autotune", lambda *a, **k: calls.append(a))
    monkeypatch.setattr(A, "_kernels", {})
    assert A.get_kernel("fwd", *shape).latency is None and not calls
    q, k, v, do = R.make_inputs(1, 640, 10, 2, 128, seed=21)
    o, lse, dq, dk, dv = hip_run(q, k, v, do, True, 5, hip_device)
    case = "autotuned B1 S640"
    pre = precast(q, k, v, do, True, hip_device)
    assert_bf16_close("O", o, R.attention(q, k, v, True, 5, cast=False), log, precast=pre[0], case=case)
    check_grads(case, (dq, dk, dv), R.grads(q, k, v, do, True, 5), pre,
                R.grads_analytic(q, k, v, do, True, 5, bf16_products=True))


def test_config1_forward_vs_cpu_oracle(hip_device):
    case = "config 1"
    log("[case] config 1: B1 S512 fwd")
    q, k, v, _ = R.config_inputs(1)
    o, lse, *_ = hip_run(q, k, v, None, True, 5, hip_device, backward=False)
    pre = precast(q, k, v, None, True, hip_device)
    assert_bf16_close("O", o, R.attention(q, k, v, True, 5, cast=False), log, precast=pre[0], case=case)
    assert_lse_close(lse, R.lse2(q, k, True, 5), log, case=case)


def test_gpu_oracle_device_agrees(hip_device):
    """The chunked fp32 oracle gives the same numbers on the GPU as on the CPU."""
    q, k, v, do = R.make_inputs(1, 384, 10, 2, 128, seed=11)
    o_c, l_c = R.forward_chunked(q, k, v, True, 5)
    g_c = R.grads_analytic(q, k, v, do, True, 5)
    e_c = R.grads_analytic(q, k, v, do, True, 5, bf16_products=True)
    dev = [t.to(hip_device) for t in (q, k, v, do)]
    o_g, l_g = R.forward_chunked(*dev[:3], True, 5)
    g_g = R.grads_analytic(*dev, True, 5)
    e_g = R.grads_analytic(*dev, True, 5, bf16_products=True)
    for a, b in zip((o_c, l_c, *g_c), (o_g, l_g, *g_g)):
        assert (a - b.cpu()).abs().max().item() < 1e-4
    # the emulation's rounding decisions may differ in a few elements between
    # the two devices' fp32 arithmetic (one bf16 ulp of one product term each)
    for a, b in zip(e_c, e_g):
        assert ((a - b.cpu()).norm() / a.norm()).item() < 1e-4
    # and the chunked closed form agrees with autograd through the reference
    for a, b in zip(g_c, R.grads(q, k, v, do, True, 5)):
        assert (a - b).abs().max().item() < 1e-4


def _full_size_case(hip_device, case, q, k, v, do, G):
    o, lse, dq, dk, dv = hip_run(q, k, v, do, True, G, hip_device)
    pre = precast(q, k, v, do, True, hip_device)
    dev = [t.to(hip_device) for t in (q, k, v, do)]
    want_o, want_lse = R.forward_chunked(*dev[:3], True, G)
    assert_bf16_close("O", o, want_o, log, precast=pre[0], case=case)
    assert_lse_close(lse, want_lse, log, case=case)
    del want_o, want_lse
    want = [t.cpu() for t in R.grads_analytic(*dev, True, G)]
    emu = [t.cpu() for t in R.grads_analytic(*dev, True, G, bf16_products=True)]
    del dev
    torch.cuda.empty_cache()
    check_grads(case, (dq, dk, dv), want, pre, emu)


@pytest.mark.parametrize("config", [2, 3, 4])
def test_full_config_vs_gpu_oracle(hip_device, config):
    case = f"config {config}"
    log(f"[case] config {config} full size")
    q, k, v, do = R.config_inputs(config)
    _full_size_case(hip_device, case, q, k, v, do, 5)


RAGGED = [(3, 4097, 10, 2), (5, 2999, 10, 2), (2, 7777, 10, 2), (1, 16384, 10, 2)]


@pytest.mark.parametrize("B,S,H,Hkv", RAGGED, ids=[f"B{b}S{s}" for b, s, _, _ in RAGGED])
def test_large_ragged_vs_gpu_oracle(hip_device, B, S, H, Hkv):
    """Sequence lengths that are no multiple of any tile (32, 64, 128, 256)
    at sizes where the launches use the packed dispatch tables with item
    counts that are no multiple of 8 (empty launch slots): the same gates as
    the full configs, against the chunked closed form on the GPU."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    tables = [lib.mm1_attn_dispatch_order(0, 0, B, S, H, Hkv, 1, 256, None, 0),
              lib.mm1_attn_dispatch_order(2, 1, B, S, H, Hkv, 1, 256, None, 0)]
    log(f"[case] ragged B={B} S={S} H={H} Hkv={Hkv} dispatch tables {tables}")
    assert min(tables) > 0
    q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=S)
    _full_size_case(hip_device, f"ragged B{B} S{S}", q, k, v, do, H // Hkv)


def _capi_run(lib, q, k, v, do, H, Hkv, causal, dkdv_tiles, dq_tiles, device):
    """Forward (default tiling) + backward through the C ABI with explicit
    backward tilings (GPU tensors): o, lse2, state, dq, dk, dv."""
    B, S = q.shape[0], q.shape[1]
    sp = torch.cuda.current_stream(device).cuda_stream
    p = lambda t: t.data_ptr()
    o, lse, st = _fwd_state(lib, q, k, v, causal, device, 0)
    ws = _workspace(lib, B, S, H, Hkv, device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    args = (B, S, H, Hkv, 128, int(causal), 128 ** -0.5)
    assert lib.mm1_attn_bwd_tiles(p(o), p(do), p(lse), p(st), st.numel(), p(dq), p(dk), p(dv),
                                  p(ws), ws.numel(), *args, dkdv_tiles, dq_tiles, sp) == 0
    torch.cuda.synchronize()
    return o, lse, st, dq, dk, dv


GROUPED = [(8, 2048, 10, 2, True), (2, 8192, 10, 2, True), (2, 7777, 10, 2, True),
           (3, 1000, 10, 2, True), (2, 2048, 10, 2, False), (1, 4096, 8, 1, True),
           (1, 3001, 16, 1, True), (2, 1111, 16, 1, False)]


@pytest.mark.parametrize("B,S,H,Hkv,causal", GROUPED,
                         ids=[f"B{b}S{s}G{h // kv}{'c' if c else 'f'}" for b, s, h, kv, c in GROUPED])
def test_grouped_dkdv_vs_gpu_oracle(hip_device, B, S, H, Hkv, causal):
    """The grouped dK/dV tiling (one workgroup walks all G heads of a KV head
    for its key tile; long key tiles split into chunks whose fp32 partials the
    dQ launch sums) at sizes where its plan splits key tiles and launches a
    dispatch table: dK/dV against the chunked closed form on the GPU, and the
    staged calls bitwise equal to the combined one."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    plan = (ctypes.c_int * 5)()
    assert lib.mm1_attn_dkdv_plan(B, S, H, Hkv, int(causal), 256, plan) == 0
    case = f"grouped B{B} S{S} H{H} Hkv{Hkv} {'causal' if causal else 'full'}"
    log(f"[case] {case} plan {list(plan)}")
    G = H // Hkv
    qc, kc, vc, doc = R.make_inputs(B, S, H, Hkv, 128, seed=S + B)
    q, k, v, do = (t.to(hip_device) for t in (qc, kc, vc, doc))
    o, lse, st, dq, dk, dv = _capi_run(lib, q, k, v, do, H, Hkv, causal, 0, 1, hip_device)
    pre = precast(qc, kc, vc, doc, causal, hip_device, tiles=(0, (0, 1)))
    want = [t.cpu() for t in R.grads_analytic(q, k, v, do, causal, G)]
    emu = [t.cpu() for t in R.grads_analytic(q, k, v, do, causal, G, bf16_products=True)]
    check_grads(case, (dq.cpu(), dk.cpu(), dv.cpu()), want, pre, emu)
    del want, emu
    # staged: prep, dK/dV, then the separate reduction
    sp = torch.cuda.current_stream(hip_device).cuda_stream
    p = lambda t: t.data_ptr()
    ws = _workspace(lib, B, S, H, Hkv, hip_device)
    sk, sv = torch.empty_like(k), torch.empty_like(v)
    args = (B, S, H, Hkv, 128, int(causal), 128 ** -0.5)
    assert lib.mm1_attn_bwd_prep(p(o), p(do), p(lse), p(st), st.numel(), p(ws), ws.numel(), *args[:5], args[6],
                                 sp) == 0
    assert lib.mm1_attn_bwd_dkdv_tiles(p(st), st.numel(), p(sk), p(sv), p(ws), ws.numel(), *args, 0, sp) == 0
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(p(ws), ws.numel(), p(sk), p(sv), B, S, H, Hkv, 128,
                                              int(causal), 0, sp) == 0
    torch.cuda.synchronize()
    assert torch.equal(sk, dk) and torch.equal(sv, dv)


def test_backward_deterministic(hip_device):
    log("[case] determinism B2 S1024")
    q, k, v, do = R.make_inputs(2, 1024, 10, 2, 128, seed=5)
    a = hip_run(q, k, v, do, True, 5, hip_device)
    b = hip_run(q, k, v, do, True, 5, hip_device)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("shape", [(2, 1000, 10, 2, True), (1, 333, 6, 3, False), (1, 256, 4, 4, True)],
                         ids=["B2S1000G5causal", "B1S333G2full", "B1S256G1causal"])
def test_backward_stages_match_combined(hip_device, shape):
    """mm1_attn_bwd (prep, dK/dV, then dQ with the group sum in its tail) and
    the separate stages (prep, dK/dV, group sum, dQ) write bitwise-identical
    gradients, and so does the reference-signature path (mm1_attn_prep +
    mm1_attn_bwd_prep_delta) given the Delta the state-based prep computed."""
    from mimansm1_v1_amd import _lib
    B, S, H, Hkv, causal = shape
    log(f"[case] stages vs combined {shape}")
    lib = _lib.load()
    q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=9))
    sp = torch.cuda.current_stream(hip_device).cuda_stream
    p = lambda t: t.data_ptr()
    o, lse, st = _fwd_state(lib, q, k, v, causal, hip_device)
    ws = _workspace(lib, B, S, H, Hkv, hip_device)
    args = (B, S, H, Hkv, 128, int(causal), 128 ** -0.5)
    S_, W_ = (p(st), st.numel()), (p(ws), ws.numel())
    outs = []
    for mode in ("combined", "staged", "reference"):
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        if mode == "combined":
            assert lib.mm1_attn_bwd(p(o), p(do), p(lse), *S_, p(dq), p(dk), p(dv), *W_, *args, sp) == 0
        elif mode == "staged":
            assert lib.mm1_attn_bwd_prep(p(o), p(do), p(lse), *S_, *W_, *args[:5], args[6], sp) == 0
            assert lib.mm1_attn_bwd_dkdv_tiles(*S_, p(dk), p(dv), *W_, *args, -1, sp) == 0
            assert lib.mm1_attn_bwd_dkdv_reduce_tiles(*W_, p(dk), p(dv), B, S, H, Hkv, 128, int(causal), -1,
                                                      sp) == 0
            assert lib.mm1_attn_bwd_dq_tiles(*S_, p(dq), *W_, *args, -1, sp) == 0
        else:
            # Delta as the state-based prep computed it (-2^E Delta in the
            # workspace, E = 0 for these inputs), through the reference
            # signature's path
            r_do, r_delta, r_lse, r_scale = _ws_regions(lib, B, S, H, Hkv)
            torch.cuda.synchronize()
            assert ws[r_scale:r_scale + 4].view(torch.float32).item() == 1.0
            delta = -ws[r_delta:r_delta + 4 * B * H * S].view(torch.float32).view(B, H, S).clone()
            st2 = torch.empty_like(st)
            ws2 = torch.empty_like(ws)
            assert lib.mm1_attn_prep(p(q), p(k), p(v), p(st2), st2.numel(), *args[:5], sp) == 0
            assert lib.mm1_attn_bwd_prep_delta(p(do), p(delta), p(lse), p(st2), st2.numel(), p(ws2), ws2.numel(),
                                               *args[:5], args[6], sp) == 0
            assert lib.mm1_attn_bwd_dkdv_tiles(p(st2), st2.numel(), p(dk), p(dv), p(ws2), ws2.numel(), *args, -1,
                                               sp) == 0
            assert lib.mm1_attn_bwd_dq_reduce_tiles(p(st2), st2.numel(), p(dq), p(dk), p(dv), p(ws2), ws2.numel(),
                                                    *args, -1, -1, sp) == 0
        torch.cuda.synchronize()
        outs.append((dq.cpu(), dk.cpu(), dv.cpu()))
    for other in outs[1:]:
        for name, x, y in zip(("dq", "dk", "dv"), outs[0], other):
            assert torch.equal(x, y), name
            assert torch.isfinite(x.float()).all(), name


def test_lse_lower_bound_and_rows_sum(hip_device):
    """lse2_i >= max_j s_ij * log2(e) and softmax rows sum to one:
    with V = all ones, O = 1 exactly (up to bf16)."""
    q, k, _, _ = R.make_inputs(1, 777, 10, 2, 128, seed=9)
    v = torch.ones(1, 777, 2, 128, dtype=torch.bfloat16)
    o, lse, *_ = hip_run(q, k, v, None, True, 5, hip_device, backward=False)
    # P is rounded to fp16 for the MFMA while l sums the fp32 values (the
    # reference rounds to bf16 there, AT:173-180), so O = 1 holds to the
    # rounding of P and of the bf16 output only.
    assert (o.float() - 1).abs().max().item() <= 8e-3
    smax = R.scores(q, k, True, 5).amax(-1) * R.LOG2E
    assert (lse - smax).min().item() >= -1e-4


def test_capi_errors_on_device(hip_device):
    import mimansm1_v1_amd._lib as L
    lib = L.load()
    q = torch.zeros(1, 64, 10, 128, dtype=torch.bfloat16, device=hip_device)
    kv = torch.zeros(1, 64, 2, 128, dtype=torch.bfloat16, device=hip_device)
    lse = torch.zeros(1, 10, 64, dtype=torch.float32, device=hip_device)
    st = torch.empty(lib.mm1_attn_fwd_state_size(1, 64, 10, 2, 128), dtype=torch.uint8, device=hip_device)
    ws = _workspace(lib, 1, 64, 10, 2, hip_device)
    rc = lib.mm1_attn_bwd(q.data_ptr(), q.data_ptr(), lse.data_ptr(), st.data_ptr(), st.numel(), q.data_ptr(),
                          kv.data_ptr(), kv.data_ptr(), ws.data_ptr(), ws.numel() - 4, 1, 64, 10, 2, 128, 1, 0.1,
                          None)
    assert rc == -4
    rc = lib.mm1_attn_fwd(q.data_ptr() + 2, kv.data_ptr(), kv.data_ptr(), q.data_ptr(), lse.data_ptr(),
                          st.data_ptr(), st.numel(), 1, 64, 10, 2, 128, 1, 0.1, None)
    assert rc == -6
    torch.cuda.synchronize()


def test_native_library_is_in_tree(hip_device):
    import mimansm1_v1_amd._lib as L
    L.load()
    maps = open("/proc/self/maps").read()
    assert str(L.library_path()) in maps


def test_golden_fixtures(hip_device):
    """Kernel vs the committed fp64 brute-force fixtures (tests/golden)."""
    from tests.golden.make_golden import load_cases
    for name, c in load_cases().items():
        B, S, H, Hkv, causal = c["meta"]
        case = f"golden {name}"
        log(f"[case] {case}")
        o, lse, dq, dk, dv = hip_run(c["q"], c["k"], c["v"], c["do"], causal, H // Hkv, hip_device)
        pre = precast(c["q"], c["k"], c["v"], c["do"], causal, hip_device)
        assert_bf16_close("O", o, c["o"], log, precast=pre[0], case=case)
        assert_lse_close(lse, c["lse2"], log, case=case)
        emu = R.grads_analytic(c["q"], c["k"], c["v"], c["do"], causal, H // Hkv, bf16_products=True)
        check_grads(case, (dq, dk, dv), (c["dq"], c["dk"], c["dv"]), pre, emu)


# ---------------------------------------------------------------------------
# Sublayer prologue (config 5): QK-RMSNorm + RoPE kernel and the full sublayer.

def assert_prologue_close(name, got, want):
    """A bf16 output of the sublayer prologue (not one of the attention
    outputs the north-star gates name) against the oracle's bf16 chain: both
    round the same fp32 values, so only fp32 summation order and rsqrt may
    flip a rounding, and RoPE's sums of two rounded products may then differ
    by one bf16 step of a product near cancellation.  Gate: rel-L2 <= 5e-3 and
    max-abs <= 2e-2 + the output's own bf16 rounding floor."""
    from tests.parity import metrics
    m = metrics(got, want.float())
    log(f"    {name:4s} max_abs {m['max_abs']:.3e} (floor {m['floor']:.3e})  rel_l2 {m['rel_l2']:.3e}")
    assert m["finite"], name
    assert m["rel_l2"] <= 5e-3 and m["max_abs"] <= 2e-2 + m["floor"], (name, m)


def _qkv_inputs(B, S, H, Hkv, seed, norm=True):
    gen = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(B, S, (H + 2 * Hkv) * 128, generator=gen) * 2).to(torch.bfloat16)
    wq = (1 + 0.3 * torch.randn(128, generator=gen)) if norm else None
    wk = (1 + 0.3 * torch.randn(128, generator=gen)) if norm else None
    cos, sin = R.rope_tables(128, S + 5, 10000.0)
    grads = [torch.randn(B, S, h, 128, generator=gen).to(torch.bfloat16) for h in (H, Hkv, Hkv)]
    return qkv, wq, wk, cos, sin, grads


@pytest.mark.parametrize("B,S,H,Hkv,norm", [(2, 100, 10, 2, True), (1, 257, 6, 3, True), (1, 64, 4, 4, False)],
                         ids=["B2S100G5", "B1S257G2", "B1S64nonorm"])
def test_qknorm_rope_kernel_vs_oracle(hip_device, B, S, H, Hkv, norm):
    """Forward: bf16 Q/K/V of the kernel against the oracle's bf16 chain
    (near bit-exact: only the fp32 mean-of-squares order and rsqrt may flip a
    rounding).  Backward: dqkv and the norm-weight gradients against CPU
    autograd through the same chain."""
    import mimansm1_v1_amd as mm
    from mimansm1_v1_amd import attention as A
    log(f"[case] qknorm_rope B={B} S={S} H={H} Hkv={Hkv} norm={norm}")
    qkv, wq, wk, cos, sin, (gq, gk, gv) = _qkv_inputs(B, S, H, Hkv, seed=S + H, norm=norm)
    dev = lambda t: None if t is None else t.to(hip_device)
    qkv_d = qkv.to(hip_device).requires_grad_(True)
    wq_d = dev(wq).requires_grad_(True) if norm else None
    wk_d = dev(wk).requires_grad_(True) if norm else None
    q, k, v = A.qknorm_rope(qkv_d, wq_d, wk_d, dev(cos), dev(sin), H, Hkv, 1e-5)
    torch.autograd.backward((q, k, v), (dev(gq), dev(gk), dev(gv)))
    torch.cuda.synchronize()

    qkv_c = qkv.clone().requires_grad_(True)
    wq_c = wq.clone().requires_grad_(True) if norm else None
    wk_c = wk.clone().requires_grad_(True) if norm else None
    wantq, wantk, wantv = R.qknorm_rope(qkv_c, wq_c, wk_c, cos, sin, H, Hkv, 1e-5)
    torch.autograd.backward((wantq, wantk, wantv), (gq, gk, gv))
    for name, got, want in (("Q", q, wantq), ("K", k, wantk)):
        got = got.detach().cpu()
        same = (got == want.detach()).float().mean().item()
        log(f"  {name}: {100 * same:.3f}% bitwise equal")
        assert same > 0.99, name
        assert_prologue_close(name, got, want.detach())
    assert torch.equal(v.detach().cpu(), wantv.detach())
    dqkv = qkv_d.grad.cpu()
    same = (dqkv == qkv_c.grad).float().mean().item()
    log(f"  dqkv: {100 * same:.3f}% bitwise equal")
    assert same > 0.98
    assert_prologue_close("dqkv", dqkv, qkv_c.grad)
    if norm:
        for name, got, want in (("dwq", wq_d.grad, wq_c.grad), ("dwk", wk_d.grad, wk_c.grad)):
            err = ((got.cpu() - want).norm() / want.norm()).item()
            log(f"  {name}: rel_l2 {err:.2e}")
            assert err < 2e-3, name


def test_sublayer_skipped_cast_is_bitwise_neutral(hip_device, monkeypatch):
    """Under bf16 autocast the "hip" sublayer keeps the attention output in
    bf16 instead of the reference's cast to x.dtype that wo casts straight
    back: output and every gradient equal the path with the cast, bitwise."""
    from mimansm1_v1_amd import attention as A
    log("[case] sublayer B2 S256: skipped fp32 round trip vs the reference's cast")
    torch.manual_seed(0)
    cfg = A.AttnConfig(max_seq_len=256)
    mod = A.Attention(cfg, A.Rotary(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta)).to(hip_device)
    with torch.no_grad():
        for lin in (mod.wq, mod.wk, mod.wv, mod.wo):
            lin.weight.normal_(0.0, 0.02)
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(2, 256, cfg.d_model, generator=gen).to(hip_device)
    dy = torch.randn(2, 256, cfg.d_model, generator=gen).to(hip_device)

    def run():
        mod.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = mod(xi, backend="hip")
        y.backward(dy.to(y.dtype))
        torch.cuda.synchronize()
        return [y.detach().cpu(), xi.grad.cpu()] + [p.grad.cpu() for p in mod.parameters() if p.grad is not None]

    skipped = run()
    monkeypatch.setattr(A, "_skip_attn_out_cast", lambda: False)   # take the reference's cast
    cast = run()
    assert len(skipped) == len(cast)
    for i, (a, b) in enumerate(zip(skipped, cast)):
        assert a.dtype == b.dtype and torch.equal(a, b), i


def test_sublayer_hip_matches_reference_backend(hip_device):
    """The config-5 sublayer (fused QKV GEMM, QK-norm + RoPE kernel, flash
    attention, wo) under bf16 autocast against the same module run with the
    reference's "math" backend: output and every gradient."""
    from mimansm1_v1_amd import attention as A
    log("[case] sublayer B2 S384 hip vs math (bf16 autocast)")
    torch.manual_seed(0)
    cfg = A.AttnConfig(max_seq_len=512)
    mod = A.Attention(cfg, A.Rotary(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta)).to(hip_device)
    with torch.no_grad():
        for lin in (mod.wq, mod.wk, mod.wv, mod.wo):
            lin.weight.normal_(0.0, 0.02)
        mod.q_norm.weight.uniform_(0.7, 1.3)
        mod.k_norm.weight.uniform_(0.7, 1.3)
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(2, 384, cfg.d_model, generator=gen).to(hip_device)
    dy = torch.randn(2, 384, cfg.d_model, generator=gen).to(hip_device)
    results = {}
    for backend in ("hip", "math"):
        mod.zero_grad(set_to_none=True)
        xi = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = mod(xi, backend=backend)
        y.backward(dy.to(y.dtype))
        torch.cuda.synchronize()
        results[backend] = [y.detach().float().cpu(), xi.grad.float().cpu()] + [
            p.grad.float().cpu() for p in (mod.wq.weight, mod.wk.weight, mod.wv.weight, mod.wo.weight,
                                           mod.q_norm.weight, mod.k_norm.weight)]
    names = ["y", "dx", "dwq", "dwk", "dwv", "dwo", "dq_norm", "dk_norm"]
    for name, got, want in zip(names, results["hip"], results["math"]):
        err = ((got - want).norm() / want.norm()).item()
        log(f"  {name}: rel_l2 {err:.2e}")
        assert torch.isfinite(got).all(), name
        assert err < 1e-2, name


@pytest.mark.parametrize("shape", [(2, 2048, 1280, 1792), (1, 100, 256, 384), (3, 77, 128, 128)],
                         ids=["T4096chunks", "T100plain", "T231plain"])
def test_bf16_linear_projection(hip_device, shape):
    """The sublayer projections' autograd Function: forward bitwise equal to
    autocast's F.linear; dX and dW against fp64 products of the same bf16
    operands (dX within bf16 rounding; dW in fp32, no less accurate than the
    bf16 dW of autograd through F.linear)."""
    from mimansm1_v1_amd import attention as A
    B, S, K, N = shape
    log(f"[case] BF16Linear {shape}")
    gen = torch.Generator().manual_seed(K + N)
    x = torch.randn(B, S, K, generator=gen).to(hip_device)
    w = (torch.randn(N, K, generator=gen) * 0.02).to(hip_device)
    dy = torch.randn(B, S, N, generator=gen).to(hip_device)
    outs = {}
    for kind in ("fn", "autograd"):
        xi, wi = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = A.BF16Linear.apply(xi, wi) if kind == "fn" else F.linear(xi, wi)
        y.backward(dy.to(y.dtype))
        torch.cuda.synchronize()
        outs[kind] = (y.detach(), xi.grad, wi.grad)
    assert torch.equal(outs["fn"][0], outs["autograd"][0])
    xb, wb, dyb = (t.to(torch.bfloat16).double() for t in (x, w, dy))
    want_dx = (dyb @ wb).float()
    want_dw = torch.einsum("bsn,bsk->nk", dyb, xb).float()
    rel = lambda a, b: ((a.float() - b).norm() / b.norm()).item()
    e_dx, e_dx_ag = rel(outs["fn"][1], want_dx), rel(outs["autograd"][1], want_dx)
    e_dw, e_dw_ag = rel(outs["fn"][2], want_dw), rel(outs["autograd"][2], want_dw)
    log(f"    dX rel_l2 {e_dx:.2e} (autograd {e_dx_ag:.2e}); dW rel_l2 {e_dw:.2e} (autograd {e_dw_ag:.2e})")
    assert outs["fn"][1].dtype == x.dtype and outs["fn"][2].dtype == w.dtype
    assert e_dx < 5e-3 and e_dw < 1e-4 and e_dw <= e_dw_ag + 1e-6


@pytest.mark.parametrize("S", [1111, 2048])
def test_bench_overlapped_step_matches_staged_step(hip_device, S):
    """bench.py's timed step with dQ beside dK/dV on a second stream (what a
    tile record with overlap_dq runs) writes the same O, lse2, dQ, dK and dV,
    bitwise, as its per-stage step on one stream."""
    import bench
    from mimansm1_v1_amd import _lib
    log(f"[case] bench step overlapped vs staged B1 S{S}")
    wl = bench.Workload(_lib.load(), 1, S, hip_device, {"fwd": 0, "dkdv": 0, "dq": 1, "overlap": True})
    outs = []
    for staged in (False, True):
        for t in (wl.o, wl.lse, wl.dq, wl.dk, wl.dv):
            t.fill_(7.0)
        marks = [torch.cuda.Event() for _ in bench.Workload.STAGES] if staged else None
        wl.step(marks)
        torch.cuda.synchronize()
        outs.append([t.clone() for t in (wl.o, wl.lse, wl.dq, wl.dk, wl.dv)])
    for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), *outs):
        assert torch.equal(x, y), name
