"""mm1_attn_bwd_noalloc (GPU): the backward whose workspace (fp16 dO, Delta,
the dK/dV partial sums) lives in the library's static device scratch instead
of a caller's buffer."""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _backward_pair(lib, B, S, H, Hkv, causal, seed, device):
    """dq, dk, dv from mm1_attn_bwd_noalloc and from mm1_attn_bwd (default
    tilings, caller workspace) on the same forward."""
    q, k, v, do = (t.to(device) for t in R.make_inputs(B, S, H, Hkv, 128, seed=seed))
    sp = torch.cuda.current_stream(device).cuda_stream
    p = lambda t: t.data_ptr()
    args = (B, S, H, Hkv, 128, int(causal), 128 ** -0.5)
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=device)
    st = torch.empty(lib.mm1_attn_fwd_state_size(B, S, H, Hkv, 128), dtype=torch.uint8, device=device)
    assert lib.mm1_attn_fwd(p(q), p(k), p(v), p(o), p(lse), p(st), st.numel(), *args, sp) == 0
    na = [torch.full_like(t, float("nan")) for t in (q, k, v)]
    rc = lib.mm1_attn_bwd_noalloc(p(o), p(do), p(lse), p(st), st.numel(), *(p(t) for t in na), *args, sp)
    assert rc == 0, lib.mm1_attn_strerror(rc)
    ws = torch.empty(lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, 128), dtype=torch.uint8, device=device)
    ref = [torch.empty_like(t) for t in (q, k, v)]
    assert lib.mm1_attn_bwd(p(o), p(do), p(lse), p(st), st.numel(), *(p(t) for t in ref), p(ws), ws.numel(),
                            *args, sp) == 0
    torch.cuda.synchronize()
    return na, ref


def test_noalloc_backward_matches_workspace_backward(hip_device):
    """Two calls in a row on one device, the second smaller (so it reads a
    scratch that holds the first call's partials): both bitwise equal to
    mm1_attn_bwd; shapes whose partials exceed the scratch are refused."""
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    for (B, S, H, Hkv, causal, seed) in [(2, 8192, 10, 2, True, 1), (1, 3000, 10, 2, True, 2),
                                         (2, 1111, 16, 1, False, 3)]:
        need = lib.mm1_attn_bwd_noalloc_scratch_size(B, S, H, Hkv, 128, int(causal))
        log(f"[case] noalloc B={B} S={S} H={H} Hkv={Hkv} causal={causal} scratch {need / 2**20:.1f} MiB")
        assert 0 < need <= 256 << 20
        got, want = _backward_pair(lib, B, S, H, Hkv, causal, seed, hip_device)
        for name, a, b in zip(("dq", "dk", "dv"), got, want):
            assert torch.equal(a, b), name
    # too large for the scratch: refused before any launch
    B, S = 1, 32768
    assert lib.mm1_attn_bwd_noalloc_scratch_size(B, S, 10, 2, 128, 1) > 256 << 20
    dummy = torch.empty(16, dtype=torch.bfloat16, device=hip_device)
    f = torch.empty(16, dtype=torch.float32, device=hip_device)
    p = dummy.data_ptr()
    nst = lib.mm1_attn_fwd_state_size(B, S, 10, 2, 128)
    assert lib.mm1_attn_bwd_noalloc(p, p, f.data_ptr(), p, nst, p, p, p, B, S, 10, 2, 128, 1,
                                    128 ** -0.5, None) == -9
