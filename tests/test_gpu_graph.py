"""The HIP kernels under HIP graph capture (GPU only).

The library allocates no device memory, never synchronises and takes its
workgroup dispatch tables as kernel arguments, so a caller can capture a
whole attention fwd+bwd step (or the SwiGLU / head passes) in a graph and
replay it.  Each test captures the C-ABI calls on preallocated tensors and
replays the graph several times, with eager launches of the same calls and
host synchronisations in between, and checks every replay bitwise against
the eager result (deterministic kernels: any difference is a capture bug)."""
from __future__ import annotations

import sys

import pytest
import torch

from oracle import reference as R

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _replay_and_compare(step, outputs, replays=3):
    """step(stream_handle) launches the calls; outputs are the tensors they
    write.  Eager result first, then capture, then replays interleaved with
    eager runs; every replay must equal the eager result bitwise."""
    cur = torch.cuda.current_stream()
    step(cur.cuda_stream)
    torch.cuda.synchronize()
    want = [t.clone() for t in outputs]
    side = torch.cuda.Stream()
    side.wait_stream(cur)
    with torch.cuda.stream(side):
        step(side.cuda_stream)                    # warm-up on the capture stream's kind
    cur.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(torch.cuda.current_stream().cuda_stream)
    for r in range(replays):
        for t in outputs:
            t.fill_(float("nan") if t.is_floating_point() else 0)   # a fill kernel, not a memset node
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outputs, want)):
            assert torch.equal(got, ref), f"replay {r}: output {i} differs from the eager result"
        step(cur.cuda_stream)                     # eager work between replays
        torch.cuda.synchronize()
        log(f"    replay {r} equal to eager")


@pytest.mark.parametrize("B,S,tiles", [(2, 1024, (-1, -1, -1)), (1, 777, (0, 1, 0))],
                         ids=["B2S1024-table", "B1S777-t010"])
def test_attention_step_graph_replays(hip_device, B, S, tiles):
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    H, Hkv, D = 10, 2, 128
    log(f"[case] attention graph B={B} S={S} tiles={tiles}")
    q, k, v, do = (t.to(hip_device) for t in R.make_inputs(B, S, H, Hkv, D, seed=S))
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=hip_device)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    st = torch.empty(lib.mm1_attn_fwd_state_size(B, S, H, Hkv, D), dtype=torch.uint8, device=hip_device)
    ws = torch.empty(lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, D), dtype=torch.uint8, device=hip_device)
    p = lambda t: t.data_ptr()
    args = (B, S, H, Hkv, D, 1, D ** -0.5)

    def step(sp):
        _lib.check(lib.mm1_attn_fwd_tiles(p(q), p(k), p(v), p(o), p(lse), p(st), st.numel(), *args, tiles[0], sp),
                   "fwd")
        _lib.check(lib.mm1_attn_bwd_tiles(p(o), p(do), p(lse), p(st), st.numel(), p(dq), p(dk), p(dv), p(ws),
                                          ws.numel(), *args, tiles[1], tiles[2], sp), "bwd")

    _replay_and_compare(step, [o, lse, dq, dk, dv])


@pytest.mark.parametrize("S", [777, 2048])
def test_overlapped_backward_graph_replays(hip_device, S):
    """The backward handle with a tile record that puts dQ on a second stream
    (fork from the caller's stream by an event, join back by another) captures
    as one graph: every replay equals the eager call bitwise."""
    from mimansm1_v1_amd import attention as A
    H, Hkv, D = 10, 2, 128
    log(f"[case] overlapped backward graph B=1 S={S}")
    q, k, v, do = (t.to(hip_device) for t in R.make_inputs(1, S, H, Hkv, D, seed=S + 3))
    shape = (1, H, S, D, True, H // Hkv)
    o, lse, state = A.FwdKernel(shape, A.FWD_TILES).run(q, k, v)
    config = dict(A.BWD_TILES, dq_block_M=256, dq_waves=8, dq_stages=3, overlap_dq=True)
    bwd = A.BwdKernel(shape, config)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    def step(_sp):   # the handle launches on torch's current stream (and its side stream)
        bwd.run_saved(o, do, lse, state, dq, dk, dv)

    _replay_and_compare(step, [dq, dk, dv])


def test_swiglu_and_head_graph_replays(hip_device):
    from mimansm1_v1_amd import _lib
    from mimansm1_v1_amd import swiglu as SG
    lib = _lib.load()
    log("[case] SwiGLU gate/up + grad and LM-head passes under graph capture")
    gen = torch.Generator().manual_seed(3)
    T, d, F, V = 300, 256, 384, 1280
    mk = lambda *s, std=1.0: (torch.randn(*s, generator=gen) * std).to(torch.bfloat16).to(hip_device)
    x, wg, wu = mk(T, d), mk(d, F, std=0.05), mk(d, F, std=0.05)
    gate, up, act = (torch.empty(T, F, dtype=torch.bfloat16, device=hip_device) for _ in range(3))
    dact = mk(T, F)
    dgu = torch.empty(T, 2 * F, dtype=torch.bfloat16, device=hip_device)
    w = mk(d, V, std=0.05)
    targets = torch.randint(0, V, (T,), generator=gen).to(hip_device)
    targets[:4] = -100
    lse = torch.empty(T, dtype=torch.float32, device=hip_device)
    tl, loss = torch.empty_like(lse), torch.empty_like(lse)
    nws = lib.mm1_lm_head_workspace_size(T, V)
    ws = torch.empty(max(nws // 4, 1), dtype=torch.float32, device=hip_device)
    scale = torch.tensor([1.0 / (T - 4)], device=hip_device)
    dlogits = torch.empty(T, V, dtype=torch.bfloat16, device=hip_device)
    p = lambda t: t.data_ptr()

    def step(sp):
        _lib.check(lib.mm1_swiglu_gate_up(p(x), p(wg), p(wu), p(gate), p(up), p(act), T, d, F,
                                          SG.MODE_TRAIN, sp), "gate_up")
        _lib.check(lib.mm1_swiglu_grad(p(dact), p(gate), p(up), p(dgu), p(dgu) + 2 * F, T, F, 2 * F, sp),
                   "grad")
        _lib.check(lib.mm1_lm_head_lse(p(x), p(w), p(targets), -100, p(lse), p(tl), p(loss), p(ws), nws,
                                       T, d, V, sp), "lse")
        _lib.check(lib.mm1_lm_head_dlogits(p(x), p(w), p(targets), -100, p(lse), p(scale), p(dlogits), V,
                                           T, d, V, 0, V, sp), "dlogits")

    _replay_and_compare(step, [gate, up, act, dgu, lse, tl, loss, dlogits])
