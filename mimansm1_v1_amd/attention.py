"""MI355X causal GQA flash attention with the call surface of Mimans M1's
``mimans.model.attention_tilelang`` (CODE/mimans/model/attention_tilelang.py).

Drop-in surface (same names, arguments, layouts and return values):

* ``flash_attention(q, k, v, causal=True, groups=5) -> out``      (AT:392-393)
* ``FlashAttention`` autograd.Function, backward returns
  ``(dq, dk, dv, None, None)``                                     (AT:360-389)
* ``get_kernel(kind, B, H, S, D, causal, groups)``, ``_kernels``,
  ``AUTOTUNE``, ``warmup``, ``flash_delta``                        (AT:94, :192-217, :326-357)
* ``AttnConfig``, ``RMSNorm``, ``Rotary``, ``rotate_half``, ``apply_rope``,
  ``Attention`` with backends ``"hip"`` (alias ``"tilelang"``), ``"sdpa"``,
  ``"flex"``, ``"math"``                                          (AT:396-518);
  with ``"hip"`` and bf16 activations the projection is one GEMM against
  wq | wk | wv followed by the QK-norm + RoPE kernel (``qknorm_rope``)
* harnesses ``reference``, ``rope_reference``, ``check_math``, ``check_gpu``,
  ``benchmark``, ``tune``                                          (AT:521-788)

Tensors: q ``[B,S,H,D]``, k/v ``[B,S,Hkv,D]`` bf16 with last-dim stride 1;
lse ``[B,H,S]`` fp32 in log2 units.  The kernels are the gfx950 HIP kernels of
``csrc/`` reached through the C ABI (``include/mm1_attn.h``); when that library
is not built every kernel entry point raises -- nothing here falls back to
another implementation.
"""
from __future__ import annotations

import math
import os
import sys
import time
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import tuned
from .harness import Report, compare, needs_gpu, time_cuda
from .harness import main as harness_main
from .wgrad import wgrad

DTYPE = torch.bfloat16
LOG2E = 1.4426950408889634

# ---------------------------------------------------------------------------
# gfx950 tilings (replace the TileLang search space and shared-memory model of
# AT:26-98).  The library compiles a fixed set per kernel and describes each
# (mm1_attn_tile_count / mm1_attn_tile_desc); index 0 is a kernel's default.
# A config is the parsed description: block_M, block_N, waves, stages,
# schedule -- for the backward both kernels' fields, prefixed dkdv_ / dq_.
LDS_PER_CU = 160 * 1024
WAVE = 64
TILE_KINDS = {"fwd": 0, "dkdv": 1, "dq": 2}    # MM1_TILES_FWD / _DKDV / _DQ


def _parse_tiles(desc: str) -> dict:
    out = {}
    for item in desc.split():
        key, val = item.split("=", 1)
        out[key] = int(val) if val.isdigit() else val
    return out


def tile_space(kind):
    """The tilings of one kernel ("fwd", "dkdv" or "dq") compiled into the library."""
    lib = _lib.load()
    code = TILE_KINDS[kind]
    return [_parse_tiles(lib.mm1_attn_tile_desc(code, i).decode())
            for i in range(lib.mm1_attn_tile_count(code))]


def fwd_configs(dim=128):
    """Forward search space (AT:66-71): the compiled forward tilings."""
    return tile_space("fwd") if dim == 128 else []


def bwd_configs(dim=128):
    """Backward search space (AT:74-79): every dK/dV tiling with every dQ tiling."""
    if dim != 128:
        return []
    return [{**{f"dkdv_{k}": v for k, v in a.items()}, **{f"dq_{k}": v for k, v in b.items()}}
            for a in tile_space("dkdv") for b in tile_space("dq")]


def tile_index(kind, config):
    """Library index of a forward config, (dK/dV, dQ) indices of a backward
    one, or None when the config names no compiled tiling."""
    config = dict(config)
    if kind == "fwd":
        space = tile_space("fwd")
        return space.index(config) if config in space else None
    # a backward record may also say how its two launches share the device
    if not isinstance(config.pop("overlap_dq", False), bool):
        return None
    parts = {}
    for sub in ("dkdv", "dq"):
        cut = len(sub) + 1
        mine = {k[cut:]: v for k, v in config.items() if k.startswith(sub + "_")}
        space = tile_space(sub)
        if mine not in space:
            return None
        parts[sub] = space.index(mine)
    if len(config) != sum(len(tile_space(sub)[i]) for sub, i in parts.items()):
        return None
    return parts["dkdv"], parts["dq"]


AUTOTUNE = True
# Index 0 of each kernel (the library's defaults), spelled out so that the
# module imports without the library; the CPU tests check they agree.
FWD_TILES = dict(block_M=256, block_N=64, waves=8, stages=2, schedule="pingpong")
BWD_TILES = dict(dkdv_block_M=128, dkdv_block_N=32, dkdv_waves=8, dkdv_stages=7,
                 dkdv_schedule="group",
                 dq_block_M=128, dq_block_N=64, dq_waves=4, dq_stages=2, dq_schedule="ring")


# ---------------------------------------------------------------------------
# Kernel handles
def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


# True: the backward runs its dQ launch on a second stream of the device,
# beside the dK/dV launch and the dK/dV partial sum on the caller's stream
# (results bitwise equal to the one-stream call).  A backward tile record's
# "overlap_dq" entry overrides this default per shape.  Measured in the full
# fwd+bwd step on gfx950 it gains 0.6-0.9% with the 256-row dQ tiling (one
# workgroup per CU) at B2 S8192 and B4 S4096 and loses 4-7% with the
# 128-row one (two per CU), so the default is one stream (mm1_attn_bwd_tiles:
# dK/dV, then dQ with the partial sum in its tail) and the shipped records
# switch it on where it was measured faster.
OVERLAP_DQ = False
_SIDE_STREAMS = {}


def _side_stream(device) -> "torch.cuda.Stream":
    stream = _SIDE_STREAMS.get(device)
    if stream is None:
        stream = _SIDE_STREAMS[device] = torch.cuda.Stream(device)   # default priority
    return stream


def _require(t: torch.Tensor, name: str, shape, dtype=DTYPE):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA (HIP) tensor, got device {t.device}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


class _Kernel:
    kind = ""

    def __init__(self, shape, config):
        batch, heads, seq_len, dim, causal, groups = shape
        if heads % groups:
            raise ValueError(f"heads={heads} is not a multiple of groups={groups}")
        self.shape = tuple(shape)
        self.config = dict(config)
        self.latency = None
        self.batch, self.heads, self.seq_len, self.dim = batch, heads, seq_len, dim
        self.causal, self.groups = bool(causal), groups
        self.kv_heads = heads // groups
        self.sm_scale = (1.0 / dim) ** 0.5
        _lib.load()
        self.tiles = tile_index(self.kind, self.config)
        if self.tiles is None:
            raise ValueError(f"{self.kind} config {self.config} is not a tiling compiled into "
                             f"the library")

    def __repr__(self):
        return f"<{type(self).__name__} shape={self.shape} config={self.config}>"


def _state(lib, B, S, H, Hkv, D, device):
    """A forward state buffer (mm1_attn_fwd_state_size bytes, uint8)."""
    return torch.empty(lib.mm1_attn_fwd_state_size(B, S, H, Hkv, D), dtype=torch.uint8, device=device)


class FwdKernel(_Kernel):
    """(q, k, v) -> (O, lse2); replaces flash_fwd (AT:110-190).  ``run``
    also returns the forward state the backward reads (the fp16 operand
    copies and the O residual, include/mm1_attn.h)."""
    kind = "fwd"

    def run(self, q, k, v):
        B, H, S, D, Hkv = self.batch, self.heads, self.seq_len, self.dim, self.kv_heads
        _require(q, "q", (B, S, H, D))
        _require(k, "k", (B, S, Hkv, D))
        _require(v, "v", (B, S, Hkv, D))
        lib = _lib.load()
        out = torch.empty_like(q)
        lse = torch.empty(B, H, S, dtype=torch.float32, device=q.device)
        state = _state(lib, B, S, H, Hkv, D, q.device)
        rc = lib.mm1_attn_fwd_tiles(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
                                    state.data_ptr(), state.numel(), B, S, H, Hkv, D, int(self.causal),
                                    self.sm_scale, self.tiles, _stream(q.device))
        _lib.check(rc, "mm1_attn_fwd_tiles")
        return out, lse, state

    def __call__(self, q, k, v):
        out, lse, _ = self.run(q, k, v)
        return out, lse


class BwdKernel(_Kernel):
    """(q, k, v, dO, lse, Delta, dQ, dK, dV) -> None, writing bf16 dQ/dK/dV in
    place.  Replaces flash_bwd (AT:242-323) + flash_unswizzle (AT:224-240) +
    the dk/dv casts (AT:389): the reference's buffers are fp32 accumulators,
    these are the final bf16 gradients.  Called this way it converts q, k, v
    itself (mm1_attn_prep) and uses the caller's Delta; ``run_saved`` is the
    backward of FlashAttention, from the forward's output and state (its
    Delta comes from 16 significant bits of O)."""
    kind = "bwd"

    def _check_grads(self, dq, dk, dv):
        B, H, S, D, Hkv = self.batch, self.heads, self.seq_len, self.dim, self.kv_heads
        _require(dq, "dq", (B, S, H, D))
        _require(dk, "dk", (B, S, Hkv, D))
        _require(dv, "dv", (B, S, Hkv, D))

    def __call__(self, q, k, v, grad_out, lse, delta, dq, dk, dv):
        B, H, S, D, Hkv = self.batch, self.heads, self.seq_len, self.dim, self.kv_heads
        _require(q, "q", (B, S, H, D))
        _require(k, "k", (B, S, Hkv, D))
        _require(v, "v", (B, S, Hkv, D))
        _require(grad_out, "grad_out", (B, S, H, D))
        _require(lse, "lse", (B, H, S), torch.float32)
        _require(delta, "delta", (B, H, S), torch.float32)
        self._check_grads(dq, dk, dv)
        lib = _lib.load()
        state = _state(lib, B, S, H, Hkv, D, q.device)
        rc = lib.mm1_attn_prep(q.data_ptr(), k.data_ptr(), v.data_ptr(), state.data_ptr(), state.numel(),
                               B, S, H, Hkv, D, _stream(q.device))
        _lib.check(rc, "mm1_attn_prep")
        ws = self._workspace(lib, q.device)
        rc = lib.mm1_attn_bwd_prep_delta(grad_out.data_ptr(), delta.data_ptr(), lse.data_ptr(), state.data_ptr(),
                                         state.numel(), ws.data_ptr(), ws.numel(), B, S, H, Hkv, D, self.sm_scale,
                                         _stream(q.device))
        _lib.check(rc, "mm1_attn_bwd_prep_delta")
        self._stages(lib, state, ws, dq, dk, dv)

    def run_saved(self, out, grad_out, lse, state, dq, dk, dv):
        """dQ, dK, dV from the forward's (out, lse, state) and dO."""
        B, H, S, D, Hkv = self.batch, self.heads, self.seq_len, self.dim, self.kv_heads
        _require(out, "out", (B, S, H, D))
        _require(grad_out, "grad_out", (B, S, H, D))
        _require(lse, "lse", (B, H, S), torch.float32)
        self._check_grads(dq, dk, dv)
        lib = _lib.load()
        ws = self._workspace(lib, out.device)
        rc = lib.mm1_attn_bwd_prep(out.data_ptr(), grad_out.data_ptr(), lse.data_ptr(), state.data_ptr(),
                                   state.numel(), ws.data_ptr(), ws.numel(), B, S, H, Hkv, D, self.sm_scale,
                                   _stream(out.device))
        _lib.check(rc, "mm1_attn_bwd_prep")
        self._stages(lib, state, ws, dq, dk, dv)

    def _workspace(self, lib, device):
        B, H, S, D, Hkv = self.batch, self.heads, self.seq_len, self.dim, self.kv_heads
        return torch.empty(lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, D), dtype=torch.uint8, device=device)

    def _stages(self, lib, state, ws, dq, dk, dv):
        B, H, S, D, Hkv = self.batch, self.heads, self.seq_len, self.dim, self.kv_heads
        shape = (B, S, H, Hkv, D, int(self.causal), self.sm_scale)
        dkdv_tiles, dq_tiles = self.tiles
        st, wsp = (state.data_ptr(), state.numel()), (ws.data_ptr(), ws.numel())
        if not self.config.get("overlap_dq", OVERLAP_DQ):
            rc = lib.mm1_attn_bwd_dkdv_tiles(*st, dk.data_ptr(), dv.data_ptr(), *wsp, *shape, dkdv_tiles,
                                             _stream(dq.device))
            _lib.check(rc, "mm1_attn_bwd_dkdv_tiles")
            rc = lib.mm1_attn_bwd_dq_reduce_tiles(*st, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), *wsp, *shape,
                                                  dkdv_tiles, dq_tiles, _stream(dq.device))
            _lib.check(rc, "mm1_attn_bwd_dq_reduce_tiles")
            return
        main = torch.cuda.current_stream(dq.device)
        side = _side_stream(dq.device)
        fork = torch.cuda.Event()
        fork.record(main)
        side.wait_event(fork)
        try:
            rc = lib.mm1_attn_bwd_dq_tiles(*st, dq.data_ptr(), *wsp, *shape, dq_tiles, side.cuda_stream)
            _lib.check(rc, "mm1_attn_bwd_dq_tiles")
            rc = lib.mm1_attn_bwd_dkdv_tiles(*st, dk.data_ptr(), dv.data_ptr(), *wsp, *shape, dkdv_tiles,
                                             main.cuda_stream)
            _lib.check(rc, "mm1_attn_bwd_dkdv_tiles")
            rc = lib.mm1_attn_bwd_dkdv_reduce_tiles(*wsp, dk.data_ptr(), dv.data_ptr(), B, S, H, Hkv, D,
                                                    int(self.causal), dkdv_tiles, main.cuda_stream)
            _lib.check(rc, "mm1_attn_bwd_dkdv_reduce_tiles")
        finally:
            # the caller's stream waits for the side stream even when a launch
            # was refused, so no buffer is reused under a running dQ kernel
            join = torch.cuda.Event()
            join.record(side)
            main.wait_event(join)


class DeltaKernel:
    """(O, dO) -> Delta [B,H,S] fp32; replaces flash_delta (AT:192-217)."""

    def __init__(self, batch, heads, seq_len, dim):
        self.shape = (batch, heads, seq_len, dim)
        _lib.load()

    def __call__(self, out, grad_out):
        B, H, S, D = self.shape
        _require(out, "O", (B, S, H, D))
        _require(grad_out, "dO", (B, S, H, D))
        delta = torch.empty(B, H, S, dtype=torch.float32, device=out.device)
        rc = _lib.load().mm1_attn_delta(out.data_ptr(), grad_out.data_ptr(), delta.data_ptr(),
                                        B, S, H, D, _stream(out.device))
        _lib.check(rc, "mm1_attn_delta")
        return delta


_kernels: dict = {}


def flash_delta(batch, heads, seq_len, dim):
    return DeltaKernel(batch, heads, seq_len, dim)


def _median_ms(fn, device, budget_ms=60.0, max_reps=25):
    """Median duration of fn() on the current stream of `device` (HIP events)."""
    stream = torch.cuda.current_stream(device)
    fn()
    torch.cuda.synchronize(device)
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize(device)
    first = (time.perf_counter() - t0) * 1e3
    reps = int(min(max_reps, max(3, budget_ms / max(first, 1e-3))))
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
    for start, end in events:
        start.record(stream)
        fn()
        end.record(stream)
    torch.cuda.synchronize(device)
    times = sorted(start.elapsed_time(end) for start, end in events)
    return times[len(times) // 2]


def autotune(kind, shape, device=None, verbose=False):
    """Time every compiled tiling of `kind` at `shape` on synthetic inputs and
    return (best config, its median ms, [(ms, config), ...]).  The search the
    reference's TileLang autotuner runs for a miss (AT:337-343), over this
    library's tilings; inputs are seeded so that runs are repeatable."""
    if kind not in ("fwd", "bwd"):
        raise ValueError(f"unknown kernel kind {kind!r}")
    batch, heads, seq_len, dim, causal, groups = shape
    device = torch.device(device or f"cuda:{torch.cuda.current_device()}")
    gen = torch.Generator(device=device).manual_seed(0)
    kv_heads = heads // groups

    def rand(*dims):
        return torch.randn(*dims, device=device, dtype=DTYPE, generator=gen)

    q, k, v = rand(batch, seq_len, heads, dim), rand(batch, seq_len, kv_heads, dim), \
        rand(batch, seq_len, kv_heads, dim)
    results = []
    # bring the clocks up before the first timing: the first tiling timed
    # from an idle GPU otherwise reads a few percent slow
    warm = FwdKernel(shape, FWD_TILES)
    t_end = time.perf_counter() + 0.2
    while time.perf_counter() < t_end:
        warm(q, k, v)
        torch.cuda.synchronize(device)
    if kind == "fwd":
        for config in fwd_configs(dim):
            handle = FwdKernel(shape, config)
            results.append((_median_ms(lambda: handle(q, k, v), device), config))
    else:
        out, lse, state = warm.run(q, k, v)
        grad_out = rand(batch, seq_len, heads, dim)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        for config in bwd_configs(dim):
            handle = BwdKernel(shape, config)
            results.append((_median_ms(lambda: handle.run_saved(out, grad_out, lse, state, dq, dk, dv),
                                       device), config))
    if verbose:
        for ms, config in results:
            print(f"    {ms:8.3f} ms  {' '.join(f'{k}={v}' for k, v in config.items())}")
    best_ms, best = min(results, key=lambda r: r[0])
    return best, best_ms, results


def get_kernel(kind, *shape):
    """Per-shape kernel handle, cached in ``_kernels`` under
    ``(kind, shape, AUTOTUNE)`` (AT:329-346).  Lookup order as in the
    reference: the tile record for this device and shape, then a timed search
    over the compiled tilings when AUTOTUNE is set and a GPU is present (its
    winner is recorded), else the defaults.  A record naming a tiling this
    build does not have is ignored."""
    if kind not in ("fwd", "bwd"):
        raise ValueError(f"unknown kernel kind {kind!r}")
    key = (kind, tuple(shape), AUTOTUNE)
    if key not in _kernels:
        cls = FwdKernel if kind == "fwd" else BwdKernel
        name = f"attention_{kind}"
        kernel = None
        remembered = tuned.lookup(name, shape)
        if remembered is not None and tile_index(kind, remembered) is not None:
            kernel = cls(shape, remembered)
        elif AUTOTUNE and torch.cuda.is_available():
            cls(shape, FWD_TILES if kind == "fwd" else BWD_TILES)   # shape check first
            config, latency, _ = autotune(kind, shape)
            kernel = cls(shape, config)
            kernel.latency = latency
            tuned.record(name, shape, tuned.config_of(kernel))
        else:
            kernel = cls(shape, FWD_TILES if kind == "fwd" else BWD_TILES)
        _kernels[key] = kernel
    return _kernels[key]


def warmup(batch, seq_len, cfg=None, causal=True):
    """Create both kernel handles up front (AT:349-357)."""
    cfg = cfg or AttnConfig()
    shape = (batch, cfg.n_heads, seq_len, cfg.head_dim, causal, cfg.groups)
    get_kernel("fwd", *shape)
    get_kernel("bwd", *shape)


# ---------------------------------------------------------------------------
# Autograd op
class FlashAttention(torch.autograd.Function):
    """Same signature and returns as AT:360-389."""

    @staticmethod
    def forward(ctx, q, k, v, causal, groups):
        batch, seq_len, heads, dim = q.shape
        if k.shape[-2] * groups != heads:
            raise ValueError(f"groups={groups} does not match heads={heads}, "
                             f"kv_heads={k.shape[-2]}")
        out, lse, state = get_kernel("fwd", batch, heads, seq_len, dim, causal, groups).run(q, k, v)
        # the backward reads the fp16 copies of q, k, v in `state`, not q, k, v
        ctx.save_for_backward(out, lse, state)
        ctx.causal, ctx.groups = causal, groups
        ctx.kv_shape, ctx.kv_dtype = k.shape, k.dtype
        return out

    @staticmethod
    def backward(ctx, grad_out):
        out, lse, state = ctx.saved_tensors
        batch, seq_len, heads, dim = out.shape
        kv_heads = ctx.kv_shape[-2]
        groups = heads // kv_heads
        grad_out = grad_out if grad_out.is_contiguous() else grad_out.contiguous()
        if grad_out.dtype != out.dtype:
            grad_out = grad_out.to(out.dtype)
        dq = torch.empty_like(out)
        dk = torch.empty(ctx.kv_shape, dtype=ctx.kv_dtype, device=out.device)
        dv = torch.empty(ctx.kv_shape, dtype=ctx.kv_dtype, device=out.device)
        get_kernel("bwd", batch, heads, seq_len, dim, ctx.causal, groups).run_saved(
            out, grad_out, lse, state, dq, dk, dv)
        return dq, dk, dv, None, None


def flash_attention(q, k, v, causal=True, groups=5):
    return FlashAttention.apply(q, k, v, causal, groups)


def flash_attention_with_lse(q, k, v, causal=True, groups=5):
    """Forward only, returning (O, lse2) -- the kernel's two outputs."""
    batch, seq_len, heads, dim = q.shape
    return get_kernel("fwd", batch, heads, seq_len, dim, causal, groups)(q, k, v)


# ---------------------------------------------------------------------------
# Sublayer (AT:396-518)
@dataclass
class AttnConfig:
    d_model: int = 1280
    n_heads: int = 10
    n_kv_heads: int = 2
    head_dim: int = 128
    rope_theta: float = 10_000.0
    max_seq_len: int = 8192
    qk_norm: bool = True
    norm_eps: float = 1e-5
    backend: str = "hip"

    def __post_init__(self):
        assert self.n_heads % self.n_kv_heads == 0
        assert self.n_heads * self.head_dim == self.d_model
        assert self.head_dim in (64, 128)

    @property
    def groups(self):
        return self.n_heads // self.n_kv_heads


class RMSNorm(nn.Module):
    """Per-head QK norm (AT:418-428): x / rms(x) * weight over the last axis,
    evaluated in fp32 and returned in x's dtype.  The fp32 products happen in
    the reference's order (normalise, then weight), which the bf16 kernel
    path (mm1_qknorm_rope_fwd) reproduces bit for bit."""

    def __init__(self, dim, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        wide = x.float()
        inv_rms = wide.square().mean(dim=-1, keepdim=True).add(self.eps).rsqrt()
        return (wide * inv_rms * self.weight.float()).to(x.dtype)


class Rotary(nn.Module):
    """Rotate-half RoPE tables (AT:431-449): for position p and frequency
    index i < D/2, the angle p * theta^(-2i/D) appears in columns i and
    i + D/2 of the fp32 [max_seq_len, D] cos and sin buffers."""

    def __init__(self, head_dim, max_seq_len, theta):
        super().__init__()
        self.head_dim = head_dim
        self.max_seq_len = max_seq_len
        self.build(theta)

    def _tables(self, theta, device=None):
        exponent = torch.arange(0, self.head_dim, 2, device=device).float() / self.head_dim
        inv_freq = (theta ** exponent).reciprocal()
        angle = torch.arange(self.max_seq_len, device=device).float()[:, None] * inv_freq[None, :]
        angle = angle.repeat(1, 2)                      # the same angle for both halves
        return angle.cos(), angle.sin()

    def build(self, theta):
        self.theta = theta
        cos, sin = self._tables(theta)
        self.register_buffer("cos", cos, persistent=False)
        self.register_buffer("sin", sin, persistent=False)

    def set_theta(self, theta):
        """New base frequency, tables rebuilt where the current ones live."""
        self.theta = theta
        self.cos, self.sin = (t.to(self.cos.device) for t in self._tables(theta))


def rotate_half(x):
    """(a, b) -> (-b, a) over the two halves of the last axis."""
    lo, hi = x.chunk(2, dim=-1)
    return torch.cat((hi.neg(), lo), dim=-1)


def apply_rope(x, cos, sin):
    """x [B,S,H,D] rotated by the first S rows of the tables, which are cast to
    x's dtype first (AT:457-461), so that a bf16 x is rotated in bf16 steps."""
    rows = x.shape[1]
    c, s = (t[:rows].to(x.dtype).unsqueeze(1) for t in (cos, sin))
    return x * c + rotate_half(x) * s


_HIP_BACKENDS = ("hip", "tilelang")


# Token chunks of the projections' weight-gradient GEMMs (wgrad.py): 8
# measured fastest for wq|wk|wv and wo at 16,384 tokens.
PROJ_DW_CHUNKS = 8


class BF16Linear(torch.autograd.Function):
    """y = x W^T of the sublayer's projections under bf16 autocast, with the
    weight gradient in the GEMM form hipBLASLt runs fastest on gfx950:
      dX = dY W, as autograd computes it;
      dW = sum over PROJ_DW_CHUNKS token chunks of dY_c^T X_c, each a GEMM with
           fp32 outputs, summed in fp32 (the reference's autocast graph rounds
           the one bf16 GEMM's dW to bf16 before its fp32 cast, AT:470-472,
           :518; this dW is the same sum without that rounding).
    x may be fp32 or bf16 (cast here, as autocast would); w is the fp32
    parameter (cast here; its gradient is returned in fp32).  The forward is
    the same F.linear on the same bf16 operands as the module's."""

    @staticmethod
    def forward(ctx, x, w):
        xb, wb = x.to(DTYPE), w.to(DTYPE)
        ctx.save_for_backward(xb, wb)
        ctx.x_dtype, ctx.w_dtype = x.dtype, w.dtype
        return F.linear(xb, wb)

    @staticmethod
    def backward(ctx, dy):
        xb, wb = ctx.saved_tensors
        n, k = wb.shape
        dy2 = dy.reshape(-1, n).to(DTYPE)
        x2 = xb.reshape(-1, k)
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = (dy2 @ wb).reshape(*dy.shape[:-1], k).to(ctx.x_dtype)
        if ctx.needs_input_grad[1]:
            dw = wgrad(dy2, x2, PROJ_DW_CHUNKS).to(ctx.w_dtype)
        return dx, dw


def _autocast_bf16() -> bool:
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == DTYPE


def _bf16_linear_applies(x) -> bool:
    """The hip backend's projections run through BF16Linear where autocast
    would run them in bf16 on the GPU."""
    return x.is_cuda and _autocast_bf16()


def _skip_attn_out_cast() -> bool:
    """Under bf16 autocast wo casts its input back to bf16, so the reference's
    cast of the attention output to x.dtype (AT:494) is a bf16 -> fp32 -> bf16
    round trip, exact both ways (its gradient too): the hip backend skips it."""
    return _autocast_bf16()


class QKNormRope(torch.autograd.Function):
    """QK-RMSNorm + RoPE of the fused projection on the gfx950 kernels
    (mm1_qknorm_rope_fwd / _bwd): qkv [B, S, (H + 2*Hkv) * D] bf16 ->
    (q [B,S,H,D], k [B,S,Hkv,D], v [B,S,Hkv,D]) bf16, the numerics of
    q_norm / k_norm + apply_rope on the wq / wk / wv outputs (AT:483-487).
    wq, wk: the RMSNorm weights [D], or None without QK-norm."""

    @staticmethod
    def forward(ctx, qkv, wq, wk, cos, sin, heads, kv_heads, eps):
        batch, seq_len, width = qkv.shape
        dim = width // (heads + 2 * kv_heads)
        if dim * (heads + 2 * kv_heads) != width:
            raise ValueError(f"qkv width {width} is not (heads + 2*kv_heads) * head_dim")
        _require(qkv, "qkv", (batch, seq_len, width))
        for t, name in ((cos, "cos"), (sin, "sin")):
            _require(t, name, (t.shape[0], dim), torch.float32)
        wqf = None if wq is None else wq.detach().float().contiguous()
        wkf = None if wk is None else wk.detach().float().contiguous()
        q = torch.empty(batch, seq_len, heads, dim, dtype=DTYPE, device=qkv.device)
        k = torch.empty(batch, seq_len, kv_heads, dim, dtype=DTYPE, device=qkv.device)
        v = torch.empty_like(k)
        ptr = lambda t: None if t is None else t.data_ptr()
        rc = _lib.load().mm1_qknorm_rope_fwd(
            qkv.data_ptr(), ptr(wqf), ptr(wkf), cos.data_ptr(), sin.data_ptr(), q.data_ptr(),
            k.data_ptr(), v.data_ptr(), batch, seq_len, heads, kv_heads, dim, cos.shape[0], eps,
            _stream(qkv.device))
        _lib.check(rc, "mm1_qknorm_rope_fwd")
        ctx.save_for_backward(qkv, wqf, wkf, cos, sin)
        ctx.meta = (heads, kv_heads, eps, None if wq is None else wq.dtype,
                    None if wk is None else wk.dtype)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        qkv, wqf, wkf, cos, sin = ctx.saved_tensors
        heads, kv_heads, eps, wq_dtype, wk_dtype = ctx.meta
        batch, seq_len, width = qkv.shape
        dim = width // (heads + 2 * kv_heads)
        shapes = ((batch, seq_len, heads, dim), (batch, seq_len, kv_heads, dim), (batch, seq_len, kv_heads, dim))
        grads = []
        for g, shp in zip((dq, dk, dv), shapes):
            g = torch.zeros(shp, dtype=DTYPE, device=qkv.device) if g is None else g
            grads.append(g.to(DTYPE).contiguous())
        dqkv = torch.empty_like(qkv)
        lib = _lib.load()
        norm = wqf is not None
        dwq = torch.empty(dim, dtype=torch.float32, device=qkv.device) if norm else None
        dwk = torch.empty_like(dwq) if norm else None
        ws_bytes = lib.mm1_qknorm_rope_bwd_workspace_size()
        ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=qkv.device)
        ptr = lambda t: None if t is None else t.data_ptr()
        rc = lib.mm1_qknorm_rope_bwd(
            qkv.data_ptr(), ptr(wqf), ptr(wkf), cos.data_ptr(), sin.data_ptr(), grads[0].data_ptr(),
            grads[1].data_ptr(), grads[2].data_ptr(), dqkv.data_ptr(), ptr(dwq), ptr(dwk),
            ws.data_ptr(), ws_bytes, batch, seq_len, heads, kv_heads, dim, cos.shape[0], eps,
            _stream(qkv.device))
        _lib.check(rc, "mm1_qknorm_rope_bwd")
        if norm:
            dwq, dwk = dwq.to(wq_dtype), dwk.to(wk_dtype)
        return dqkv, dwq, dwk, None, None, None, None, None


def qknorm_rope(qkv, wq, wk, cos, sin, heads, kv_heads, eps=1e-5):
    """The attention kernel's q, k, v from the fused projection (see QKNormRope)."""
    return QKNormRope.apply(qkv, wq, wk, cos, sin, heads, kv_heads, eps)


class Attention(nn.Module):
    """GQA attention sublayer (AT:464-518): projections wq / wk / wv to 10 query
    and 2 KV heads of 128, QK-RMSNorm, RoPE, causal attention, projection wo
    back to d_model; no biases.  ``backend`` "hip" (also accepted under the
    reference's name "tilelang") runs the gfx950 kernels; "sdpa", "flex" and
    "math" run torch's library attention, flex attention, and the fp32 math."""

    def __init__(self, cfg: AttnConfig, rope: Rotary):
        super().__init__()
        self.cfg = cfg
        self.rope = rope
        q_width, kv_width = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim
        linear = lambda n_in, n_out: nn.Linear(n_in, n_out, bias=False)
        self.wq, self.wk, self.wv = (linear(cfg.d_model, w) for w in (q_width, kv_width, kv_width))
        self.wo = linear(q_width, cfg.d_model)
        norm = (lambda: RMSNorm(cfg.head_dim, cfg.norm_eps)) if cfg.qk_norm else nn.Identity
        self.q_norm, self.k_norm = norm(), norm()
        self.scale = 1.0 / math.sqrt(cfg.head_dim)

    def _heads(self, t, n):
        return t.unflatten(-1, (n, self.cfg.head_dim))

    def project(self, x):
        """QKV projections, QK-norm and RoPE: the inputs of the attention kernel."""
        cfg, rope = self.cfg, self.rope
        q = apply_rope(self.q_norm(self._heads(self.wq(x), cfg.n_heads)), rope.cos, rope.sin)
        k = apply_rope(self.k_norm(self._heads(self.wk(x), cfg.n_kv_heads)), rope.cos, rope.sin)
        return q, k, self._heads(self.wv(x), cfg.n_kv_heads)

    def project_fused(self, x):
        """The same q, k, v from one GEMM against wq | wk | wv and the QK-norm +
        RoPE kernel; None when the projection is not bf16 (fp32 activations
        outside autocast keep the reference's fp32 norm and rotation)."""
        cfg = self.cfg
        w = torch.cat((self.wq.weight, self.wk.weight, self.wv.weight), dim=0)
        qkv = BF16Linear.apply(x, w) if _bf16_linear_applies(x) else F.linear(x, w)
        if qkv.dtype != DTYPE or not qkv.is_cuda or cfg.head_dim != 128:
            return None
        qn = self.q_norm.weight if cfg.qk_norm else None
        kn = self.k_norm.weight if cfg.qk_norm else None
        return qknorm_rope(qkv.contiguous(), qn, kn, self.rope.cos, self.rope.sin,
                           cfg.n_heads, cfg.n_kv_heads, cfg.norm_eps)

    # the non-kernel backends, on BSHD q / k / v; each returns BSHD output
    def _attend_sdpa(self, q, k, v, x):
        to_bhsd = lambda t: t.transpose(1, 2)
        out = F.scaled_dot_product_attention(to_bhsd(q), to_bhsd(k), to_bhsd(v), is_causal=True,
                                             scale=self.scale, enable_gqa=True)
        return out.transpose(1, 2)

    def _attend_flex(self, q, k, v, x):
        from torch.nn.attention.flex_attention import create_block_mask, flex_attention
        n = q.shape[1]
        causal = create_block_mask(lambda b, h, qi, ki: ki <= qi, None, None, n, n, device=x.device)
        out = flex_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                             block_mask=causal, scale=self.scale, enable_gqa=True)
        return out.transpose(1, 2)

    def _attend_math(self, q, k, v, x):
        # fp32 scores scaled by multiplication, as the reference's math branch
        return _attention_fp32(q, k, v, True, self.cfg.groups, self.scale).to(x.dtype)

    def forward(self, x, backend=None):
        cfg = self.cfg
        backend = backend or cfg.backend
        hip = backend in _HIP_BACKENDS
        fused = self.project_fused(x) if hip and x.is_cuda else None
        q, k, v = fused if fused is not None else self.project(x)
        if hip:
            out = flash_attention(*(t.to(DTYPE).contiguous() for t in (q, k, v)), True, cfg.groups)
            if not _skip_attn_out_cast():
                out = out.to(x.dtype)
        else:
            attend = {"sdpa": self._attend_sdpa, "flex": self._attend_flex, "math": self._attend_math}
            if backend not in attend:
                raise ValueError(f"unknown backend {backend!r}")
            out = attend[backend](q, k, v, x)
        out = out.flatten(2)
        if hip and _bf16_linear_applies(out):
            return BF16Linear.apply(out, self.wo.weight)
        return self.wo(out)


# ---------------------------------------------------------------------------
# Reference math and harnesses (AT:521-788)
def _attention_fp32(q, k, v, causal, groups, scale=None):
    """softmax(q k^T * scale [causal]) v in fp32 on BSHD tensors, KV head
    h // groups for query head h; fp32 BSHD result.  `scale` None divides the
    scores by sqrt(D) (the form of AT:525), a number multiplies them."""
    n, dim = q.shape[1], q.shape[-1]
    expand = lambda t: t.float().repeat_interleave(groups, dim=2).transpose(1, 2)   # B H S D
    qh, kh, vh = q.float().transpose(1, 2), expand(k), expand(v)
    s = torch.matmul(qh, kh.transpose(-1, -2).contiguous())
    s = s / math.sqrt(dim) if scale is None else s * scale
    if causal:
        future = torch.ones(n, n, dtype=torch.bool, device=q.device).triu(1)
        s = s.masked_fill(future, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vh.contiguous()).transpose(1, 2)


def reference(q, k, v, causal, groups):
    """The fp32 attention math the kernels answer to, returned in q.dtype
    (AT:521-530)."""
    return _attention_fp32(q, k, v, causal, groups).to(q.dtype)


def rope_reference(x, theta):
    """RoPE as a complex rotation: the pair (x_i, x_{i+D/2}) is the complex
    number x_i + j x_{i+D/2}, multiplied by exp(j p theta^(-2i/D)) at position
    p (AT:533-541) -- an independent form of apply_rope's rotate-half."""
    n, dim = x.shape[1], x.shape[-1]
    half = dim // 2
    freq = torch.tensor(float(theta), dtype=torch.float64) ** (-2.0 * torch.arange(half, dtype=torch.float64) / dim)
    turn = torch.polar(torch.ones(n, half, dtype=torch.float64),
                       torch.arange(n, dtype=torch.float64)[:, None] * freq)
    z = torch.complex(x[..., :half].double(), x[..., half:].double()) * turn[None, :, None, :]
    return torch.cat((z.real, z.imag), dim=-1).to(x.dtype)


def _math_checks(report: Report):
    cfg = AttnConfig(backend="math")
    gen = torch.Generator().manual_seed(0)
    randn = lambda *shape: torch.randn(*shape, generator=gen)

    report.section("gfx950 tilings")
    try:
        spaces = {"fwd": fwd_configs(), "bwd": bwd_configs()}
    except _lib.LibraryMissing as exc:
        report.note(f"library not built ({exc}); tiling checks skipped")
    else:
        report.note(f"{len(spaces['fwd'])} forward and {len(spaces['bwd'])} backward tilings")
        report.expect("defaults are the library's index 0",
                      spaces["fwd"][0] == FWD_TILES and spaces["bwd"][0] == BWD_TILES)
        report.expect("every tiling maps back to its own index",
                      [tile_index("fwd", c) for c in spaces["fwd"]] == list(range(len(spaces["fwd"])))
                      and len({tile_index("bwd", c) for c in spaces["bwd"]}) == len(spaces["bwd"]))
        report.expect("every workgroup fits 1024 threads",
                      max(c["waves"] for c in spaces["fwd"]) * WAVE <= 1024)

    report.section("RoPE")
    rope = Rotary(128, 96, 10_000.0)
    x = randn(2, 96, 3, 128)
    rotated = apply_rope(x, rope.cos, rope.sin)
    err = (rotated - rope_reference(x, 10_000.0)).abs().max().item()
    report.expect("rotate-half equals the complex rotation", err < 1e-4, err)
    err = (rotated.norm(dim=-1) - x.norm(dim=-1)).abs().max().item()
    report.expect("rotation keeps each head vector's norm", err < 1e-4, err)
    # q.k after rotation depends only on the distance between the positions
    a, b = randn(128), randn(128)
    ra = apply_rope(a.expand(1, 96, 1, 128).contiguous(), rope.cos, rope.sin)[0, :, 0]
    rb = apply_rope(b.expand(1, 96, 1, 128).contiguous(), rope.cos, rope.sin)[0, :, 0]
    spread = max((torch.stack([ra[p] @ rb[p + d] for p in range(0, 96 - d, 7)]).std().item()
                  for d in (0, 5, 40)))
    report.expect("scores depend on relative position only", spread < 1e-3, spread)
    rope.set_theta(500_000.0)
    fresh = Rotary(128, 96, 500_000.0)
    report.expect("set_theta rebuilds the tables", rope.theta == 500_000.0 and torch.equal(rope.cos, fresh.cos))

    report.section("QK RMSNorm")
    norm = RMSNorm(16)
    y = norm(randn(5, 16) * 7)
    rms = y.square().mean(-1).sqrt()
    report.expect("unit root-mean-square rows", (rms - 1).abs().max() < 1e-3, (rms - 1).abs().max().item())
    z = randn(5, 16)
    drift = (norm(z * 3.5) - norm(z)).abs().max().item()     # up to eps / (2 mean(z^2)) relative
    report.expect("invariant to scaling its input", drift < 1e-4, drift)

    report.section("sublayer")
    layer = Attention(cfg, Rotary(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta))
    count = sum(p.numel() for p in layer.parameters())
    report.expect("parameter count 3,932,416", count == 3_932_416, count)
    report.expect("projections carry no bias", all(m.bias is None for m in (layer.wq, layer.wk, layer.wv, layer.wo)))
    x = randn(2, 40, cfg.d_model)
    y = layer(x, backend="math")
    report.expect("output keeps the input's shape", tuple(y.shape) == tuple(x.shape))
    gap = (y - layer(x, backend="sdpa")).abs().max().item()
    report.expect("math and sdpa backends agree", gap < 2e-3, gap)
    later = x.clone()
    later[:, 30:] = randn(2, 10, cfg.d_model) * 5
    leak = (layer(later, backend="math")[:, :30] - y[:, :30]).abs().max().item()
    report.expect("positions never see later positions", leak < 1e-5, leak)
    x.requires_grad_(True)
    layer(x, backend="math").square().mean().backward()
    grads = [x.grad] + [p.grad for p in layer.parameters()]
    report.expect("gradients reach the input and every parameter, finite",
                  all(g is not None and bool(torch.isfinite(g).all()) for g in grads))

    report.section("constants")
    report.expect("softmax scale (1/D)^0.5 is 1/sqrt(D)", math.isclose((1.0 / 128) ** 0.5, 1 / math.sqrt(128),
                                                                        rel_tol=1e-15))
    report.expect("LOG2E is log2(e)", math.isclose(LOG2E, math.log2(math.e), rel_tol=1e-15))


def check_math(quiet=False) -> Report:
    """CPU checks of the module's host side and math (the reference's
    check(), AT:544-630): tilings, RoPE, QK-norm, the sublayer, constants."""
    report = Report("attention math", quiet=quiet)
    torch.manual_seed(0)
    _math_checks(report)
    return report.finish()


def check_gpu(seq_len=512, batch=2, quiet=False) -> Report:
    """The autograd op against the fp32 reference math on the GPU, causal and
    full, plus a repeat of the backward (the reference's check_gpu,
    AT:633-678, whose gate is max|d| / max|ref| < 2e-2; relative L2 is
    reported beside it).  Inputs ~ N(0,1) from seed 0."""
    report = Report("attention gpu", quiet=quiet)
    if not needs_gpu("check_gpu"):
        return report
    dev = torch.device("cuda")
    report.note(f"{torch.cuda.get_device_name(dev)} ({torch.cuda.get_device_properties(dev).gcnArchName})")
    cfg = AttnConfig()
    gen = torch.Generator(device=dev).manual_seed(0)
    leaf = lambda heads: torch.randn(batch, seq_len, heads, cfg.head_dim, device=dev, dtype=DTYPE,
                                     generator=gen).requires_grad_(True)
    q, k, v = leaf(cfg.n_heads), leaf(cfg.n_kv_heads), leaf(cfg.n_kv_heads)
    d_out = torch.randn(q.shape, device=dev, dtype=DTYPE, generator=gen)
    for causal in (True, False):
        report.section(f"{'causal' if causal else 'full'} B{batch} S{seq_len}")
        got = torch.autograd.grad(flash_attention(q, k, v, causal, cfg.groups), (q, k, v), d_out,
                                  create_graph=False)
        out = flash_attention(q, k, v, causal, cfg.groups)
        exact = [t.detach().float().requires_grad_(True) for t in (q, k, v)]
        want_out = _attention_fp32(*exact, causal, cfg.groups)
        want = torch.autograd.grad(want_out, exact, d_out.float())
        for name, a, b in zip(("O", "dQ", "dK", "dV"), (out,) + tuple(got), (want_out,) + tuple(want)):
            e = compare(a, b)
            report.expect(f"{name}: max|d|/max|ref| < 2e-2", e["finite"] and e["max_rel"] < 2e-2, e["max_rel"])
            report.note(f"{name}: max-abs {e['max_abs']:.3e}, rel-L2 {e['rel_l2']:.3e}")
    report.section("determinism")
    first, second = (torch.autograd.grad(flash_attention(q, k, v, True, cfg.groups), (q, k, v), d_out)
                     for _ in range(2))
    report.expect("two backward passes are bitwise equal", all(torch.equal(a, b) for a, b in zip(first, second)))
    return report.finish()


def attention_flops(batch, seq_len, heads=10, dim=128, causal=True):
    """Algorithmic FLOPs: fwd 2 GEMMs, bwd 5 GEMMs of 2*S*S*D each, halved when
    causal.  Returns (fwd, bwd)."""
    half = 0.5 if causal else 1.0
    gemm = 2.0 * batch * heads * seq_len * seq_len * dim * half
    return 2 * gemm, 5 * gemm


def benchmark(batch=8, seq_len=2048, iters=30, quiet=False) -> dict:
    """fwd+bwd of the HIP autograd op and of torch SDPA, HIP-event timed
    (the reference's benchmark, AT:681-748).  TFLOP/s counts 7*B*H*S^2*D for
    causal fwd+bwd; the reference's own 5*B*H*S^2*D count (AT:690) is shown
    beside it.  Returns {name: ms}."""
    if not needs_gpu("benchmark"):
        return {}
    cfg = AttnConfig()
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    leaf = lambda heads: torch.randn(batch, seq_len, heads, cfg.head_dim, device=dev, dtype=DTYPE,
                                     generator=gen).requires_grad_(True)
    q, k, v = leaf(cfg.n_heads), leaf(cfg.n_kv_heads), leaf(cfg.n_kv_heads)
    d_out = torch.randn(q.shape, device=dev, dtype=DTYPE, generator=gen)
    steps = {
        "hip": lambda: torch.autograd.grad(flash_attention(q, k, v, True, cfg.groups), (q, k, v), d_out),
        "sdpa": lambda: torch.autograd.grad(
            F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                           is_causal=True, enable_gqa=True), (q, k, v), d_out.transpose(1, 2)),
    }
    fwd, bwd = attention_flops(batch, seq_len, cfg.n_heads, cfg.head_dim)
    ms = {}
    for name, step in steps.items():
        try:
            ms[name] = time_cuda(step, warmup=10, iters=iters)
        except RuntimeError as exc:   # a torch attention backend may be missing from a build
            print(f"{name}: unavailable ({exc})")
    if not quiet:
        for name, t in sorted(ms.items(), key=lambda kv: kv[1]):
            print(f"  {name:6s} {t:8.3f} ms  {(fwd + bwd) / t * 1e-9:7.1f} TFLOP/s"
                  f"  (reference count {(fwd + bwd) * 5 / 7 / t * 1e-9:7.1f})")
    return ms


def tune(batch=8, seq_len=2048):
    """Time the compiled tilings at one shape and record the winners (the
    reference's tune(), AT:751-769); ``python -m mimansm1_v1_amd.tune`` does
    every training shape."""
    try:
        spaces = {"fwd": fwd_configs(), "bwd": bwd_configs()}
    except _lib.LibraryMissing as exc:
        print(f"library not built: {exc}")
        return None
    for kind, space in spaces.items():
        print(f"{kind}: {len(space)} tilings")
    if not torch.cuda.is_available():
        for kind, space in spaces.items():
            for config in space:
                print(f"  {kind}  {config}")
        return None
    cfg = AttnConfig()
    shape = (batch, cfg.n_heads, seq_len, cfg.head_dim, True, cfg.groups)
    winners = {}
    for kind in spaces:
        config, latency, _ = autotune(kind, shape, verbose=True)
        tuned.record(f"attention_{kind}", shape, config)
        _kernels.pop((kind, shape, AUTOTUNE), None)
        winners[kind] = (config, latency)
        print(f"{kind} winner {latency:.3f} ms: {config}")
    return winners


if __name__ == "__main__":
    sys.exit(harness_main("mimansm1_v1_amd.attention",
                          {"check": check_math, "gpu": check_gpu, "bench": benchmark, "tune": tune}))
