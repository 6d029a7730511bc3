"""MI355X SwiGLU feed-forward with the call surface of Mimans M1's
``mimans.model.swiglu_tilelang`` (CODE/mimans/model/swiglu_tilelang.py, "SW").

Drop-in surface (same names, arguments, layouts and return values):

* ``get_kernel(kind, *shape)``, ``_kernels``, ``AUTOTUNE``, ``warmup`` with
  kinds ``"gate_up"`` (x, w_gate, w_up) -> act, ``"split"`` -> (gate, up) and
  ``"grad"`` (d_act, gate, up) -> (d_gate, d_up)                  (SW:243-273)
* ``FusedSwiGLU`` / ``fused_swiglu(x, w_gate, w_up, w_down)``      (SW:276-305)
* ``FFNConfig``, ``SwiGLU`` with backends ``"hip"`` (alias ``"tilelang"``),
  ``"torch"``, ``"math"``; ``reference``                         (SW:308-365)
* harnesses ``check_math``, ``check_gpu``, ``benchmark``, ``tune`` (SW:368-638)

The kernels are the gfx950 HIP kernels of ``csrc/swiglu.hip`` behind the C ABI
(``include/mm1_swiglu.h``): the gate/up GEMM with the SwiGLU epilogue fused
(one launch writes gate, up and act for training), and the elementwise
gradient.  The down projection and the backward's GEMMs are hipBLASLt through
torch, as in the reference.  Without the built library every kernel entry
point raises; nothing falls back to another implementation.
"""
from __future__ import annotations

import argparse
import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import tuned
from .wgrad import wgrad

DTYPE = torch.bfloat16
MODE_ACT, MODE_SPLIT, MODE_TRAIN = 0, 1, 2     # MM1_SWIGLU_ACT / _SPLIT / _TRAIN

# The gfx950 tilings (one per kernel; SW:59-100 describes the reference's
# TileLang search space instead).
GATE_UP_TILES = dict(block_M=256, block_N=128, block_K=64, waves=8, stages=2)
GRAD_TILES = dict(cols_per_thread=8, threads=256)
# Token chunks of the down projection's weight gradient (wgrad.py): 2
# measured fastest at 16,384 tokens (271 -> 174 us).
DOWN_DW_CHUNKS = 2
AUTOTUNE = True


def gate_up_configs():
    return [dict(GATE_UP_TILES)]


def grad_configs():
    return [dict(GRAD_TILES)]


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require(t, name, shape, dtype=DTYPE):
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


class _GateUp:
    """(x [T,d], w_gate [d,F], w_up [d,F]) -> outputs of one gate/up launch."""

    def __init__(self, tokens, d_model, ffn, mode):
        if d_model % 128 or ffn % 128:
            raise ValueError(f"d_model={d_model} and ffn={ffn} must be multiples of 128")
        self.shape = (tokens, d_model, ffn)
        self.mode = mode
        self.config = dict(GATE_UP_TILES)
        self.latency = None
        _lib.load()

    def launch(self, x, w_gate, w_up):
        T, d, Fh = self.shape
        _require(x, "x", (T, d))
        _require(w_gate, "w_gate", (d, Fh))
        _require(w_up, "w_up", (d, Fh))
        new = lambda: torch.empty(T, Fh, dtype=DTYPE, device=x.device)
        gate = up = act = None
        if self.mode != MODE_ACT:
            gate, up = new(), new()
        if self.mode != MODE_SPLIT:
            act = new()
        ptr = lambda t: None if t is None else t.data_ptr()
        rc = _lib.load().mm1_swiglu_gate_up(x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), ptr(gate),
                                            ptr(up), ptr(act), T, d, Fh, self.mode, _stream(x.device))
        _lib.check(rc, "mm1_swiglu_gate_up")
        return gate, up, act

    def __repr__(self):
        return f"<{type(self).__name__} shape={self.shape} config={self.config}>"


class GateUpKernel(_GateUp):
    """gate_up_swiglu (SW:119-156): act = bf16(silu(x w_gate) * (x w_up))."""

    def __init__(self, tokens, d_model, ffn):
        super().__init__(tokens, d_model, ffn, MODE_ACT)

    def __call__(self, x, w_gate, w_up):
        return self.launch(x, w_gate, w_up)[2]


class SplitKernel(_GateUp):
    """gate_up_split (SW:158-200): (bf16(x w_gate), bf16(x w_up))."""

    def __init__(self, tokens, d_model, ffn):
        super().__init__(tokens, d_model, ffn, MODE_SPLIT)

    def __call__(self, x, w_gate, w_up):
        gate, up, _ = self.launch(x, w_gate, w_up)
        return gate, up


class TrainKernel(_GateUp):
    """gate_up_split plus FusedSwiGLU.forward's ``F.silu(gate) * up``
    (SW:283-284) in one launch: (gate, up, act)."""

    def __init__(self, tokens, d_model, ffn):
        super().__init__(tokens, d_model, ffn, MODE_TRAIN)

    def __call__(self, x, w_gate, w_up):
        return self.launch(x, w_gate, w_up)


class GradKernel:
    """swiglu_grad (SW:202-240): (d_act, gate, up) -> (d_gate, d_up).  With
    ``out`` = a [T, 2F] tensor the two results are written into its halves
    (returned as views), the layout the backward's GEMMs consume."""

    def __init__(self, tokens, ffn):
        self.shape = (tokens, ffn)
        self.config = dict(GRAD_TILES)
        self.latency = None
        _lib.load()

    def __call__(self, d_act, gate, up, out=None):
        T, Fh = self.shape
        for name, t in (("d_act", d_act), ("gate", gate), ("up", up)):
            _require(t, name, (T, Fh))
        if out is None:
            d_gate, d_up, ld = torch.empty_like(gate), torch.empty_like(gate), Fh
        else:
            _require(out, "out", (T, 2 * Fh))
            d_gate, d_up, ld = out[:, :Fh], out[:, Fh:], 2 * Fh
        rc = _lib.load().mm1_swiglu_grad(d_act.data_ptr(), gate.data_ptr(), up.data_ptr(),
                                         d_gate.data_ptr(), d_up.data_ptr(), T, Fh, ld,
                                         _stream(d_act.device))
        _lib.check(rc, "mm1_swiglu_grad")
        return d_gate, d_up

    def __repr__(self):
        return f"<GradKernel shape={self.shape} config={self.config}>"


_KINDS = {"gate_up": GateUpKernel, "split": SplitKernel, "train": TrainKernel, "grad": GradKernel}
_kernels: dict = {}


def get_kernel(kind, *shape):
    """Per-shape kernel handle cached under ``(kind, shape, AUTOTUNE)``
    (SW:243-261).  Each kernel has one gfx950 tiling, so the lookup order of
    the reference (tile record, search, defaults) always ends in it; a record
    is written for the shape when AUTOTUNE is set, as the reference's search
    would."""
    if kind not in _KINDS:
        raise ValueError(f"unknown kernel kind {kind!r}")
    key = (kind, tuple(shape), AUTOTUNE)
    if key not in _kernels:
        kernel = _KINDS[kind](*shape)
        name = f"swiglu_{kind}"
        if AUTOTUNE and tuned.lookup(name, shape) is None and torch.cuda.is_available():
            tuned.record(name, shape, tuned.config_of(kernel))
        _kernels[key] = kernel
    return _kernels[key]


def warmup(tokens, cfg=None):
    """Create the handles up front (SW:264-273)."""
    cfg = cfg or FFNConfig()
    get_kernel("gate_up", tokens, cfg.d_model, cfg.ffn_hidden)
    get_kernel("split", tokens, cfg.d_model, cfg.ffn_hidden)
    get_kernel("train", tokens, cfg.d_model, cfg.ffn_hidden)
    get_kernel("grad", tokens, cfg.ffn_hidden)


class FusedSwiGLU(torch.autograd.Function):
    """Same signature and returns as SW:276-301.  Forward: one HIP launch for
    gate, up and act (the reference's split kernel plus its two elementwise
    torch ops), then act @ w_down.  Backward: d_act = grad_out @ w_down^T, the
    HIP gradient kernel writing [d_gate | d_up] into one [T, 2F] buffer, and
    the reference's GEMMs with the two gate/up weight gradients from one
    product (x^T [d_gate | d_up]), d_x accumulated in one addmm, and the
    down-projection weight gradient over two token chunks (wgrad.py)."""

    @staticmethod
    def forward(ctx, x, w_gate, w_up, w_down):
        tokens, d_model = x.shape
        ffn = w_gate.shape[1]
        gate, up, act = get_kernel("train", tokens, d_model, ffn)(x, w_gate, w_up)
        out = act @ w_down
        ctx.save_for_backward(x, w_gate, w_up, w_down, gate, up, act)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, w_gate, w_up, w_down, gate, up, act = ctx.saved_tensors
        tokens, ffn = gate.shape
        grad_out = grad_out.contiguous()
        if grad_out.dtype != x.dtype:
            grad_out = grad_out.to(x.dtype)
        d_act = grad_out @ w_down.t()
        d_gu = torch.empty(tokens, 2 * ffn, dtype=x.dtype, device=x.device)
        d_gate, d_up = get_kernel("grad", tokens, ffn)(d_act, gate, up, out=d_gu)
        d_x = torch.addmm(d_gate @ w_gate.t(), d_up, w_up.t())
        d_w = x.t() @ d_gu
        # fp32 sum of two token chunks (wgrad.py), rounded to the weight's
        # dtype once, as the single bf16 GEMM rounds it
        d_w_down = wgrad(act, grad_out, DOWN_DW_CHUNKS).to(w_down.dtype)
        return d_x, d_w[:, :ffn], d_w[:, ffn:], d_w_down


def fused_swiglu(x, w_gate, w_up, w_down):
    return FusedSwiGLU.apply(x, w_gate, w_up, w_down)


@dataclass
class FFNConfig:
    d_model: int = 1280
    ffn_hidden: int = 3328
    backend: str = "hip"

    def __post_init__(self):
        assert self.ffn_hidden % 128 == 0
        assert self.d_model % 128 == 0

    @property
    def params(self):
        return 3 * self.d_model * self.ffn_hidden


class SwiGLU(nn.Module):
    """Same parameters, initialisation and backends as SW:323-359; the kernel
    backend is ``"hip"``, and the reference's name ``"tilelang"`` is an alias."""

    def __init__(self, cfg: FFNConfig):
        super().__init__()
        self.cfg = cfg
        self.w_gate = nn.Parameter(torch.empty(cfg.d_model, cfg.ffn_hidden))
        self.w_up = nn.Parameter(torch.empty(cfg.d_model, cfg.ffn_hidden))
        self.w_down = nn.Parameter(torch.empty(cfg.ffn_hidden, cfg.d_model))
        std = 0.02
        nn.init.normal_(self.w_gate, std=std)
        nn.init.normal_(self.w_up, std=std)
        nn.init.normal_(self.w_down, std=std / math.sqrt(2 * 27))

    def forward(self, x, backend=None):
        cfg = self.cfg
        backend = backend or cfg.backend
        shape = x.shape
        flat = x.reshape(-1, cfg.d_model)
        if backend in ("hip", "tilelang"):
            # bf16 kernels: the fp32 residual stream and raw parameters are cast
            # here, as the reference does (SW:335-343)
            out = fused_swiglu(flat.to(DTYPE).contiguous(), self.w_gate.to(DTYPE),
                               self.w_up.to(DTYPE), self.w_down.to(DTYPE))
            out = out.to(x.dtype)
        elif backend == "torch":
            out = (F.silu(flat @ self.w_gate) * (flat @ self.w_up)) @ self.w_down
        elif backend == "math":
            gate = flat.float() @ self.w_gate.float()
            up = flat.float() @ self.w_up.float()
            out = ((gate * torch.sigmoid(gate)) * up) @ self.w_down.float()
            out = out.to(x.dtype)
        else:
            raise ValueError(f"unknown backend {backend!r}")
        return out.reshape(shape)


def reference(x, w_gate, w_up, w_down):
    """The fp32 reference (SW:362-365)."""
    gate = x.float() @ w_gate.float()
    up = x.float() @ w_up.float()
    return ((gate * torch.sigmoid(gate)) * up) @ w_down.float()


def swiglu_flops(tokens, cfg=None):
    """fwd + bwd FLOPs of the FFN: three GEMMs forward, six backward (SW:584)."""
    cfg = cfg or FFNConfig()
    return 2.0 * tokens * cfg.d_model * cfg.ffn_hidden * 3 * 3


# ---------------------------------------------------------------------------
# Harnesses (SW:368-638)
def check_math():
    """CPU checks of the host-side pieces (SW:368-494)."""
    passed = True

    def check(label, condition):
        nonlocal passed
        passed &= bool(condition)
        print(f"  {'ok  ' if condition else 'FAIL'}  {label}")

    torch.manual_seed(0)
    cfg = FFNConfig()
    layers, tokens = 27, 8 * 2048

    print("hbm traffic, one ffn forward at 8x2048 tokens")
    unfused = 6 * tokens * cfg.ffn_hidden * 2
    fused = 2 * tokens * cfg.ffn_hidden * 2
    print(f"    unfused {unfused / 1e6:7.1f} MB, fused act {fused / 1e6:7.1f} MB")
    check("fusion removes two thirds of the intermediate traffic", fused * 3 == unfused)

    print("\ntilings (gfx950)")
    check("gate_up default is compiled", GATE_UP_TILES in gate_up_configs())
    check("grad default is compiled", GRAD_TILES in grad_configs())
    check("ffn and d_model fit the gate/up tile",
          cfg.ffn_hidden % GATE_UP_TILES["block_N"] == 0 and cfg.d_model % GATE_UP_TILES["block_K"] == 0)
    lds = GATE_UP_TILES["stages"] * 2 * GATE_UP_TILES["block_K"] * (
        GATE_UP_TILES["block_M"] + 2 * GATE_UP_TILES["block_N"])
    check(f"gate/up ring fits LDS ({lds // 1024} KiB of 160)", lds <= 160 * 1024)

    print("\nsilu derivative")
    z = torch.randn(2000, dtype=torch.float64) * 3
    z.requires_grad_(True)
    F.silu(z).sum().backward()
    sig = torch.sigmoid(z.detach())
    analytic = sig * (1 + z.detach() * (1 - sig))
    err = (z.grad - analytic).abs().max().item()
    check(f"matches sigmoid(z)*(1+z*(1-sigmoid(z))) ({err:.2e})", err < 1e-12)
    check("silu(0)=0 and dsilu(0)=0.5",
          abs(F.silu(torch.zeros(1)).item()) < 1e-12 and abs(torch.sigmoid(torch.zeros(1)).item() - 0.5) < 1e-12)

    print("\nmodule")
    ffn = SwiGLU(cfg)
    n = sum(p.numel() for p in ffn.parameters())
    check(f"parameters {n:,} == 3*{cfg.d_model}*{cfg.ffn_hidden}", n == cfg.params)
    x = torch.randn(2, 16, cfg.d_model)
    y = ffn(x, backend="torch")
    check(f"shape {tuple(x.shape)} -> {tuple(y.shape)}", y.shape == x.shape)
    err = (y - ffn(x, backend="math")).abs().max().item()
    check(f"torch and fp32 reference agree ({err:.2e})", err < 1e-4)
    x = torch.randn(2, 8, cfg.d_model, requires_grad=True)
    ffn(x, backend="torch").sum().backward()
    check("finite gradients everywhere",
          torch.isfinite(x.grad).all() and all(torch.isfinite(p.grad).all() for p in ffn.parameters()))

    print("\n" + ("all math checks passed" if passed else "FAILURES ABOVE"))
    return passed


def check_gpu(tokens=4096):
    """The fused op against the fp32 reference on the GPU (SW:497-556)."""
    if not torch.cuda.is_available():
        print("needs a HIP device")
        return None
    cfg = FFNConfig()
    torch.manual_seed(0)
    dev = "cuda"
    x = torch.randn(tokens, cfg.d_model, device=dev, dtype=DTYPE, requires_grad=True)
    wg = (torch.randn(cfg.d_model, cfg.ffn_hidden, device=dev, dtype=DTYPE) * 0.02).requires_grad_(True)
    wu = (torch.randn(cfg.d_model, cfg.ffn_hidden, device=dev, dtype=DTYPE) * 0.02).requires_grad_(True)
    wd = (torch.randn(cfg.ffn_hidden, cfg.d_model, device=dev, dtype=DTYPE) * 0.02).requires_grad_(True)
    grad_out = torch.randn(tokens, cfg.d_model, device=dev, dtype=DTYPE)
    act = get_kernel("gate_up", tokens, cfg.d_model, cfg.ffn_hidden)(x, wg, wu)
    want_act = F.silu(x.float() @ wg.float()) * (x.float() @ wu.float())
    rel = ((act.float() - want_act).abs().max() / want_act.abs().max()).item()
    print(f"fused activation vs fp32: rel err {rel:.3e}  {'ok' if rel < 2e-2 else 'FAIL'}")
    results = {"act": rel}
    out = fused_swiglu(x, wg, wu, wd)
    out.backward(grad_out, retain_graph=True)
    mine = [t.grad.clone() for t in (x, wg, wu, wd)]
    for t in (x, wg, wu, wd):
        t.grad = None
    want = reference(x, wg, wu, wd).to(DTYPE)
    want.backward(grad_out)
    theirs = [t.grad.clone() for t in (x, wg, wu, wd)]
    for name, a, b in zip(("out", "d_x", "d_w_gate", "d_w_up", "d_w_down"), [out] + mine, [want] + theirs):
        rel = ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp(min=1e-6)).item()
        results[name] = rel
        print(f"  {name:9s} rel err {rel:.3e}  {'ok' if rel < 3e-2 else 'FAIL'}")
    return results


def benchmark(tokens=16384):
    """Fused op vs eager torch, fwd + bwd (SW:559-610)."""
    if not torch.cuda.is_available():
        print("needs a HIP device")
        return None
    cfg = FFNConfig()
    dev = "cuda"
    x = torch.randn(tokens, cfg.d_model, device=dev, dtype=DTYPE, requires_grad=True)
    wg = torch.randn(cfg.d_model, cfg.ffn_hidden, device=dev, dtype=DTYPE, requires_grad=True)
    wu = torch.randn(cfg.d_model, cfg.ffn_hidden, device=dev, dtype=DTYPE, requires_grad=True)
    wd = torch.randn(cfg.ffn_hidden, cfg.d_model, device=dev, dtype=DTYPE, requires_grad=True)
    grad_out = torch.randn(tokens, cfg.d_model, device=dev, dtype=DTYPE)
    flops = swiglu_flops(tokens, cfg)

    def time_it(fn, iters=30):
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(True), torch.cuda.Event(True)
        start.record()
        for _ in range(iters):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / iters

    def clear():
        for t in (x, wg, wu, wd):
            t.grad = None

    def eager():
        ((F.silu(x @ wg) * (x @ wu)) @ wd).backward(grad_out, retain_graph=True)
        clear()

    def hip():
        fused_swiglu(x, wg, wu, wd).backward(grad_out, retain_graph=True)
        clear()

    results = {"eager": time_it(eager), "hip": time_it(hip)}
    for name, ms in sorted(results.items(), key=lambda kv: kv[1]):
        print(f"  {name:10s} {ms:8.3f} ms   {flops / ms * 1e-9:7.1f} TFLOP/s")
    return results


def tune(tokens=16384):
    """The gfx950 build has one tiling per kernel: list them (SW:613-632)."""
    print(f"gate_up candidates {len(gate_up_configs())}: {gate_up_configs()}")
    print(f"grad candidates    {len(grad_configs())}: {grad_configs()}")


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--check", action="store_true")
    parser.add_argument("--gpu", action="store_true")
    parser.add_argument("--bench", action="store_true")
    parser.add_argument("--tune", action="store_true")
    args = parser.parse_args()
    if not any(vars(args).values()):
        args.check = True
    if args.check:
        check_math()
    if args.gpu:
        check_gpu()
    if args.bench:
        benchmark()
    if args.tune:
        tune()
