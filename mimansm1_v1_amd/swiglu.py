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

import math
import sys
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
    """The feed-forward block (SW:323-359): raw parameters w_gate, w_up
    [d_model, ffn] and w_down [ffn, d_model], drawn from N(0, 0.02^2) in that
    order, w_down's deviation divided by sqrt(2 * 27 layers).  Backends:
    ``"hip"`` (the gfx950 kernels; the reference's name ``"tilelang"`` is an
    alias), ``"torch"`` (eager, in the input's dtype) and ``"math"`` (fp32)."""

    _STD = 0.02

    def __init__(self, cfg: FFNConfig):
        super().__init__()
        self.cfg = cfg
        d, f = cfg.d_model, cfg.ffn_hidden
        for name, shape, std in (("w_gate", (d, f), self._STD), ("w_up", (d, f), self._STD),
                                 ("w_down", (f, d), self._STD / math.sqrt(2 * 27))):
            self.register_parameter(name, nn.Parameter(torch.empty(shape).normal_(0.0, std)))

    def _weights(self, dtype=None):
        ws = (self.w_gate, self.w_up, self.w_down)
        return ws if dtype is None else tuple(w.to(dtype) for w in ws)

    def _run_hip(self, rows, out_dtype):
        # the kernels take bf16 operands: the fp32 residual stream and the raw
        # parameters (which autocast does not reach) are cast here (SW:335-343)
        return fused_swiglu(rows.to(DTYPE).contiguous(), *self._weights(DTYPE)).to(out_dtype)

    def _run_torch(self, rows, out_dtype):
        w_gate, w_up, w_down = self._weights()
        return (F.silu(rows @ w_gate) * (rows @ w_up)) @ w_down

    def _run_math(self, rows, out_dtype):
        return reference(rows, *self._weights()).to(out_dtype)

    def forward(self, x, backend=None):
        backend = backend or self.cfg.backend
        runs = {"hip": self._run_hip, "tilelang": self._run_hip, "torch": self._run_torch,
                "math": self._run_math}
        if backend not in runs:
            raise ValueError(f"unknown backend {backend!r}")
        return runs[backend](x.reshape(-1, self.cfg.d_model), x.dtype).reshape(x.shape)


def reference(x, w_gate, w_up, w_down):
    """The fp32 math of the block (SW:362-365): (silu(x Wg) * (x Wu)) Wd with
    silu(g) = g * sigmoid(g), evaluated in that order."""
    xf = x.float()
    g = xf @ w_gate.float()
    return (g * g.sigmoid() * (xf @ w_up.float())) @ w_down.float()


def swiglu_flops(tokens, cfg=None):
    """fwd + bwd FLOPs of the FFN: three GEMMs forward, six backward (SW:584)."""
    cfg = cfg or FFNConfig()
    return 2.0 * tokens * cfg.d_model * cfg.ffn_hidden * 3 * 3


# ---------------------------------------------------------------------------
# Harnesses (SW:368-638)
def check_math(quiet=False) -> Report:
    """CPU checks (the reference's check(), SW:368-494): what the fusion saves,
    the gfx950 tiling, the SiLU derivative the gradient kernel uses, the
    module."""
    report = Report("swiglu math", quiet=quiet)
    cfg = FFNConfig()
    gen = torch.Generator().manual_seed(0)
    tokens = 8 * 2048

    report.section("intermediate HBM traffic of one forward (8 x 2048 tokens)")
    per_tensor = tokens * cfg.ffn_hidden * 2
    # unfused: gate and up written, read by silu(gate) * up, act written, read by down
    unfused, fused = 6 * per_tensor, 2 * per_tensor
    report.note(f"[T, F] bf16 tensor {per_tensor / 1e6:.1f} MB: unfused {unfused / 1e6:.0f} MB, fused {fused / 1e6:.0f} MB")
    report.expect("the fused epilogue cuts it to a third", unfused == 3 * fused)

    report.section("gfx950 tiling")
    t = GATE_UP_TILES
    report.expect("defaults are the compiled tilings", gate_up_configs() == [t] and grad_configs() == [GRAD_TILES])
    report.expect("d_model and ffn are whole tiles", cfg.ffn_hidden % t["block_N"] == 0 and cfg.d_model % t["block_K"] == 0)
    ring = t["stages"] * t["block_K"] * (t["block_M"] + 2 * t["block_N"]) * 2
    report.expect("the LDS ring fits 160 KiB", ring <= 160 * 1024, f"{ring // 1024} KiB")

    report.section("SiLU derivative (the gradient kernel's formula)")
    g = (torch.randn(4096, generator=gen, dtype=torch.float64) * 4).requires_grad_(True)
    (auto,) = torch.autograd.grad(F.silu(g).sum(), g)
    sg = torch.sigmoid(g.detach())
    closed = sg + g.detach() * sg * (1 - sg)
    err = (auto - closed).abs().max().item()
    report.expect("d silu(g)/dg = s + g s (1 - s), s = sigmoid(g)", err < 1e-12, err)
    zero = torch.zeros(1, dtype=torch.float64, requires_grad=True)
    (at_zero,) = torch.autograd.grad(F.silu(zero).sum(), zero)
    report.expect("silu(0) = 0 with slope 1/2", F.silu(zero).item() == 0.0 and at_zero.item() == 0.5)

    report.section("module")
    torch.manual_seed(0)
    block = SwiGLU(cfg)
    count = sum(p.numel() for p in block.parameters())
    report.expect("parameter count 3 * d_model * ffn", count == cfg.params, count)
    x = torch.randn(3, 11, cfg.d_model, generator=gen)
    y = block(x, backend="torch")
    report.expect("output keeps the input's shape", tuple(y.shape) == tuple(x.shape))
    gap = (y - block(x, backend="math")).abs().max().item()
    report.expect("eager and fp32 backends agree", gap < 1e-4, gap)
    x.requires_grad_(True)
    block(x, backend="torch").square().mean().backward()
    report.expect("gradients reach the input and every weight, finite",
                  all(t.grad is not None and bool(torch.isfinite(t.grad).all()) for t in (x, *block.parameters())))
    return report.finish()


def check_gpu(tokens=4096, quiet=False) -> Report:
    """The fused op against the fp32 math on the GPU (the reference's
    check_gpu, SW:497-556, gate max|d| / max|ref| < 3e-2): the fused
    activation kernel, then fused_swiglu's output and four gradients.  x ~
    N(0,1), weights ~ N(0, 0.02^2), seed 0."""
    report = Report("swiglu gpu", quiet=quiet)
    if not needs_gpu("check_gpu"):
        return report
    cfg = FFNConfig()
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    draw = lambda *shape, scale=1.0: (torch.randn(*shape, device=dev, generator=gen) * scale).to(DTYPE)
    x = draw(tokens, cfg.d_model)
    weights = [draw(cfg.d_model, cfg.ffn_hidden, scale=0.02), draw(cfg.d_model, cfg.ffn_hidden, scale=0.02),
               draw(cfg.ffn_hidden, cfg.d_model, scale=0.02)]
    d_out = draw(tokens, cfg.d_model)

    report.section(f"gate/up kernel, {tokens} tokens")
    act = get_kernel("gate_up", tokens, cfg.d_model, cfg.ffn_hidden)(x, weights[0], weights[1])
    g = x.float() @ weights[0].float()
    e = compare(act, g * g.sigmoid() * (x.float() @ weights[1].float()))
    report.expect("act: max|d|/max|ref| < 2e-2", e["finite"] and e["max_rel"] < 2e-2, e["max_rel"])

    report.section("fused_swiglu forward + backward")
    leaves = [t.clone().requires_grad_(True) for t in (x, *weights)]
    out = fused_swiglu(*leaves)
    got = (out,) + torch.autograd.grad(out, leaves, d_out)
    exact = [t.detach().float().requires_grad_(True) for t in (x, *weights)]
    ref_out = reference(*exact)
    want = (ref_out,) + torch.autograd.grad(ref_out, exact, d_out.float())
    for name, a, b in zip(("out", "d_x", "d_w_gate", "d_w_up", "d_w_down"), got, want):
        e = compare(a, b)
        report.expect(f"{name}: max|d|/max|ref| < 3e-2", e["finite"] and e["max_rel"] < 3e-2, e["max_rel"])
        report.note(f"{name}: rel-L2 {e['rel_l2']:.3e}")
    return report.finish()


def benchmark(tokens=16384, quiet=False) -> dict:
    """fwd + bwd of the fused op and of eager torch at `tokens` tokens (the
    reference's benchmark, SW:559-610), HIP-event timed.  Returns {name: ms}."""
    if not needs_gpu("benchmark"):
        return {}
    cfg = FFNConfig()
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    leaf = lambda *shape: torch.randn(*shape, device=dev, dtype=DTYPE, generator=gen).requires_grad_(True)
    x = leaf(tokens, cfg.d_model)
    wg, wu, wd = leaf(cfg.d_model, cfg.ffn_hidden), leaf(cfg.d_model, cfg.ffn_hidden), leaf(cfg.ffn_hidden, cfg.d_model)
    d_out = torch.randn(tokens, cfg.d_model, device=dev, dtype=DTYPE, generator=gen)
    leaves = (x, wg, wu, wd)
    steps = {
        "hip": lambda: torch.autograd.grad(fused_swiglu(*leaves), leaves, d_out),
        "eager": lambda: torch.autograd.grad((F.silu(x @ wg) * (x @ wu)) @ wd, leaves, d_out),
    }
    ms = {name: time_cuda(step, warmup=10, iters=30) for name, step in steps.items()}
    if not quiet:
        flops = swiglu_flops(tokens, cfg)
        for name, t in sorted(ms.items(), key=lambda kv: kv[1]):
            print(f"  {name:6s} {t:8.3f} ms  {flops / t * 1e-9:7.1f} TFLOP/s")
    return ms


def tune(tokens=16384):
    """The gfx950 build compiles one tiling per kernel (the reference
    autotunes TileLang's space, SW:613-632): list them."""
    for name, space in (("gate_up", gate_up_configs()), ("grad", grad_configs())):
        print(f"{name}: {len(space)} tiling(s): {space}")
    return {"gate_up": gate_up_configs(), "grad": grad_configs()}


if __name__ == "__main__":
    sys.exit(harness_main("mimansm1_v1_amd.swiglu",
                          {"check": check_math, "gpu": check_gpu, "bench": benchmark, "tune": tune}))
