"""MI355X fused cross-entropy head with the call surface of Mimans M1's
``mimans.model.lm_head_tilelang`` (CODE/mimans/model/lm_head_tilelang.py, "LM").

Drop-in surface (same names, arguments and return values):

* ``get_kernel((tokens, d_model, vocab))(hidden, weight) -> lse``,
  ``_kernels``, ``AUTOTUNE``, ``warmup``                          (LM:159-182)
* ``accum_dtype``, ``gather_target_logits``                     (LM:185-190)
* ``FusedCrossEntropy`` / ``fused_cross_entropy(hidden, weight, targets, chunk)``
                                                                 (LM:193-247)
* ``HeadConfig``, ``LMHead`` (tied or own matrix, logit scale, backends
  ``"hip"`` (alias ``"tilelang"``) and ``"torch"``)              (LM:250-335)
* harnesses ``check_math``, ``check_gpu``, ``benchmark``, ``tune`` (LM:338-590)

The kernels are the gfx950 HIP kernels of ``csrc/lm_head.hip`` behind the C ABI
(``include/mm1_lm_head.h``): the forward computes, in one GEMM pass over the
vocabulary, each token's log-sum-exp and target logit without storing the
[tokens, vocab] logits; the backward computes bf16 d_logits one vocabulary
chunk at a time in a second GEMM pass and hands them to two hipBLASLt GEMMs
(d_hidden, d_weight).  On a 288 GB MI355X the default chunk is the whole
vocabulary (1.6 GB of bf16 d_logits at 8 x 2048 tokens), where the
reference's 4096-entry chunks were sized for a much smaller card.  Without the
built library the kernel entry points raise; there is no CPU fallback.
"""
from __future__ import annotations

import argparse
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import tuned

DTYPE = torch.bfloat16
IGNORE_INDEX = -100
AUTOTUNE = True
# The gfx950 tiling of both vocabulary GEMMs (LM:61-85 describes the
# reference's TileLang search space instead).
LSE_TILES = dict(block_M=256, block_N=256, block_K=64, waves=8, stages=2)
VOCAB_CHUNK = 49152


def lse_configs():
    return [dict(LSE_TILES)]


def logits_bytes(tokens, vocab, elem=2):
    return tokens * vocab * elem


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


class LseKernel:
    """(hidden [T, d], weight [d, V]) -> lse [T] fp32 (natural log); with
    ``targets`` also the target logits and per-token losses."""

    def __init__(self, tokens, d_model, vocab):
        if d_model % 128 or vocab % 128:
            raise ValueError(f"d_model={d_model} and vocab={vocab} must be multiples of 128")
        self.shape = (tokens, d_model, vocab)
        self.config = dict(LSE_TILES)
        self.latency = None
        _lib.load()

    def forward(self, hidden, weight, targets=None, ignore_index=IGNORE_INDEX):
        T, d, V = self.shape
        _require(hidden, "hidden", (T, d))
        _require(weight, "weight", (d, V))
        lib = _lib.load()
        dev = hidden.device
        lse = torch.empty(T, dtype=torch.float32, device=dev)
        tl = loss = None
        if targets is not None:
            _require(targets, "targets", (T,), torch.int64)
            tl = torch.empty(T, dtype=torch.float32, device=dev)
            loss = torch.empty(T, dtype=torch.float32, device=dev)
        ws_bytes = lib.mm1_lm_head_workspace_size(T, V)
        ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=dev)
        ptr = lambda t: None if t is None else t.data_ptr()
        rc = lib.mm1_lm_head_lse(hidden.data_ptr(), weight.data_ptr(), ptr(targets), int(ignore_index),
                                 lse.data_ptr(), ptr(tl), ptr(loss), ws.data_ptr(), ws_bytes, T, d, V,
                                 _stream(dev))
        _lib.check(rc, "mm1_lm_head_lse")
        return lse, tl, loss

    def __call__(self, hidden, weight):
        return self.forward(hidden, weight)[0]

    def dlogits(self, hidden, weight, targets, lse, scale, v0, vn, out=None, ignore_index=IGNORE_INDEX):
        """bf16 d_logits of vocabulary entries [v0, v0 + vn) into out [T, vn]."""
        T, d, V = self.shape
        if out is None:
            out = torch.empty(T, vn, dtype=DTYPE, device=hidden.device)
        rc = _lib.load().mm1_lm_head_dlogits(hidden.data_ptr(), weight.data_ptr(), targets.data_ptr(),
                                             int(ignore_index), lse.data_ptr(), scale.data_ptr(),
                                             out.data_ptr(), out.stride(0), T, d, V, v0, vn,
                                             _stream(hidden.device))
        _lib.check(rc, "mm1_lm_head_dlogits")
        return out

    def __repr__(self):
        return f"<LseKernel shape={self.shape} config={self.config}>"


_kernels: dict = {}


def get_kernel(shape):
    """Per-shape handle cached under ``(shape, AUTOTUNE)`` (LM:159-174); the
    gfx950 build has one tiling, which is recorded for the shape when
    AUTOTUNE is set, as the reference's search would record its winner."""
    key = (tuple(shape), AUTOTUNE)
    if key not in _kernels:
        kernel = LseKernel(*shape)
        if AUTOTUNE and tuned.lookup("lm_head_lse", shape) is None and torch.cuda.is_available():
            tuned.record("lm_head_lse", shape, tuned.config_of(kernel))
        _kernels[key] = kernel
    return _kernels[key]


def warmup(tokens, d_model=1280, vocab=49152):
    """Create the handle up front (LM:177-182)."""
    get_kernel((tokens, d_model, vocab))


def accum_dtype(tensor):
    """fp32 for the dtypes trained in, never narrower than the input (LM:185-189)."""
    return torch.promote_types(tensor.dtype, torch.float32)


def gather_target_logits(hidden, weight, targets):
    """The target's logit in the accumulation dtype (LM:186-190)."""
    acc = accum_dtype(hidden)
    valid = targets.clamp(min=0)
    rows = weight.index_select(1, valid).t()
    return (hidden.to(acc) * rows.to(acc)).sum(-1)


class FusedCrossEntropy(torch.autograd.Function):
    """Same signature and returns as LM:193-243: the mean cross entropy over
    tokens whose target is not IGNORE_INDEX (0 when there are none).  bf16
    HIP tensors only."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, chunk):
        tokens, d_model = hidden.shape
        vocab = weight.shape[1]
        if not (hidden.is_cuda and hidden.dtype is DTYPE and weight.dtype is DTYPE):
            raise ValueError("fused_cross_entropy runs the HIP kernels: hidden and weight must be bf16 "
                             f"HIP tensors (got {hidden.dtype} on {hidden.device}, {weight.dtype})")
        kernel = get_kernel((tokens, d_model, vocab))
        targets = targets.contiguous()
        lse, _, per_token = kernel.forward(hidden, weight, targets)
        count = (targets != IGNORE_INDEX).sum().clamp(min=1)
        loss = per_token.sum() / count
        ctx.save_for_backward(hidden, weight, targets, lse, count)
        ctx.chunk = chunk
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        hidden, weight, targets, lse, count = ctx.saved_tensors
        tokens, d_model = hidden.shape
        vocab = weight.shape[1]
        chunk = max(128, (min(ctx.chunk, vocab) // 128) * 128)
        kernel = get_kernel((tokens, d_model, vocab))
        scale = (grad_loss.float() / count).reshape(1).contiguous()
        if chunk >= vocab:
            # the whole vocabulary at once: two plain GEMMs on the bf16 d_logits
            dl = kernel.dlogits(hidden, weight, targets, lse, scale, 0, vocab)
            return dl @ weight.t(), hidden.t() @ dl, None, None
        d_weight = torch.empty_like(weight)
        d_hidden = torch.zeros(tokens, d_model, dtype=torch.float32, device=hidden.device)
        for start in range(0, vocab, chunk):
            stop = min(start + chunk, vocab)
            dl = kernel.dlogits(hidden, weight, targets, lse, scale, start, stop - start)
            d_hidden += (dl @ weight[:, start:stop].t()).float()
            d_weight[:, start:stop] = hidden.t() @ dl
        return d_hidden.to(hidden.dtype), d_weight, None, None


def fused_cross_entropy(hidden, weight, targets, chunk=VOCAB_CHUNK):
    return FusedCrossEntropy.apply(hidden, weight, targets, chunk)


@dataclass
class HeadConfig:
    d_model: int = 1280
    vocab: int = 49152
    tied: bool = True
    chunk: int = VOCAB_CHUNK
    logit_scale: float = None

    def __post_init__(self):
        assert self.vocab % 128 == 0
        assert self.d_model % 128 == 0
        # logits scaled by 1/sqrt(d_model) by default (LM:259-270)
        if self.logit_scale is None:
            self.logit_scale = self.d_model ** -0.5

    @property
    def params(self):
        return self.d_model * self.vocab


class LMHead(nn.Module):
    """Same structure as LM:279-335: a tied head reads the embedding matrix
    (no parameters of its own), an untied one owns [d_model, vocab]; the input
    is scaled by ``logit_scale`` before the kernel.  Kernel backend ``"hip"``
    (``"tilelang"`` is an alias), or ``"torch"``."""

    def __init__(self, cfg: HeadConfig, embedding: nn.Embedding = None):
        super().__init__()
        self.cfg = cfg
        if cfg.tied:
            assert embedding is not None, "tied head needs the embedding module"
            self.embedding = [embedding]
            self.weight = None
        else:
            self.embedding = None
            self.weight = nn.Parameter(torch.empty(cfg.d_model, cfg.vocab))
            nn.init.normal_(self.weight, std=0.02)

    def matrix(self):
        if self.cfg.tied:
            return self.embedding[0].weight.t()
        return self.weight

    def forward(self, hidden, targets=None, backend="hip"):
        shape = hidden.shape
        flat = hidden.reshape(-1, self.cfg.d_model)
        if self.cfg.logit_scale != 1.0:
            flat = flat * self.cfg.logit_scale
        weight = self.matrix()
        if targets is None:
            return (flat @ weight).reshape(*shape[:-1], self.cfg.vocab)
        flat_targets = targets.reshape(-1)
        if backend in ("hip", "tilelang"):
            # bf16 kernels: cast the fp32 stream and the (transposed view of
            # the) tied matrix to contiguous bf16 here, as LM:313-323 does
            flat = flat.to(DTYPE).contiguous()
            weight = weight.to(DTYPE).contiguous()
            return fused_cross_entropy(flat, weight, flat_targets, self.cfg.chunk)
        if backend == "torch":
            acc = accum_dtype(flat)
            valid = (flat_targets != IGNORE_INDEX).sum().clamp(min=1)
            return F.cross_entropy(flat.to(acc) @ weight.to(acc), flat_targets, ignore_index=IGNORE_INDEX,
                                   reduction="sum") / valid
        raise ValueError(f"unknown backend {backend!r}")


def lm_head_flops(tokens, cfg=None):
    """(forward, backward) GEMM flops: the log-sum-exp pass; the d_logits
    pass plus d_hidden and d_weight."""
    cfg = cfg or HeadConfig()
    unit = 2.0 * tokens * cfg.d_model * cfg.vocab
    return unit, 3 * unit


# ---------------------------------------------------------------------------
# Harnesses (LM:338-590)
def check_math():
    """CPU checks of the host-side pieces and the math (LM:338-476)."""
    passed = True

    def check(label, condition):
        nonlocal passed
        passed &= bool(condition)
        print(f"  {'ok  ' if condition else 'FAIL'}  {label}")

    torch.manual_seed(0)
    cfg = HeadConfig()
    tokens = 8 * 2048
    naive, fused = logits_bytes(tokens, cfg.vocab), tokens * 4
    print(f"logits bf16 {naive / 1e6:.1f} MB; fused lse {fused / 1e6:.4f} MB")
    check("logits alone exceed 1.5 GB", naive > 1.5e9)
    check("fused output is under a megabyte", fused < 1e6)
    check("one-chunk backward d_logits fit a 288 GB card many times over",
          logits_bytes(tokens, cfg.chunk) < 4e9)

    print("\nonline logsumexp recurrence")
    x = torch.randn(64, 5000, dtype=torch.float64) * 8
    m = torch.full((64,), float("-inf"), dtype=torch.float64)
    s = torch.zeros(64, dtype=torch.float64)
    for start in range(0, 5000, 128):
        tile = x[:, start:start + 128]
        prev = m.clone()
        m = torch.maximum(m, tile.max(dim=1).values)
        s = s * torch.exp(prev - m) + torch.exp(tile - m.unsqueeze(1)).sum(1)
    err = (torch.log(s) + m - torch.logsumexp(x, dim=1)).abs().max().item()
    check(f"matches torch.logsumexp ({err:.2e})", err < 1e-12)

    print("\ncross entropy identity")
    logits = torch.randn(200, 500, dtype=torch.float64)
    targets = torch.randint(0, 500, (200,))
    manual = (torch.logsumexp(logits, dim=1) - logits[torch.arange(200), targets]).mean()
    check("lse - target_logit == cross_entropy", (manual - F.cross_entropy(logits, targets)).abs() < 1e-12)

    print("\ngradient identity")
    logits = torch.randn(64, 200, dtype=torch.float64, requires_grad=True)
    targets = torch.randint(0, 200, (64,))
    F.cross_entropy(logits, targets).backward()
    analytic = (torch.softmax(logits.detach(), dim=1) - F.one_hot(targets, 200).double()) / 64
    check("d_logits == (softmax - onehot)/N", (logits.grad - analytic).abs().max() < 1e-12)

    print("\nhost logic")
    check("gather_target_logits is the target column's dot product",
          torch.allclose(gather_target_logits(torch.eye(4), torch.arange(12.0).reshape(4, 3),
                                              torch.tensor([2, 0, 1, 2])),
                         torch.tensor([2.0, 3.0, 7.0, 11.0])))
    emb = nn.Embedding(cfg.vocab, cfg.d_model)
    head = LMHead(cfg, emb)
    check("tied head holds no parameters of its own", sum(p.numel() for p in head.parameters()) == 0)
    check("shares the embedding matrix", head.matrix().data_ptr() == emb.weight.data_ptr())
    check("default logit scale 1/sqrt(d_model)", abs(cfg.logit_scale - cfg.d_model ** -0.5) < 1e-15)
    print("\n" + ("all math checks passed" if passed else "FAILURES ABOVE"))
    return passed


def check_gpu(tokens=4096):
    """lse, loss and gradients against the fp32 reference path (LM:479-520)."""
    if not torch.cuda.is_available():
        print("needs a HIP device")
        return None
    cfg = HeadConfig()
    torch.manual_seed(0)
    hidden = (torch.randn(tokens, cfg.d_model, device="cuda", dtype=DTYPE) * 0.1).requires_grad_(True)
    weight = (torch.randn(cfg.d_model, cfg.vocab, device="cuda", dtype=DTYPE) * 0.02).requires_grad_(True)
    targets = torch.randint(0, cfg.vocab, (tokens,), device="cuda")
    lse = get_kernel((tokens, cfg.d_model, cfg.vocab))(hidden, weight)
    want = torch.logsumexp(hidden.float() @ weight.float(), dim=-1)
    err = (lse - want).abs().max().item()
    print(f"lse vs reference: max err {err:.3e}  {'ok' if err < 5e-3 else 'FAIL'}")
    results = {"lse": err}
    loss = fused_cross_entropy(hidden, weight, targets)
    loss.backward()
    mine = [hidden.grad.clone(), weight.grad.clone()]
    hidden.grad = weight.grad = None
    ref = F.cross_entropy(hidden.float() @ weight.float(), targets)
    ref.backward()
    theirs = [hidden.grad.clone(), weight.grad.clone()]
    hidden.grad = weight.grad = None
    print(f"loss {loss.item():.6f} vs {ref.item():.6f}")
    results["loss"] = abs(loss.item() - ref.item())
    for name, a, b in zip(("d_hidden", "d_weight"), mine, theirs):
        rel = ((a.float() - b.float()).abs().max() / b.float().abs().max().clamp(min=1e-6)).item()
        results[name] = rel
        print(f"  {name:9s} rel err {rel:.3e}  {'ok' if rel < 3e-2 else 'FAIL'}")
    return results


def benchmark(tokens=16384):
    """Fused vs the naive fp32 logits path, fwd + bwd (LM:523-572)."""
    if not torch.cuda.is_available():
        print("needs a HIP device")
        return None
    cfg = HeadConfig()
    hidden = (torch.randn(tokens, cfg.d_model, device="cuda", dtype=DTYPE) * 0.1).requires_grad_(True)
    weight = (torch.randn(cfg.d_model, cfg.vocab, device="cuda", dtype=DTYPE) * 0.02).requires_grad_(True)
    targets = torch.randint(0, cfg.vocab, (tokens,), device="cuda")

    def time_it(fn, iters=20):
        for _ in range(5):
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
        hidden.grad = weight.grad = None

    def naive():
        F.cross_entropy(hidden.float() @ weight.float(), targets).backward()
        clear()

    def fused():
        fused_cross_entropy(hidden, weight, targets).backward()
        clear()

    results = {"fused": time_it(fused), "naive": time_it(naive)}
    for name, ms in sorted(results.items(), key=lambda kv: kv[1]):
        print(f"  {name:8s} {ms:8.3f} ms")
    return results


def tune(tokens=16384):
    """The gfx950 build has one tiling: list it (LM:575-590)."""
    print(f"lse candidates {len(lse_configs())}: {lse_configs()}")


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
