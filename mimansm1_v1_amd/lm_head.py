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

import sys
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import tuned
from .harness import Report, compare, needs_gpu, time_cuda
from .harness import main as harness_main

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
    """Output head with the fused loss (LM:279-335).  Tied (the default): the
    head reads the transpose of the embedding matrix and owns no parameters;
    untied: its own [d_model, vocab] matrix from N(0, 0.02^2).  The hidden
    states are multiplied by ``logit_scale`` before the matrix, which scales
    the logits without touching the kernel.  ``forward(hidden)`` returns the
    logits; with ``targets`` it returns the mean cross-entropy over the
    targets that are not IGNORE_INDEX, through the gfx950 kernels (backend
    ``"hip"``, alias ``"tilelang"``) or torch (``"torch"``)."""

    def __init__(self, cfg: HeadConfig, embedding: nn.Embedding = None):
        super().__init__()
        self.cfg = cfg
        if cfg.tied and embedding is None:
            raise ValueError("a tied head needs the embedding module")
        # the embedding is held in a list so that it is not registered twice
        self.embedding = [embedding] if cfg.tied else None
        self.weight = None if cfg.tied else nn.Parameter(torch.empty(cfg.d_model, cfg.vocab).normal_(0.0, 0.02))

    def matrix(self):
        """[d_model, vocab]: the tied embedding's transpose (a view) or own matrix."""
        return self.embedding[0].weight.t() if self.cfg.tied else self.weight

    def _loss_hip(self, rows, weight, targets):
        # bf16 kernels: the fp32 stream and the tied matrix's transposed view
        # become contiguous bf16 here (LM:313-323)
        return fused_cross_entropy(rows.to(DTYPE).contiguous(), weight.to(DTYPE).contiguous(), targets,
                                   self.cfg.chunk)

    def _loss_torch(self, rows, weight, targets):
        # sum over valid rows / their count (at least 1): an all-ignored batch
        # gives 0, as the fused path does
        acc = accum_dtype(rows)
        total = F.cross_entropy(rows.to(acc) @ weight.to(acc), targets, ignore_index=IGNORE_INDEX,
                                reduction="sum")
        return total / (targets != IGNORE_INDEX).sum().clamp(min=1)

    def forward(self, hidden, targets=None, backend="hip"):
        rows = hidden.reshape(-1, self.cfg.d_model)
        if self.cfg.logit_scale != 1.0:
            rows = rows * self.cfg.logit_scale
        weight = self.matrix()
        if targets is None:
            return (rows @ weight).reshape(*hidden.shape[:-1], self.cfg.vocab)
        losses = {"hip": self._loss_hip, "tilelang": self._loss_hip, "torch": self._loss_torch}
        if backend not in losses:
            raise ValueError(f"unknown backend {backend!r}")
        return losses[backend](rows, weight, targets.reshape(-1))


def lm_head_flops(tokens, cfg=None):
    """(forward, backward) GEMM flops: the log-sum-exp pass; the d_logits
    pass plus d_hidden and d_weight."""
    cfg = cfg or HeadConfig()
    unit = 2.0 * tokens * cfg.d_model * cfg.vocab
    return unit, 3 * unit


# ---------------------------------------------------------------------------
# Harnesses (LM:338-590)
def _online_lse(x, tile):
    """Row log-sum-exp by the running (max, sum) recurrence over column tiles,
    the recurrence the kernel's partials and their combine carry out."""
    run_max = torch.full(x.shape[:1], float("-inf"), dtype=x.dtype)
    run_sum = torch.zeros(x.shape[:1], dtype=x.dtype)
    for block in x.split(tile, dim=1):
        new_max = torch.maximum(run_max, block.amax(dim=1))
        run_sum = run_sum * (run_max - new_max).exp() + (block - new_max[:, None]).exp().sum(dim=1)
        run_max = new_max
    return run_max + run_sum.log()


def check_math(quiet=False) -> Report:
    """CPU checks (the reference's check(), LM:338-476): memory saved, the
    online log-sum-exp, the loss and gradient identities the kernels use, the
    module's host logic."""
    report = Report("lm head math", quiet=quiet)
    cfg = HeadConfig()
    gen = torch.Generator().manual_seed(0)
    tokens = 8 * 2048

    report.section("memory at 8 x 2048 tokens")
    logits, lse = logits_bytes(tokens, cfg.vocab), tokens * 4
    report.note(f"bf16 logits {logits / 1e9:.2f} GB, fused forward output {lse / 1e3:.0f} KB")
    report.expect("the logits the fused forward never stores exceed 1.5 GB", logits > 1.5e9)
    report.expect("its output is under 1 MB", lse < 1e6)
    report.expect("the default backward chunk (the whole vocabulary) is under 4 GB of d_logits",
                  logits_bytes(tokens, cfg.chunk) < 4e9)

    report.section("log-sum-exp")
    x = torch.randn(48, 6000, generator=gen, dtype=torch.float64) * 10
    err = (_online_lse(x, 256) - torch.logsumexp(x, dim=1)).abs().max().item()
    report.expect("running (max, sum) over 256-column tiles equals logsumexp", err < 1e-11, err)

    report.section("loss and gradient identities")
    z = torch.randn(150, 700, generator=gen, dtype=torch.float64, requires_grad=True)
    t = torch.randint(0, 700, (150,), generator=gen)
    loss = F.cross_entropy(z, t)
    by_lse = (torch.logsumexp(z, dim=1) - z.gather(1, t[:, None])[:, 0]).mean()
    report.expect("cross-entropy = mean(lse - target logit)", (loss - by_lse).abs().item() < 1e-12)
    (dz,) = torch.autograd.grad(loss, z)
    closed = (torch.softmax(z.detach(), dim=1) - F.one_hot(t, 700).double()) / 150
    report.expect("d loss / d logits = (softmax - onehot) / tokens", (dz - closed).abs().max().item() < 1e-12)

    report.section("host logic")
    h, w = torch.randn(5, 4, generator=gen), torch.randn(4, 9, generator=gen)
    t = torch.tensor([8, 0, 3, 3, 5])
    report.expect("gather_target_logits picks each row's target logit",
                  torch.allclose(gather_target_logits(h, w, t), (h @ w)[torch.arange(5), t]))
    emb = nn.Embedding(cfg.vocab, cfg.d_model)
    head = LMHead(cfg, emb)
    report.expect("a tied head owns no parameters", sum(p.numel() for p in head.parameters()) == 0)
    report.expect("and reads the embedding's own storage", head.matrix().data_ptr() == emb.weight.data_ptr())
    report.expect("default logit scale 1/sqrt(d_model)", cfg.logit_scale == cfg.d_model ** -0.5)
    return report.finish()


def check_gpu(tokens=4096, quiet=False) -> Report:
    """The fused head against fp32 torch on the GPU (the reference's
    check_gpu, LM:479-520): the log-sum-exp kernel, the loss, and both
    gradients (gate max|d| / max|ref| < 3e-2).  hidden ~ N(0, 0.1^2),
    weight ~ N(0, 0.02^2), uniform targets, seed 0."""
    report = Report("lm head gpu", quiet=quiet)
    if not needs_gpu("check_gpu"):
        return report
    cfg = HeadConfig()
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    hidden = (torch.randn(tokens, cfg.d_model, device=dev, generator=gen) * 0.1).to(DTYPE)
    weight = (torch.randn(cfg.d_model, cfg.vocab, device=dev, generator=gen) * 0.02).to(DTYPE)
    targets = torch.randint(0, cfg.vocab, (tokens,), device=dev, generator=gen)
    logits = hidden.float() @ weight.float()

    report.section(f"log-sum-exp kernel, {tokens} tokens x {cfg.vocab}")
    err = (get_kernel((tokens, cfg.d_model, cfg.vocab))(hidden, weight) - torch.logsumexp(logits, dim=1)).abs().max()
    report.expect("lse max-abs < 5e-3", err.item() < 5e-3, err.item())

    report.section("fused_cross_entropy forward + backward")
    leaves = [hidden.clone().requires_grad_(True), weight.clone().requires_grad_(True)]
    loss = fused_cross_entropy(*leaves, targets)
    got = torch.autograd.grad(loss, leaves)
    exact = [hidden.float().requires_grad_(True), weight.float().requires_grad_(True)]
    ref = F.cross_entropy(exact[0] @ exact[1], targets)
    want = torch.autograd.grad(ref, exact)
    gap = abs(loss.item() - ref.item())
    report.expect("loss within 1e-3 of fp32", gap < 1e-3, gap)
    for name, a, b in zip(("d_hidden", "d_weight"), got, want):
        e = compare(a, b)
        report.expect(f"{name}: max|d|/max|ref| < 3e-2", e["finite"] and e["max_rel"] < 3e-2, e["max_rel"])
        report.note(f"{name}: rel-L2 {e['rel_l2']:.3e}")
    return report.finish()


def benchmark(tokens=16384, quiet=False) -> dict:
    """fwd + bwd of the fused head and of fp32 torch logits + cross-entropy
    (the reference's benchmark, LM:523-572), HIP-event timed.  Returns
    {name: ms}."""
    if not needs_gpu("benchmark"):
        return {}
    cfg = HeadConfig()
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    hidden = (torch.randn(tokens, cfg.d_model, device=dev, generator=gen) * 0.1).to(DTYPE).requires_grad_(True)
    weight = (torch.randn(cfg.d_model, cfg.vocab, device=dev, generator=gen) * 0.02).to(DTYPE).requires_grad_(True)
    targets = torch.randint(0, cfg.vocab, (tokens,), device=dev, generator=gen)
    steps = {
        "fused": lambda: torch.autograd.grad(fused_cross_entropy(hidden, weight, targets), (hidden, weight)),
        "torch fp32": lambda: torch.autograd.grad(F.cross_entropy(hidden.float() @ weight.float(), targets),
                                                  (hidden, weight)),
    }
    ms = {name: time_cuda(step, warmup=5, iters=20) for name, step in steps.items()}
    if not quiet:
        fwd, bwd = lm_head_flops(tokens, cfg)
        for name, t in sorted(ms.items(), key=lambda kv: kv[1]):
            print(f"  {name:10s} {t:8.3f} ms  {(fwd + bwd) / t * 1e-9:7.1f} TFLOP/s")
    return ms


def tune(tokens=16384):
    """The gfx950 build compiles one tiling (the reference autotunes
    TileLang's space, LM:575-590): list it."""
    print(f"lse: {len(lse_configs())} tiling(s): {lse_configs()}")
    return {"lse": lse_configs()}


if __name__ == "__main__":
    sys.exit(harness_main("mimansm1_v1_amd.lm_head",
                          {"check": check_math, "gpu": check_gpu, "bench": benchmark, "tune": tune}))
