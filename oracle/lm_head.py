"""CPU oracle for the fused cross-entropy head -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline
may import this module, and only as the checker; the product path
(``mimansm1_v1_amd``) never calls it.

What it restates (citations to /root/reference/CODE/mimans/model/lm_head_tilelang.py):

* ``lse(hidden, weight)`` -- the log-sum-exp kernel's output (:92-156):
  log sum_v exp(hidden . weight[:, v]) over fp32 logits of the bf16 inputs.
* ``target_logits(hidden, weight, targets)`` -- gather_target_logits
  (:186-190): the target column's dot product in fp32 (ignored targets
  clamped to 0, as the reference does).
* ``loss(hidden, weight, targets, ignore_index)`` -- FusedCrossEntropy.forward
  (:193-209): sum over valid tokens of (lse - target_logit) / max(count, 1).
* ``dlogits(hidden, weight, targets, lse, scale, ignore_index)`` -- the
  per-chunk ``probs`` of FusedCrossEntropy.backward (:226-238):
  (exp(logits - lse) - onehot) * mask * scale, in fp32.
* ``grads(hidden, weight, targets, ignore_index)`` -- d_hidden, d_weight by
  autograd of the fp32 F.cross_entropy(reduction sum) / count (the torch
  backend of LMHead.forward, :326-334; what check_gpu compares against).
* ``online_lse(x, block)`` -- the kernel's online recurrence (running max and
  rescaled sum over vocabulary tiles, :133-151), as the reference's own check
  writes it (:393-406).

How it is pinned (tests/test_oracle.py): ``online_lse`` and ``lse`` against
torch.logsumexp (a library routine) in fp64 (< 1e-12, the reference's check);
``loss`` against F.cross_entropy with ignore_index; ``dlogits`` against
autograd of F.cross_entropy (the reference's gradient identity, :420-428) in
fp64; planted mistakes (a dropped one-hot, the mean over all tokens instead
of the valid ones) fail.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

IGNORE_INDEX = -100


def logits(hidden, weight, dtype=torch.float32):
    return hidden.to(dtype) @ weight.to(dtype)


def online_lse(x, block=128):
    m = torch.full(x.shape[:1], float("-inf"), dtype=x.dtype)
    s = torch.zeros(x.shape[:1], dtype=x.dtype)
    for start in range(0, x.shape[1], block):
        tile = x[:, start:start + block]
        prev = m.clone()
        m = torch.maximum(m, tile.max(dim=1).values)
        s = s * torch.exp(prev - m) + torch.exp(tile - m.unsqueeze(1)).sum(1)
    return torch.log(s) + m


def lse(hidden, weight, dtype=torch.float32):
    return torch.logsumexp(logits(hidden, weight, dtype), dim=-1)


def target_logits(hidden, weight, targets, dtype=torch.float32):
    valid = targets.clamp(min=0)
    rows = weight.index_select(1, valid).t()
    return (hidden.to(dtype) * rows.to(dtype)).sum(-1)


def loss(hidden, weight, targets, ignore_index=IGNORE_INDEX, dtype=torch.float32):
    mask = targets != ignore_index
    count = mask.sum().clamp(min=1)
    per_token = torch.where(mask, lse(hidden, weight, dtype) - target_logits(hidden, weight, targets, dtype),
                            torch.zeros((), dtype=dtype))
    return per_token.sum() / count


def dlogits(hidden, weight, targets, lse_, scale, ignore_index=IGNORE_INDEX, dtype=torch.float32):
    lg = logits(hidden, weight, dtype)
    probs = torch.exp(lg - lse_.to(dtype).unsqueeze(1))
    mask = targets != ignore_index
    rows = torch.arange(lg.shape[0])
    probs[rows[mask], targets[mask]] -= 1.0
    return probs * mask.unsqueeze(1).to(dtype) * scale


def grads(hidden, weight, targets, ignore_index=IGNORE_INDEX, dtype=torch.float32):
    """(loss, d_hidden, d_weight) by autograd through the fp32 torch path."""
    h = hidden.detach().to(dtype).requires_grad_(True)
    w = weight.detach().to(dtype).requires_grad_(True)
    count = (targets != ignore_index).sum().clamp(min=1)
    out = F.cross_entropy(h @ w, targets, ignore_index=ignore_index, reduction="sum") / count
    out.backward()
    return out.detach(), h.grad, w.grad


def make_inputs(tokens, d_model=1280, vocab=49152, seed=0, h_std=0.1, w_std=0.02, n_ignore=0):
    """Seeded CPU inputs: hidden [T, d] bf16 ~ N(0, h_std^2), weight [d, V]
    bf16 ~ N(0, w_std^2) (the reference check's scales, :435-437), targets
    uniform in [0, V) with the first n_ignore set to ignore_index."""
    gen = torch.Generator().manual_seed(seed)
    hidden = (torch.randn(tokens, d_model, generator=gen) * h_std).to(torch.bfloat16)
    weight = (torch.randn(d_model, vocab, generator=gen) * w_std).to(torch.bfloat16)
    targets = torch.randint(0, vocab, (tokens,), generator=gen)
    targets[:n_ignore] = IGNORE_INDEX
    return hidden, weight, targets
