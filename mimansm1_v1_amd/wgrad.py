"""Weight gradients dW = A^T B of the bf16 projections around the attention
and the SwiGLU feed-forward, over all tokens.

A GEMM whose reduction runs over the B*S tokens (16,384 at the training
shapes) but whose output is only a weight's size (1792 x 1280 for wq|wk|wv,
3328 x 1280 for w_down) has too few output tiles to fill 256 CUs.  Splitting
the tokens into chunks gives hipBLASLt a batched GEMM with `chunks` times the
tiles; the chunks' products come out in fp32 and are summed in fp32, so the
result is the same sum as one GEMM, rounded once at the end (measured on
MI355X: wq|wk|wv 157 -> 110 + 15 us with 8 chunks, w_down 271 -> 174 us with
2 chunks).  hipBLASLt's own GEMM runs on any other shape.
"""
from __future__ import annotations

import torch


def wgrad(a: torch.Tensor, b: torch.Tensor, chunks: int) -> torch.Tensor:
    """sum over tokens t of a[t]^T b[t] in fp32: a [T, M], b [T, N] -> [M, N]
    fp32.  Splits T into `chunks` when it divides evenly into chunks of at
    least 64 tokens; else one GEMM with fp32 output."""
    t, m = a.shape
    n = b.shape[1]
    if chunks > 1 and t % chunks == 0 and t >= 64 * chunks:
        return torch.bmm(a.reshape(chunks, t // chunks, m).transpose(1, 2),
                         b.reshape(chunks, t // chunks, n).contiguous(),
                         out_dtype=torch.float32).sum(0)
    return torch.mm(a.t(), b, out_dtype=torch.float32)
