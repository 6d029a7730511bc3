"""CPU oracle for the causal GQA flash-attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker or the timed CPU
baseline; the product path (``mimansm1_v1_amd``) never calls it.

What it restates (all citations are to /root/reference):

* ``attention(q, k, v, causal, groups)`` -- the fp32 reference attention of
  CODE/mimans/model/attention_tilelang.py:521-530 (K/V repeated per group,
  scores / sqrt(D), causal mask incl. the diagonal, softmax, P V, cast to
  q.dtype).
* ``lse2(q, k, causal, groups)`` -- the log-sum-exp the forward kernel stores,
  in log2 units: lse2 = log2(l) + m * log2(e)/sqrt(D)  (AT:114, :186-188), i.e.
  log2(e) * logsumexp_j(q.k_j / sqrt(D)).
* ``delta(o, do)`` -- Delta = rowsum(O * dO) in fp32 (AT:212-214).
* ``grads(q, k, v, do, causal, groups)`` -- dQ, dK, dV by autograd through
  ``attention`` (the method of AT:654-656).
* ``grads_analytic(...)`` -- the same gradients from the closed-form
  softmax-attention backward, computed per (batch, head) chunk so that the
  full-size configs fit (usable on a GPU device for the large parity tests);
  with ``bf16_products=True`` the reference kernel's bf16 rounding points
  (P before dV, dS * sm_scale before dK / dQ, Delta from the bf16 output O).
* ``rope(x, theta)`` -- explicit pairwise rotation (AT:533-541).
* ``rope_tables``, ``rmsnorm``, ``apply_rope``, ``qknorm_rope`` -- the
  sublayer prologue (config 5): the Rotary cos/sin tables (AT:438-444), the
  QK-RMSNorm in fp32 cast back to the input dtype (AT:423-428), the
  rotate-half RoPE in the input dtype with the tables cast to it (AT:452-461),
  applied to the wq | wk | wv outputs as Attention.forward does (AT:483-487).
* ``make_inputs(config)`` -- the seeded input recipe of BASELINE.json configs
  1-5: CPU ``torch.Generator().manual_seed(seed)``, draws in the order Q, K, V,
  dO (config 4 adds per-head sigma ~ U(0.5, 3) and RoPE in fp32 before the
  bf16 cast).

How it is pinned (tests/test_oracle.py): against the plain-C fp64 brute force
in ``oracle/brute_attn.c`` (forward, lse2, an independent derivation of the
backward, Delta through the identity rowsum(O * dO) = sum_j P_ij dP_ij, and
the backward with the reference kernel's bf16 rounding points, which pins
``grads_analytic(bf16_products=True)``), against torch's
``scaled_dot_product_attention`` (a library
routine), against closed forms (S=1, constant V, constant K, lse2 lower bound)
and invariants (causal no-leak, batch permutation, identical heads), and
against the committed fixtures in ``tests/golden/``.  No function here is left
"parity unpinned".
"""
from __future__ import annotations

import math

import torch

LOG2E = 1.4426950408889634


def _expand_kv(t: torch.Tensor, groups: int) -> torch.Tensor:
    # [B,S,Hkv,D] -> [B,S,H,D]; query head h reads KV head h // groups (AT:523-524)
    return t.repeat_interleave(groups, dim=2)


def scores(q, k, causal, groups, dtype=torch.float32):
    """[B,H,Sq,Sk] scaled scores with -inf above the diagonal when causal."""
    dim = q.size(-1)
    qh = q.to(dtype).permute(0, 2, 1, 3)                               # b h i d
    kh = _expand_kv(k.to(dtype), groups).permute(0, 2, 3, 1).contiguous()  # b h d j
    s = torch.matmul(qh, kh) / math.sqrt(dim)
    if causal:
        n = q.size(1)
        keep = torch.ones(n, n, dtype=torch.bool, device=q.device).tril()
        s = s.masked_fill(~keep, float("-inf"))
    return s


def attention(q, k, v, causal, groups, dtype=torch.float32, cast=True):
    """Reference attention (AT:521-530); returns [B,S,H,D] in q.dtype when cast."""
    p = scores(q, k, causal, groups, dtype).softmax(-1)
    vh = _expand_kv(v.to(dtype), groups).permute(0, 2, 1, 3).contiguous()
    out = torch.matmul(p, vh).permute(0, 2, 1, 3)
    return out.to(q.dtype) if cast else out


def lse2(q, k, causal, groups, dtype=torch.float32):
    """[B,H,S] log2-unit log-sum-exp of the scaled scores (AT:186-188)."""
    return torch.logsumexp(scores(q, k, causal, groups, dtype), dim=-1) * LOG2E


def delta(o, do):
    """[B,H,S] fp32 rowsum(O * dO) (AT:212-214)."""
    return (o.float() * do.float()).sum(-1).permute(0, 2, 1).contiguous()


def grads(q, k, v, do, causal, groups, dtype=torch.float32):
    """(dq, dk, dv) in `dtype` by autograd through `attention` (AT:654-656)."""
    qf, kf, vf = (t.detach().to(dtype).requires_grad_(True) for t in (q, k, v))
    out = attention(qf, kf, vf, causal, groups, dtype, cast=False)
    out.backward(do.to(dtype))
    return qf.grad, kf.grad, vf.grad


@torch.no_grad()
def forward_chunked(q, k, v, causal, groups, dtype=torch.float32):
    """(O fp32 [B,S,H,D], lse2 [B,H,S]) computed one (batch, head) at a time."""
    B, S, H, D = q.shape
    out = torch.empty(B, S, H, D, dtype=dtype, device=q.device)
    lse = torch.empty(B, H, S, dtype=dtype, device=q.device)
    keep = torch.ones(S, S, dtype=torch.bool, device=q.device).tril() if causal else None
    for b in range(B):
        for h in range(H):
            g = h // groups
            qh, kh, vh = q[b, :, h].to(dtype), k[b, :, g].to(dtype), v[b, :, g].to(dtype)
            s = torch.matmul(qh, kh.t().contiguous()) / math.sqrt(D)
            if keep is not None:
                s = s.masked_fill(~keep, float("-inf"))
            lse[b, h] = torch.logsumexp(s, dim=-1) * LOG2E
            out[b, :, h] = torch.matmul(s.softmax(-1), vh)
    return out, lse


@torch.no_grad()
def grads_analytic(q, k, v, do, causal, groups, dtype=torch.float32, bf16_products=False):
    """Closed-form backward of softmax attention, one (batch, head) at a time:
        P = softmax(s), dP = dO V^T, Delta_i = sum_j P_ij dP_ij,
        dS = P * (dP - Delta), dQ = dS K / sqrt(D), dK = dS^T Q / sqrt(D),
        dV = P^T dO; dK, dV summed over the query heads of each KV head.
    Returns fp32 (dq, dk, dv).

    bf16_products=True emulates the rounding points of the reference's
    TileLang backward (AT:297-314), everything else in `dtype`: P rounded to
    bf16 before dV = P^T dO (:306-307); dS * sm_scale rounded to bf16 before
    dK and dQ (:310-314); Delta = rowsum(bf16(O) * dO) from this function's
    own forward output O = P V rounded to bf16, as the reference's flash_delta
    reads the forward's bf16 O (:380, :212-214).  The distance of that
    emulation from the exact math is the error the reference's own kernel
    arithmetic costs."""
    B, S, H, D = q.shape
    Hkv = k.shape[2]
    scale = 1.0 / math.sqrt(D)
    dq = torch.zeros(B, S, H, D, dtype=dtype, device=q.device)
    dk = torch.zeros(B, S, Hkv, D, dtype=dtype, device=q.device)
    dv = torch.zeros(B, S, Hkv, D, dtype=dtype, device=q.device)
    keep = torch.ones(S, S, dtype=torch.bool, device=q.device).tril() if causal else None
    for b in range(B):
        for h in range(H):
            g = h // groups
            qh, kh, vh = q[b, :, h].to(dtype), k[b, :, g].to(dtype), v[b, :, g].to(dtype)
            doh = do[b, :, h].to(dtype)
            s = torch.matmul(qh, kh.t().contiguous()) * scale
            if keep is not None:
                s = s.masked_fill(~keep, float("-inf"))
            p = s.softmax(-1)
            dp = torch.matmul(doh, vh.t().contiguous())
            if bf16_products:
                ob = torch.matmul(p, vh).to(torch.bfloat16).to(dtype)
                dlt = (ob * doh).sum(-1, keepdim=True)
                dsb = (p * (dp - dlt) * scale).to(torch.bfloat16).to(dtype)
                pb = p.to(torch.bfloat16).to(dtype)
                dq[b, :, h] = torch.matmul(dsb, kh)
                dk[b, :, g] += torch.matmul(dsb.t().contiguous(), qh)
                dv[b, :, g] += torch.matmul(pb.t().contiguous(), doh)
                continue
            dlt = (p * dp).sum(-1, keepdim=True)
            ds = p * (dp - dlt)
            dq[b, :, h] = torch.matmul(ds, kh) * scale
            dk[b, :, g] += torch.matmul(ds.t().contiguous(), qh) * scale
            dv[b, :, g] += torch.matmul(p.t().contiguous(), doh)
    return dq, dk, dv


def rope(x, theta, dtype=torch.float64):
    """Rotate pairs (x_i, x_{i+D/2}) by angle pos * theta^(-2i/D) (AT:533-541)."""
    B, S, H, D = x.shape
    half = D // 2
    freqs = 1.0 / (theta ** (2 * torch.arange(half, dtype=torch.float64) / D))
    ang = torch.arange(S, dtype=torch.float64)[:, None] * freqs[None, :]
    c = ang.cos().to(dtype).view(1, S, 1, half)
    s = ang.sin().to(dtype).view(1, S, 1, half)
    xd = x.to(dtype)
    lo, hi = xd[..., :half], xd[..., half:]
    return torch.cat([lo * c - hi * s, lo * s + hi * c], dim=-1)


def rope_tables(head_dim, max_seq_len, theta):
    """fp32 cos/sin tables [max_seq_len, head_dim], halves repeated (AT:438-444)."""
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    angles = torch.outer(torch.arange(max_seq_len).float(), freqs)
    table = torch.cat((angles, angles), dim=-1)
    return table.cos(), table.sin()


def rmsnorm(x, w, eps):
    """x * rsqrt(mean(x^2) + eps) * w in fp32, cast back to x.dtype (AT:423-428)."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (xf * w.float()).to(x.dtype)


def rotate_half(x):
    left, right = x.chunk(2, dim=-1)
    return torch.cat((-right, left), dim=-1)


def apply_rope(x, cos, sin):
    """x * cos + rotate_half(x) * sin with the tables cast to x.dtype (AT:452-461)."""
    seq_len = x.shape[1]
    c = cos[:seq_len].to(x.dtype).unsqueeze(1)
    s = sin[:seq_len].to(x.dtype).unsqueeze(1)
    return x * c + rotate_half(x) * s


def qknorm_rope(qkv, wq, wk, cos, sin, heads, kv_heads, eps=1e-5):
    """The attention kernel's inputs from the fused projection qkv
    [B, S, (heads + 2*kv_heads) * D] (columns wq | wk | wv outputs), as
    Attention.forward computes them (AT:483-487); wq = wk = None: no QK-norm."""
    B, S, _ = qkv.shape
    D = qkv.shape[-1] // (heads + 2 * kv_heads)
    q = qkv[..., :heads * D].reshape(B, S, heads, D)
    k = qkv[..., heads * D:(heads + kv_heads) * D].reshape(B, S, kv_heads, D)
    v = qkv[..., (heads + kv_heads) * D:].reshape(B, S, kv_heads, D)
    if wq is not None:
        q, k = rmsnorm(q, wq, eps), rmsnorm(k, wk, eps)
    return apply_rope(q, cos, sin).contiguous(), apply_rope(k, cos, sin).contiguous(), v.contiguous()


# BASELINE.json configs (index = position in its "configs" list + 1).
CONFIGS = {
    1: dict(batch=1, seq=512, heads=10, kv_heads=2, dim=128, bwd=False),
    2: dict(batch=8, seq=2048, heads=10, kv_heads=2, dim=128, bwd=True),
    3: dict(batch=2, seq=8192, heads=10, kv_heads=2, dim=128, bwd=True),
    4: dict(batch=4, seq=4096, heads=10, kv_heads=2, dim=128, bwd=True, rope_sigma=True),
}


def make_inputs(batch, seq, heads=10, kv_heads=2, dim=128, seed=0, rope_sigma=False,
                dtype=torch.bfloat16, **_):
    """Seeded CPU inputs (q, k, v, do) in `dtype`; draws Q, K, V, dO in order.
    With rope_sigma (config 4): sigma ~ U(0.5, 3) per query head and per KV head
    (drawn after dO), Q and K scaled by it and rotated by RoPE base 10000 at
    positions 0..S-1 in fp32, then cast."""
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, seq, heads, dim, generator=gen)
    k = torch.randn(batch, seq, kv_heads, dim, generator=gen)
    v = torch.randn(batch, seq, kv_heads, dim, generator=gen)
    do = torch.randn(batch, seq, heads, dim, generator=gen)
    if rope_sigma:
        sq = torch.empty(heads).uniform_(0.5, 3.0, generator=gen)
        sk = torch.empty(kv_heads).uniform_(0.5, 3.0, generator=gen)
        q = rope(q * sq.view(1, 1, heads, 1), 10_000.0, torch.float32)
        k = rope(k * sk.view(1, 1, kv_heads, 1), 10_000.0, torch.float32)
    return tuple(t.to(dtype) for t in (q, k, v, do))


def config_inputs(config, seed=0, batch=None, dtype=torch.bfloat16):
    c = dict(CONFIGS[config])
    if batch is not None:
        c["batch"] = batch
    return make_inputs(seed=seed, dtype=dtype, **c)
