"""CPU oracle for the SwiGLU feed-forward kernels -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline
may import this module, and only as the checker; the product path
(``mimansm1_v1_amd``) never calls it.

What it restates (citations to /root/reference/CODE/mimans/model/swiglu_tilelang.py):

* ``act_fused(x, wg, wu)`` -- gate_up_swiglu (:119-156): gate and up
  accumulated in fp32, act = bf16(gate / (1 + exp(-gate)) * up) (:151-152).
* ``split(x, wg, wu)`` -- gate_up_split (:158-200): bf16(gate), bf16(up)
  from the fp32 accumulators (:189-198).
* ``act_train(gate, up)`` -- FusedSwiGLU.forward's ``F.silu(gate) * up`` on
  the bf16 gate and up (:283-284): the silu rounded to bf16, then the product
  rounded to bf16 (torch's bf16 tensor ops compute in fp32 and round).
* ``grad(d_act, gate, up)`` -- swiglu_grad (:202-240): bf16 inputs read into
  fp32, s = sigmoid(g), dGate = bf16(dA u s (1 + g (1 - s))),
  dUp = bf16(dA g s) (:226-236).
* ``reference(x, wg, wu, wd)`` -- the module's fp32 reference (:362-365):
  (silu(x wg) * (x wu)) wd in fp32.
* ``grads(x, wg, wu, wd, grad_out)`` -- dX, dWg, dWu, dWd by autograd through
  ``reference`` in fp32 (what check_gpu compares against, :537-547).
* ``manual_grads(...)`` -- the same gradients from FusedSwiGLU.backward's
  formulas (:288-301) in any dtype, used to pin ``grads`` in fp64.

How it is pinned (tests/test_oracle.py): the silu derivative against
autograd in fp64 and its closed values at 0 (the reference's own checks,
:413-424); ``manual_grads`` against fp64 autograd of ``reference`` (the
reference's :426-462 check, < 1e-10); ``act_train`` against the explicit
rounding sequence; ``split`` / ``act_fused`` against a float64 product
rounded once; a planted mistake (a dropped (1 + g(1 - s)) factor) fails.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _gemm32(x, w):
    return x.float() @ w.float()


def act_fused(x, wg, wu):
    g, u = _gemm32(x, wg), _gemm32(x, wu)
    return (g / (1.0 + torch.exp(-g)) * u).to(torch.bfloat16)


def split(x, wg, wu):
    return _gemm32(x, wg).to(torch.bfloat16), _gemm32(x, wu).to(torch.bfloat16)


def act_train(gate, up):
    """F.silu(gate) * up on bf16 tensors, written as its rounding steps."""
    s = F.silu(gate.float()).to(torch.bfloat16)
    return (s.float() * up.float()).to(torch.bfloat16)


def grad(d_act, gate, up):
    a, g, u = d_act.float(), gate.float(), up.float()
    s = torch.sigmoid(g)
    d_gate = a * u * s * (1.0 + g * (1.0 - s))
    d_up = a * g * s
    return d_gate.to(torch.bfloat16), d_up.to(torch.bfloat16)


def reference(x, wg, wu, wd):
    gate = x.float() @ wg.float()
    up = x.float() @ wu.float()
    return ((gate * torch.sigmoid(gate)) * up) @ wd.float()


def grads(x, wg, wu, wd, grad_out, dtype=torch.float32):
    """(out, dX, dWg, dWu, dWd) by autograd through ``reference`` in `dtype`."""
    leaves = [t.detach().to(dtype).requires_grad_(True) for t in (x, wg, wu, wd)]
    g = leaves[0] @ leaves[1]
    u = leaves[0] @ leaves[2]
    out = ((g * torch.sigmoid(g)) * u) @ leaves[3]
    out.backward(grad_out.to(dtype))
    return (out.detach(),) + tuple(t.grad for t in leaves)


def manual_grads(x, wg, wu, wd, grad_out):
    """FusedSwiGLU.backward's formulas (:288-301) in the inputs' dtype."""
    gate, up = x @ wg, x @ wu
    act = F.silu(gate) * up
    d_act = grad_out @ wd.t()
    s = torch.sigmoid(gate)
    d_gate = d_act * up * s * (1 + gate * (1 - s))
    d_up = d_act * F.silu(gate)
    return (d_gate @ wg.t() + d_up @ wu.t(), x.t() @ d_gate, x.t() @ d_up, act.t() @ grad_out)


def make_inputs(tokens, d_model=1280, ffn=3328, seed=0, std=0.02):
    """Seeded CPU inputs (x, wg, wu, wd, grad_out) in bf16: x, grad_out ~ N(0,1),
    weights ~ N(0, std^2) (the check's recipe, :521-530)."""
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, d_model, generator=gen)
    wg = torch.randn(d_model, ffn, generator=gen) * std
    wu = torch.randn(d_model, ffn, generator=gen) * std
    wd = torch.randn(ffn, d_model, generator=gen) * std
    go = torch.randn(tokens, d_model, generator=gen)
    return tuple(t.to(torch.bfloat16) for t in (x, wg, wu, wd, go))
