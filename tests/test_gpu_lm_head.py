"""Fused cross-entropy head HIP kernels vs the oracle on identical seeded bf16
inputs (GPU only).

Gates: lse and the per-token loss (fp32, accumulation order the only
difference) within 2e-3 absolute of the fp32 oracle; the target logit
within 1e-3; bf16 d_logits within one bf16 ulp of the oracle's fp32 value
(plus 1e-6 of the largest magnitude for values near zero); the fused op's
loss within 2e-3 and its gradients with the reference harness's own gate,
max|d| / max|ref| < 3e-2 (lm_head_tilelang.py:514-519), plus relative L2
<= 1e-2."""
from __future__ import annotations

import sys

import pytest
import torch
import torch.nn.functional as F

from oracle import lm_head as LMO

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


SHAPES = [(300, 1280, 49152), (256, 128, 384), (1, 256, 128), (777, 384, 1280)]


@pytest.mark.parametrize("T,d,V", SHAPES, ids=[f"T{t}d{d}V{v}" for t, d, v in SHAPES])
def test_lse_target_logit_and_loss_vs_oracle(hip_device, T, d, V):
    from mimansm1_v1_amd import lm_head as L
    log(f"[case] lse T={T} d={d} V={V}")
    h, w, t = LMO.make_inputs(T, d, V, seed=T + V, h_std=1.0, w_std=0.05, n_ignore=min(5, T - 1))
    hd, wd, td = h.to(hip_device), w.to(hip_device), t.to(hip_device)
    kern = L.get_kernel((T, d, V))
    lse, tl, loss = kern.forward(hd, wd, td)
    lse_only = kern(hd, wd)
    torch.cuda.synchronize()
    want_lse = LMO.lse(h, w)
    want_tl = LMO.target_logits(h, w, t)
    mask = t != LMO.IGNORE_INDEX
    want_loss = torch.where(mask, want_lse - want_tl, torch.zeros(()))
    e_lse = (lse.cpu() - want_lse).abs().max().item()
    e_tl = (tl.cpu() - want_tl).abs().max().item()     # ignored tokens: column 0, as the oracle's clamp
    e_loss = (loss.cpu() - want_loss).abs().max().item()
    log(f"    lse {e_lse:.2e}  target_logit {e_tl:.2e}  loss {e_loss:.2e}")
    assert e_lse < 2e-3 and e_tl < 1e-3 and e_loss < 2e-3
    assert torch.equal(lse_only.cpu(), lse.cpu())
    assert (loss.cpu()[~mask] == 0).all()


@pytest.mark.parametrize("T,d,V,v0,vn", [(300, 1280, 49152, 0, 49152), (300, 1280, 49152, 8192, 4096),
                                         (129, 256, 384, 128, 256)])
def test_dlogits_vs_oracle(hip_device, T, d, V, v0, vn):
    from mimansm1_v1_amd import lm_head as L
    log(f"[case] dlogits T={T} d={d} V={V} chunk [{v0}, {v0 + vn})")
    h, w, t = LMO.make_inputs(T, d, V, seed=7 + T, h_std=1.0, w_std=0.05, n_ignore=3)
    t[10] = v0 + 5                      # some targets inside the chunk
    t[11] = v0 + vn - 1
    hd, wd, td = h.to(hip_device), w.to(hip_device), t.to(hip_device)
    kern = L.get_kernel((T, d, V))
    lse, _, _ = kern.forward(hd, wd, td)
    scale = torch.tensor([0.5], device=hip_device)
    out = kern.dlogits(hd, wd, td, lse, scale, v0, vn)
    torch.cuda.synchronize()
    want = LMO.dlogits(h, w, t, lse.cpu(), 0.5)[:, v0:v0 + vn]
    g, wv = out.cpu().double(), want.double()
    ulp = torch.pow(2.0, torch.floor(torch.log2(wv.abs().clamp(min=2.0 ** -126)))) * 2.0 ** -7
    bad = (g - wv).abs() > ulp + 1e-6 * wv.abs().max()
    log(f"    max_abs {(g - wv).abs().max().item():.3e}  beyond 1 ulp: {int(bad.sum())}")
    assert not bad.any()
    assert (out.cpu()[:3] == 0).all()    # ignored tokens


@pytest.mark.parametrize("T,V,chunk", [(512, 49152, 49152), (512, 49152, 8192), (200, 1280, 256)])
def test_fused_cross_entropy_vs_fp32_reference(hip_device, T, V, chunk):
    from mimansm1_v1_amd import lm_head as L
    log(f"[case] fused CE T={T} V={V} chunk={chunk}")
    h, w, t = LMO.make_inputs(T, 1280, V, seed=T, n_ignore=8)
    hd = h.to(hip_device).requires_grad_(True)
    wd = w.to(hip_device).requires_grad_(True)
    td = t.to(hip_device)
    loss = L.fused_cross_entropy(hd, wd, td, chunk)
    loss.backward()
    want_loss, want_dh, want_dw = LMO.grads(h.to(hip_device), w.to(hip_device), td)
    e = abs(loss.item() - want_loss.item())
    log(f"    loss {loss.item():.6f} vs {want_loss.item():.6f} ({e:.1e})")
    assert e < 2e-3
    for name, a, b in (("d_hidden", hd.grad, want_dh), ("d_weight", wd.grad, want_dw)):
        a, b = a.float().cpu(), b.float().cpu()
        rel = ((a - b).abs().max() / b.abs().max()).item()
        l2 = ((a - b).norm() / b.norm()).item()
        log(f"    {name:9s} max|d|/max|ref| {rel:.3e}  rel_l2 {l2:.3e}")
        assert rel < 3e-2 and l2 < 1e-2, name


def test_all_ignored_and_lm_head_module(hip_device):
    from mimansm1_v1_amd import lm_head as L
    log("[case] all ignored; LMHead hip vs torch backends")
    h, w, t = LMO.make_inputs(64, 1280, 1280, seed=2)
    hd, wd = h.to(hip_device), w.to(hip_device)
    ign = torch.full((64,), LMO.IGNORE_INDEX, device=hip_device)
    assert L.fused_cross_entropy(hd, wd, ign).item() == 0.0
    torch.manual_seed(0)
    cfg = L.HeadConfig(vocab=2048)
    emb = torch.nn.Embedding(cfg.vocab, cfg.d_model).to(hip_device)
    head = L.LMHead(cfg, emb)
    x = torch.randn(2, 50, cfg.d_model, device=hip_device)
    targets = torch.randint(0, cfg.vocab, (2, 50), device=hip_device)
    targets[0, :4] = L.IGNORE_INDEX
    got = head(x, targets, backend="hip")
    alias = head(x, targets, backend="tilelang")
    want = head(x, targets, backend="torch")
    log(f"    loss hip {got.item():.6f} torch {want.item():.6f}")
    assert abs(got.item() - want.item()) < 1e-2
    assert got.item() == alias.item()


def test_fused_cross_entropy_deterministic(hip_device):
    from mimansm1_v1_amd import lm_head as L
    log("[case] fused CE determinism")
    h, w, t = (x.to(hip_device) for x in LMO.make_inputs(300, 1280, 4096, seed=9, n_ignore=2))
    runs = []
    for _ in range(2):
        hd, wd = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
        loss = L.fused_cross_entropy(hd, wd, t, 1024)
        loss.backward()
        runs.append((loss.item(), hd.grad.cpu(), wd.grad.cpu()))
    assert runs[0][0] == runs[1][0]
    assert torch.equal(runs[0][1], runs[1][1]) and torch.equal(runs[0][2], runs[1][2])
