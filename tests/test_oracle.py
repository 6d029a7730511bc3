"""Pins the CPU oracle (oracle/reference.py) -- no GPU.

Each restated function is checked against something that does not share its
code: the fp64 C brute force (oracle/brute_attn.c, direct loops and a chain-
rule backward), torch's scaled_dot_product_attention, closed forms and
invariants, and the committed fixtures.  The last group plants mistakes in the
oracle and shows the pins catch them."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle import reference as R
from tests.golden.make_golden import CASES, load_cases

SHAPES = [  # (B, S, H, Hkv)
    (1, 1, 10, 2),
    (2, 7, 10, 2),
    (1, 19, 4, 4),
    (2, 13, 6, 3),
    (1, 24, 8, 1),
]


def _np(t):
    return t.detach().double().numpy()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_forward_and_lse_match_brute_force(shape, causal):
    B, S, H, Hkv = shape
    q, k, v, _ = R.make_inputs(B, S, H, Hkv, 128, seed=S, dtype=torch.float64)
    o_ref, lse_ref = brute.fwd(_np(q), _np(k), _np(v), causal)
    o = R.attention(q, k, v, causal, H // Hkv, torch.float64)
    lse = R.lse2(q, k, causal, H // Hkv, torch.float64)
    assert np.abs(_np(o) - o_ref).max() < 1e-12
    assert np.abs(_np(lse) - lse_ref).max() < 1e-12
    o_c, lse_c = R.forward_chunked(q, k, v, causal, H // Hkv, torch.float64)
    assert np.abs(_np(o_c) - o_ref).max() < 1e-12
    assert np.abs(_np(lse_c) - lse_ref).max() < 1e-12


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_gradients_match_brute_force(shape, causal):
    B, S, H, Hkv = shape
    q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=S + 1, dtype=torch.float64)
    want = brute.bwd(_np(q), _np(k), _np(v), _np(do), causal)
    for got in (R.grads(q, k, v, do, causal, H // Hkv, torch.float64),
                R.grads_analytic(q, k, v, do, causal, H // Hkv, torch.float64)):
        for g, w in zip(got, want):
            assert np.abs(_np(g) - w).max() < 1e-11


def test_fp32_oracle_close_to_fp64():
    q, k, v, do = R.make_inputs(2, 64, 10, 2, 128, seed=3)
    o64 = R.attention(q, k, v, True, 5, torch.float64, cast=False)
    o32 = R.attention(q, k, v, True, 5, cast=False)
    assert (o32.double() - o64).abs().max() < 1e-5
    for a, b in zip(R.grads(q, k, v, do, True, 5), R.grads(q, k, v, do, True, 5, torch.float64)):
        assert (a.double() - b).abs().max() < 1e-4


@pytest.mark.parametrize("causal", [True, False])
def test_matches_sdpa(causal):
    q, k, v, _ = R.make_inputs(2, 96, 10, 2, 128, seed=4, dtype=torch.float32)
    want = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                          is_causal=causal, enable_gqa=True).transpose(1, 2)
    got = R.attention(q, k, v, causal, 5)
    assert (got - want).abs().max() < 2e-5


def test_single_position_returns_v():
    q, k, v, _ = R.make_inputs(3, 1, 10, 2, 128, seed=5, dtype=torch.float64)
    o = R.attention(q, k, v, True, 5, torch.float64)
    assert torch.equal(o, v.repeat_interleave(5, dim=2))
    # one key: lse2 is the single scaled score in log2 units
    s = (q * k.repeat_interleave(5, dim=2)).sum(-1) / math.sqrt(128) * R.LOG2E
    assert (R.lse2(q, k, True, 5, torch.float64) - s.permute(0, 2, 1)).abs().max() < 1e-12


def test_constant_v_and_constant_k():
    q, k, v, _ = R.make_inputs(1, 40, 10, 2, 128, seed=6, dtype=torch.float64)
    c = torch.full_like(v, 0.75)
    assert (R.attention(q, k, c, True, 5, torch.float64) - 0.75).abs().max() < 1e-14
    # K = 0: every visible score is 0, so O_i is the prefix mean of V and
    # lse2_i = log2(i + 1).
    z = torch.zeros_like(k)
    o = R.attention(q, z, v, True, 5, torch.float64)
    prefix = v.cumsum(1) / torch.arange(1, 41, dtype=torch.float64).view(1, 40, 1, 1)
    assert (o - prefix.repeat_interleave(5, dim=2)).abs().max() < 1e-12
    lse = R.lse2(q, z, True, 5, torch.float64)
    assert (lse - torch.log2(torch.arange(1, 41, dtype=torch.float64))).abs().max() < 1e-12


def test_lse_lower_bound():
    q, k, _, _ = R.make_inputs(2, 50, 10, 2, 128, seed=7, dtype=torch.float64)
    lse = R.lse2(q, k, True, 5, torch.float64)
    smax = R.scores(q, k, True, 5, torch.float64).amax(-1) * R.LOG2E
    assert (lse - smax).min() >= 0


def test_causal_no_leak_and_batch_permutation():
    q, k, v, _ = R.make_inputs(2, 33, 10, 2, 128, seed=8, dtype=torch.float64)
    o = R.attention(q, k, v, True, 5, torch.float64)
    q2, k2, v2 = q.clone(), k.clone(), v.clone()
    q2[:, -1] += 10
    k2[:, -1] -= 3
    v2[:, -1] *= 7
    o2 = R.attention(q2, k2, v2, True, 5, torch.float64)
    assert torch.equal(o[:, :-1], o2[:, :-1])
    perm = torch.tensor([1, 0])
    assert torch.equal(R.attention(q[perm], k[perm], v[perm], True, 5, torch.float64), o[perm])


def test_identical_heads_in_a_group_give_identical_outputs():
    q, k, v, _ = R.make_inputs(1, 20, 10, 2, 128, seed=9, dtype=torch.float64)
    q[:, :, 1] = q[:, :, 0]
    q[:, :, 7] = q[:, :, 0]  # head 7 reads KV head 1: different output
    o = R.attention(q, k, v, True, 5, torch.float64)
    assert torch.equal(o[:, :, 1], o[:, :, 0])
    assert not torch.allclose(o[:, :, 7], o[:, :, 0])


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
def test_delta_identity_against_brute_force(shape, causal):
    """Delta = rowsum(O * dO) (AT:212-214) is pinned by the identity
    sum_d O_id dO_id = sum_j P_ij (dO_i . V_j) = sum_j P_ij dP_ij: R.delta on
    the brute force's own O must give the brute force's sum over keys of
    P * dP, which never forms O."""
    B, S, H, Hkv = shape
    q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=S + 40, dtype=torch.float64)
    o_ref, _ = brute.fwd(_np(q), _np(k), _np(v), causal)
    *_, want = brute.bwd(_np(q), _np(k), _np(v), _np(do), causal, with_delta=True)
    # R.delta accumulates in fp32, as the reference's kernel does: agreement
    # to fp32 accuracy over the 128-term sums
    got = R.delta(torch.from_numpy(o_ref), do)
    assert np.abs(_np(got) - want).max() < 1e-6 * max(1.0, np.abs(want).max()) * 8


def test_delta_identity_catches_planted_mistakes():
    """Plausible mistakes in Delta fail the identity: the wrong operand (O * O),
    the sum over heads instead of head_dim, a dropped transpose to [B, H, S]."""
    q, k, v, do = R.make_inputs(2, 9, 10, 2, 128, seed=44, dtype=torch.float64)
    o_ref, _ = brute.fwd(_np(q), _np(k), _np(v), True)
    *_, want = brute.bwd(_np(q), _np(k), _np(v), _np(do), True, with_delta=True)
    o = torch.from_numpy(o_ref)
    wrong = [
        (o * o).sum(-1).permute(0, 2, 1),                                   # wrong operand
        (o * do).sum(-1).sum(-1, keepdim=True).expand(2, 9, 10).permute(0, 2, 1),   # summed over heads too
        (o * do).sum(-1).reshape(2, 10, 9),                                 # [B,S,H] read as [B,H,S]
    ]
    for w in wrong:
        assert np.abs(_np(w) - want).max() > 1e-3


EMUL_SHAPES = [(1, 1, 10, 2), (2, 7, 10, 2), (1, 19, 4, 4), (2, 13, 6, 3), (1, 24, 8, 1), (1, 48, 10, 2)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", EMUL_SHAPES)
def test_emulated_rounding_matches_brute_force(shape, causal):
    """grads_analytic(bf16_products=True) -- the reference kernel's rounding
    points, whose distance from the exact math the GPU parity gates report
    and allow -- is pinned to the fp64 C brute force with the same rounding
    points (brute_attn_bwd_emul: bf16(P) before dV, bf16(P (dP - Delta)
    sm_scale) before dK / dQ, Delta from bf16(O)).  Both evaluate the values
    they round in fp64, so every rounding decision agrees and the results
    match to fp64 summation order; the emulation is also shown to differ from
    the exact backward (else the pin would not see the rounding points)."""
    B, S, H, Hkv = shape
    q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=S + 60, dtype=torch.float64)
    want = brute.bwd_emul(_np(q), _np(k), _np(v), _np(do), causal)[:3]
    exact = brute.bwd(_np(q), _np(k), _np(v), _np(do), causal)
    got = R.grads_analytic(q, k, v, do, causal, H // Hkv, torch.float64, bf16_products=True)
    for name, g, w, e in zip(("dq", "dk", "dv"), got, want, exact):
        scale = max(1.0, np.abs(w).max())
        assert np.abs(_np(g) - w).max() < 1e-10 * scale, name
        if S > 1:
            assert np.abs(w - e).max() > 1e-5 * scale, name
    # the fp32 evaluation the GPU tests use: the same formulas; near a
    # rounding boundary its fp32 values may round to the other neighbour,
    # which moves a result by about one bf16 ulp of one product term
    got32 = R.grads_analytic(q.float(), k.float(), v.float(), do.float(), causal, H // Hkv,
                             bf16_products=True)
    for name, g, w in zip(("dq", "dk", "dv"), got32, want):
        assert np.abs(_np(g) - w).max() < 1e-2 * max(1.0, np.abs(w).max()), name


def test_emulated_rounding_pin_catches_planted_mistakes():
    """Emulations with a rounding point dropped, moved or added fail the pin
    by orders of magnitude: no bf16 on dS; bf16 of dS before the sm_scale
    product; Delta from the exact O; P rounded for dS as well; dV from the
    unrounded P."""
    B, S, H, Hkv = 1, 48, 10, 2
    q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=99, dtype=torch.float64)
    want = brute.bwd_emul(_np(q), _np(k), _np(v), _np(do), True)[:3]
    scale = 1 / math.sqrt(128)
    bf = lambda t: t.to(torch.bfloat16).double()

    def emul(variant):
        dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
        keep = torch.ones(S, S, dtype=torch.bool).tril()
        for h in range(H):
            g = h // 5
            qh, kh, vh, doh = q[0, :, h], k[0, :, g], v[0, :, g], do[0, :, h]
            p = (qh @ kh.t() * scale).masked_fill(~keep, float("-inf")).softmax(-1)
            dp = doh @ vh.t()
            o = p @ vh
            dlt = ((o if variant == "exact_o" else bf(o)) * doh).sum(-1, keepdim=True)
            pp = bf(p) if variant == "p_rounded" else p
            if variant == "no_ds_round":
                dsb = pp * (dp - dlt) * scale
            elif variant == "round_before_scale":
                dsb = bf(pp * (dp - dlt)) * scale
            else:
                dsb = bf(pp * (dp - dlt) * scale)
            dq[0, :, h] = dsb @ kh
            dk[0, :, g] += dsb.t() @ qh
            dv[0, :, g] += (p if variant == "exact_p_dv" else bf(p)).t() @ doh
        return dq, dk, dv

    def err(got):
        return max(np.abs(_np(g) - w).max() / max(1.0, np.abs(w).max()) for g, w in zip(got, want))

    assert err(emul("reference")) < 1e-10
    for variant in ("no_ds_round", "round_before_scale", "exact_o", "p_rounded", "exact_p_dv"):
        assert err(emul(variant)) > 1e-5, variant


def test_golden_fixtures_reproduce():
    cases = load_cases()
    assert set(cases) == set(CASES)
    for name, c in cases.items():
        B, S, H, Hkv, causal = c["meta"]
        G = H // Hkv
        o = R.attention(c["q"], c["k"], c["v"], causal, G, cast=False)
        assert (o - c["o"]).abs().max() < 1e-5, name
        assert (R.lse2(c["q"], c["k"], causal, G) - c["lse2"]).abs().max() < 1e-5, name
        for got, key in zip(R.grads(c["q"], c["k"], c["v"], c["do"], causal, G), ("dq", "dk", "dv")):
            assert (got - c[key]).abs().max() < 1e-4, (name, key)


def test_config_input_recipe():
    q, k, v, do = R.make_inputs(1, 64, 10, 2, 128, seed=0)
    q2, *_ = R.make_inputs(1, 64, 10, 2, 128, seed=0)
    assert torch.equal(q, q2) and q.dtype == torch.bfloat16
    # config 4: sigma-scaled, RoPE-rotated Q/K; rotation preserves per-vector norms
    qr, kr, _, _ = R.make_inputs(1, 64, 10, 2, 128, seed=0, rope_sigma=True, dtype=torch.float32)
    gen = torch.Generator().manual_seed(0)
    raw_q = torch.randn(1, 64, 10, 128, generator=gen)
    ratio = qr.norm(dim=-1) / raw_q.norm(dim=-1)
    per_head = ratio.mean(dim=(0, 1))
    assert (ratio - per_head).abs().max() < 1e-4      # one sigma per head
    assert per_head.min() >= 0.5 and per_head.max() <= 3.0


def test_rope_matches_rotation_of_pairs():
    x = torch.randn(1, 12, 2, 128, dtype=torch.float64)
    y = R.rope(x, 10_000.0)
    i, pos = 5, 9
    ang = pos * 10_000.0 ** (-2 * i / 128)
    a, b = x[0, pos, 0, i], x[0, pos, 0, i + 64]
    assert abs(y[0, pos, 0, i] - (a * math.cos(ang) - b * math.sin(ang))) < 1e-12
    assert abs(y[0, pos, 0, i + 64] - (a * math.sin(ang) + b * math.cos(ang))) < 1e-12


# ---------------------------------------------------------------------------
# Planted mistakes: a wrong oracle must fail the pins above.
def test_planted_wrong_gqa_mapping_is_caught(monkeypatch):
    q, k, v, _ = R.make_inputs(1, 9, 10, 2, 128, seed=11, dtype=torch.float64)
    o_ref, _ = brute.fwd(_np(q), _np(k), _np(v), True)
    # query head h reading KV head h % Hkv instead of h // groups
    monkeypatch.setattr(R, "_expand_kv", lambda t, g: t.repeat(1, 1, g, 1))
    o = R.attention(q, k, v, True, 5, torch.float64)
    assert np.abs(_np(o) - o_ref).max() > 1e-3


def test_planted_strict_causal_mask_is_caught():
    q, k, v, _ = R.make_inputs(1, 9, 10, 2, 128, seed=12, dtype=torch.float64)
    o_ref, _ = brute.fwd(_np(q), _np(k), _np(v), True)
    s = R.scores(q, k, False, 5, torch.float64)
    wrong = s.masked_fill(~torch.ones(9, 9, dtype=torch.bool).tril(-1), float("-inf"))
    p = wrong.softmax(-1).nan_to_num(0.0)
    o = torch.matmul(p, v.repeat_interleave(5, dim=2).permute(0, 2, 1, 3)).permute(0, 2, 1, 3)
    assert np.abs(_np(o) - o_ref).max() > 1e-3


def test_planted_missing_group_sum_is_caught():
    q, k, v, do = R.make_inputs(1, 9, 10, 2, 128, seed=13, dtype=torch.float64)
    _, dk_ref, _ = brute.bwd(_np(q), _np(k), _np(v), _np(do), True)
    _, dk, _ = R.grads_analytic(q, k, v, do, True, 5, torch.float64)
    # keep only the first query head of each group instead of summing all five
    dk_one = R.grads_analytic(q[:, :, ::5].contiguous(), k, v, do[:, :, ::5].contiguous(),
                              True, 1, torch.float64)[1]
    assert np.abs(_np(dk) - dk_ref).max() < 1e-11
    assert np.abs(_np(dk_one) - dk_ref).max() > 1e-3


def test_planted_lse_natural_log_is_caught():
    q, k, v, _ = R.make_inputs(1, 9, 10, 2, 128, seed=14, dtype=torch.float64)
    _, lse_ref = brute.fwd(_np(q), _np(k), _np(v), True)
    wrong = torch.logsumexp(R.scores(q, k, True, 5, torch.float64), dim=-1)  # missing log2(e)
    assert np.abs(_np(wrong) - lse_ref).max() > 1e-3


# ---------------------------------------------------------------------------
# Sublayer prologue (config 5): tables, RMSNorm, rotate-half RoPE.

def test_rope_tables_closed_form():
    """cos/sin at position p, column j: angle p * theta^(-2(j mod D/2)/D);
    position 0 is the identity rotation."""
    cos, sin = R.rope_tables(128, 40, 10000.0)
    assert cos.shape == (40, 128) and cos.dtype == torch.float32
    assert torch.equal(cos[0], torch.ones(128)) and torch.equal(sin[0], torch.zeros(128))
    for p, j in [(1, 0), (7, 3), (39, 63), (39, 127), (12, 100)]:
        ang = p * 10000.0 ** (-2 * (j % 64) / 128)
        assert abs(cos[p, j].item() - math.cos(ang)) < 2e-6
        assert abs(sin[p, j].item() - math.sin(ang)) < 2e-6


def test_rotate_half_rope_equals_pairwise_rotation():
    """In fp64 the rotate-half form rotates the pairs (d, d + D/2): it equals
    the explicit pairwise rotation (an independent formula) and keeps norms."""
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(2, 33, 3, 128, generator=gen, dtype=torch.float64)
    freqs = 1.0 / (10000.0 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    ang = torch.outer(torch.arange(33, dtype=torch.float64), freqs)
    table = torch.cat((ang, ang), dim=-1)
    got = R.apply_rope(x, table.cos(), table.sin())
    assert torch.allclose(got, R.rope(x, 10000.0), atol=1e-12)
    assert torch.allclose(got.norm(dim=-1), x.norm(dim=-1), atol=1e-10)
    # rotating twice by a half turn of each pair: rotate_half(rotate_half(x)) = -x
    assert torch.equal(R.rotate_half(R.rotate_half(x)), -x)


def test_rmsnorm_closed_forms():
    """Unit weight: each output row has mean square 1 / (1 + eps / ms); a
    constant row c maps to sign(c) |c| / sqrt(c^2 + eps); scale invariance."""
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(4, 5, 128, generator=gen) * 3
    w = torch.ones(128)
    y = R.rmsnorm(x, w, 1e-5)
    ms = x.pow(2).mean(-1)
    assert torch.allclose(y.pow(2).mean(-1), 1 / (1 + 1e-5 / ms), rtol=1e-5)
    c = torch.full((1, 128), -0.3)
    assert torch.allclose(R.rmsnorm(c, w, 1e-5), torch.full((1, 128), -0.3 / math.sqrt(0.09 + 1e-5)))
    assert torch.allclose(R.rmsnorm(5 * x, w, 0.0), R.rmsnorm(x, w, 0.0), atol=1e-6)
    wv = torch.linspace(0.5, 2, 128)
    assert torch.allclose(R.rmsnorm(x, wv, 1e-5), y * wv, atol=1e-6)
    # bf16 in, bf16 out: one rounding of the fp32 result
    xb = x.to(torch.bfloat16)
    assert torch.equal(R.rmsnorm(xb, wv, 1e-5), R.rmsnorm(xb.float(), wv, 1e-5).to(torch.bfloat16))


def test_qknorm_rope_column_split():
    """qkv columns are wq | wk | wv outputs: V is the untouched last slice and
    Q / K are the normalised, rotated first slices (no norm: pure rotation)."""
    gen = torch.Generator().manual_seed(3)
    qkv = torch.randn(2, 9, (6 + 2 * 3) * 128, generator=gen)
    cos, sin = R.rope_tables(128, 16, 10000.0)
    q, k, v = R.qknorm_rope(qkv, None, None, cos, sin, 6, 3)
    assert q.shape == (2, 9, 6, 128) and k.shape == (2, 9, 3, 128) and v.shape == (2, 9, 3, 128)
    assert torch.equal(v.reshape(2, 9, -1), qkv[..., 9 * 128:])
    assert torch.equal(q[:, 0], qkv[:, 0, :6 * 128].reshape(2, 6, 128))   # position 0: identity
    assert torch.allclose(k.norm(dim=-1), qkv[..., 6 * 128:9 * 128].reshape(2, 9, 3, 128).norm(dim=-1),
                          rtol=1e-5)
    w = torch.ones(128)
    qn, _, _ = R.qknorm_rope(qkv, w, w, cos, sin, 6, 3)
    assert torch.allclose(qn.pow(2).mean(-1), torch.ones(2, 9, 6), rtol=1e-3)


# ---------------------------------------------------------------------------
# SwiGLU oracle (oracle/swiglu.py)
from oracle import swiglu as SW  # noqa: E402


def _ulp_bf16(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (8 significant bits)."""
    e = torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -126)))
    return torch.pow(2.0, e - 7)


def test_swiglu_manual_grads_match_fp64_autograd():
    """FusedSwiGLU.backward's formulas against autograd (the reference's own
    check, swiglu_tilelang.py:426-462), in fp64."""
    gen = torch.Generator().manual_seed(1)
    m, d, h = 32, 64, 96
    x = torch.randn(m, d, generator=gen, dtype=torch.float64)
    wg = torch.randn(d, h, generator=gen, dtype=torch.float64) * 0.1
    wu = torch.randn(d, h, generator=gen, dtype=torch.float64) * 0.1
    wd = torch.randn(h, d, generator=gen, dtype=torch.float64) * 0.1
    go = torch.randn(m, d, generator=gen, dtype=torch.float64)
    auto = SW.grads(x, wg, wu, wd, go, dtype=torch.float64)
    manual = SW.manual_grads(x, wg, wu, wd, go)
    assert torch.allclose(auto[0], SW.reference(x, wg, wu, wd).double(), rtol=1e-6, atol=1e-6)
    for a, b in zip(manual, auto[1:]):
        assert ((a - b).abs().max() / b.abs().max()).item() < 1e-10


def test_swiglu_grad_oracle_is_the_derivative():
    """grad() equals autograd of silu(g) * u (fp64) rounded to bf16, to one
    bf16 ulp; a dropped (1 + g(1 - s)) factor is caught."""
    gen = torch.Generator().manual_seed(2)
    a, g, u = (torch.randn(64, 96, generator=gen).mul(s).to(torch.bfloat16) for s in (1.0, 3.0, 2.0))
    gd, ud = g.double().requires_grad_(True), u.double().requires_grad_(True)
    (F.silu(gd) * ud).backward(a.double())
    dg, du = SW.grad(a, g, u)
    for got, want in ((dg, gd.grad), (du, ud.grad)):
        err = (got.double() - want).abs()
        assert (err <= _ulp_bf16(want) + 1e-30).all()
    s = torch.sigmoid(g.float())
    wrong = (a.float() * u.float() * s).to(torch.bfloat16)          # missing (1 + g (1 - s))
    assert (wrong.double() - gd.grad).abs().max() > 0.1


def test_swiglu_silu_derivative_closed_form():
    """The reference's checks (swiglu_tilelang.py:413-424)."""
    z = (torch.randn(2000, dtype=torch.float64) * 3).requires_grad_(True)
    F.silu(z).sum().backward()
    s = torch.sigmoid(z.detach())
    assert (z.grad - s * (1 + z.detach() * (1 - s))).abs().max() < 1e-12
    assert F.silu(torch.zeros(1)).item() == 0.0 and torch.sigmoid(torch.zeros(1)).item() == 0.5


def test_swiglu_forward_oracles_round_once():
    """split / act_fused are the fp64 products rounded once (to one bf16 ulp:
    the oracle accumulates in fp32); act_train is F.silu(gate) * up on bf16."""
    x, wg, wu, _, _ = SW.make_inputs(48, d_model=128, ffn=64, seed=3)
    g64, u64 = x.double() @ wg.double(), x.double() @ wu.double()
    gate, up = SW.split(x, wg, wu)
    for got, want in ((gate, g64), (up, u64)):
        assert ((got.double() - want).abs() <= _ulp_bf16(want) + 1e-30).all()
    act = SW.act_fused(x, wg, wu)
    want = g64 * torch.sigmoid(g64) * u64
    assert ((act.double() - want).abs() <= _ulp_bf16(want) + 1e-12).all()
    assert torch.equal(SW.act_train(gate, up), F.silu(gate) * up)
    assert torch.equal(SW.act_train(gate, up), (F.silu(gate.float()).to(torch.bfloat16) * up))


def test_swiglu_reference_matches_module_math_backend():
    from mimansm1_v1_amd import swiglu as S
    torch.manual_seed(0)
    cfg = S.FFNConfig(d_model=256, ffn_hidden=384)
    ffn = S.SwiGLU(cfg)
    x = torch.randn(3, 5, 256)
    want = SW.reference(x.reshape(-1, 256), ffn.w_gate, ffn.w_up, ffn.w_down).reshape(3, 5, 256)
    assert (ffn(x, backend="math") - want).abs().max() < 1e-6


# ---------------------------------------------------------------------------
# Cross-entropy head oracle (oracle/lm_head.py)
from oracle import lm_head as LMO  # noqa: E402


def test_lm_online_lse_and_lse_match_logsumexp():
    """The kernel's online recurrence and the oracle's lse against
    torch.logsumexp (the reference's check, lm_head_tilelang.py:393-406)."""
    x = torch.randn(64, 5000, dtype=torch.float64) * 8
    assert (LMO.online_lse(x, 128) - torch.logsumexp(x, dim=1)).abs().max() < 1e-12
    h = torch.randn(16, 32, dtype=torch.float64)
    w = torch.randn(32, 300, dtype=torch.float64)
    assert torch.allclose(LMO.lse(h, w, torch.float64), torch.logsumexp(h @ w, dim=1), rtol=0, atol=1e-12)
    big = torch.tensor([[1e4, 1e4 + 1.0]], dtype=torch.float64)
    assert torch.isfinite(LMO.online_lse(big, 1)).all()


def test_lm_loss_matches_cross_entropy_with_ignore_index():
    gen = torch.Generator().manual_seed(4)
    h = torch.randn(40, 24, generator=gen, dtype=torch.float64)
    w = torch.randn(24, 256, generator=gen, dtype=torch.float64) * 0.3
    t = torch.randint(0, 256, (40,), generator=gen)
    t[:7] = LMO.IGNORE_INDEX
    want = F.cross_entropy(h @ w, t, ignore_index=LMO.IGNORE_INDEX)
    assert (LMO.loss(h, w, t, dtype=torch.float64) - want).abs() < 1e-12
    assert LMO.loss(h, w, torch.full_like(t, LMO.IGNORE_INDEX), dtype=torch.float64).item() == 0.0
    # planted mistake: averaging over every token instead of the valid ones
    wrong = (torch.logsumexp(h @ w, 1) - LMO.target_logits(h, w, t, torch.float64))[7:].sum() / 40
    assert (wrong - want).abs() > 1e-3


def test_lm_dlogits_is_the_cross_entropy_gradient():
    """dlogits = (softmax - onehot) * mask * scale equals autograd of the summed
    cross entropy times scale (the reference's gradient identity, :420-428);
    dropping the one-hot is caught."""
    gen = torch.Generator().manual_seed(5)
    h = torch.randn(32, 16, generator=gen, dtype=torch.float64)
    w = torch.randn(16, 128, generator=gen, dtype=torch.float64) * 0.5
    t = torch.randint(0, 128, (32,), generator=gen)
    t[3] = LMO.IGNORE_INDEX
    lg = (h @ w).requires_grad_(True)
    scale = 0.37
    (F.cross_entropy(lg, t, ignore_index=LMO.IGNORE_INDEX, reduction="sum") * scale).backward()
    got = LMO.dlogits(h, w, t, LMO.lse(h, w, torch.float64), scale, dtype=torch.float64)
    assert (got - lg.grad).abs().max() < 1e-12
    no_onehot = torch.softmax(h @ w, 1) * (t != LMO.IGNORE_INDEX).unsqueeze(1) * scale
    assert (no_onehot - lg.grad).abs().max() > 0.1


def test_lm_grads_oracle_matches_manual_chain_rule():
    gen = torch.Generator().manual_seed(6)
    h = torch.randn(24, 16, generator=gen, dtype=torch.float64)
    w = torch.randn(16, 256, generator=gen, dtype=torch.float64) * 0.2
    t = torch.randint(0, 256, (24,), generator=gen)
    t[:2] = LMO.IGNORE_INDEX
    loss, dh, dw = LMO.grads(h, w, t, dtype=torch.float64)
    count = (t != LMO.IGNORE_INDEX).sum()
    dl = LMO.dlogits(h, w, t, LMO.lse(h, w, torch.float64), 1.0 / count.item(), dtype=torch.float64)
    assert (dh - dl @ w.t()).abs().max() < 1e-12
    assert (dw - h.t() @ dl).abs().max() < 1e-12
    assert (loss - LMO.loss(h, w, t, dtype=torch.float64)).abs() < 1e-12
