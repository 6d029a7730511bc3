"""Writes tests/golden/attn_cases.npz: small seeded attention cases with their
expected outputs.

Inputs are generated with oracle.reference.make_inputs (CPU generator, draws
Q, K, V, dO) and stored as bf16 bit patterns (uint16).  Expected outputs come
from the fp64 brute force in oracle/brute_attn.c (independent of torch) run on
those exact bf16 values: O (before the bf16 cast), lse2 (log2 units), dQ, dK,
dV, all stored as float32.  The reference repository holds no golden vectors
of its own for this path, so these are the fixtures the tests pin against.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import brute  # noqa: E402
from oracle import reference as R  # noqa: E402

OUT = Path(__file__).with_name("attn_cases.npz")

# name: (B, S, H, Hkv, causal, seed, rope_sigma)
CASES = {
    "s1_causal": (1, 1, 10, 2, True, 1, False),
    "s9_causal": (1, 9, 10, 2, True, 2, False),
    "s33_full_mha": (1, 33, 2, 2, False, 3, False),
    "s40_g3_causal": (1, 40, 3, 1, True, 4, False),
    "s24_rope_sigma": (1, 24, 5, 1, True, 5, True),
}


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def main():
    arrays = {}
    for name, (B, S, H, Hkv, causal, seed, rope_sigma) in CASES.items():
        q, k, v, do = R.make_inputs(B, S, H, Hkv, 128, seed=seed, rope_sigma=rope_sigma)
        qd, kd, vd, dod = (t.double().numpy() for t in (q, k, v, do))
        o, lse = brute.fwd(qd, kd, vd, causal)
        dq, dk, dv = brute.bwd(qd, kd, vd, dod, causal)
        arrays[f"{name}/meta"] = np.array([B, S, H, Hkv, int(causal)], dtype=np.int64)
        for key, t in (("q", q), ("k", k), ("v", v), ("do", do)):
            arrays[f"{name}/{key}"] = bf16_bits(t)
        for key, a in (("o", o), ("lse2", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
            arrays[f"{name}/{key}"] = a.astype(np.float32)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size / 1024:.0f} KiB, {len(CASES)} cases)")


def load_cases():
    """{name: dict(meta=(B,S,H,Hkv,causal), q,k,v,do as bf16 tensors, o,lse2,dq,dk,dv fp32)}"""
    data = np.load(OUT, allow_pickle=False)
    cases = {}
    for name in CASES:
        B, S, H, Hkv, causal = (int(x) for x in data[f"{name}/meta"])
        c = {"meta": (B, S, H, Hkv, bool(causal))}
        for key in ("q", "k", "v", "do"):
            c[key] = torch.from_numpy(data[f"{name}/{key}"].view(np.int16).copy()).view(torch.bfloat16)
        for key in ("o", "lse2", "dq", "dk", "dv"):
            c[key] = torch.from_numpy(data[f"{name}/{key}"].copy())
        cases[name] = c
    return cases


if __name__ == "__main__":
    main()
