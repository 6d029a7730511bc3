"""ctypes wrapper of brute_attn.c (fp64 brute force) -- test infrastructure only."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libbrute_attn.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        dp, ci, cd = ctypes.POINTER(ctypes.c_double), ctypes.c_int, ctypes.c_double
        lib.brute_attn_fwd.argtypes = [dp] * 5 + [ci] * 6 + [cd]
        lib.brute_attn_bwd.argtypes = [dp] * 8 + [ci] * 6 + [cd]
        lib.brute_attn_bwd_emul.argtypes = [dp] * 8 + [ci] * 6 + [cd]
        lib.brute_bf16.argtypes = [cd]
        lib.brute_bf16.restype = cd
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def fwd(q, k, v, causal, sm_scale=None):
    """q [B,S,H,D], k/v [B,S,Hkv,D] float64 arrays -> (o [B,S,H,D], lse2 [B,H,S])."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float64) for x in (q, k, v))
    B, S, H, D = q.shape
    Hkv = k.shape[2]
    sm_scale = D ** -0.5 if sm_scale is None else sm_scale
    o = np.zeros_like(q)
    lse = np.zeros((B, H, S))
    load().brute_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, S, H, Hkv, D,
                          int(causal), sm_scale)
    return o, lse


def _bwd(fn, q, k, v, do, causal, sm_scale):
    q, k, v, do = (np.ascontiguousarray(x, dtype=np.float64) for x in (q, k, v, do))
    B, S, H, D = q.shape
    Hkv = k.shape[2]
    sm_scale = D ** -0.5 if sm_scale is None else sm_scale
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    delta = np.zeros((B, H, S))
    fn(_ptr(q), _ptr(k), _ptr(v), _ptr(do), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(delta),
       B, S, H, Hkv, D, int(causal), sm_scale)
    return dq, dk, dv, delta


def bwd(q, k, v, do, causal, sm_scale=None, with_delta=False):
    """Exact fp64 backward -> (dq, dk, dv[, delta]); delta_i = sum_j P_ij dP_ij."""
    dq, dk, dv, delta = _bwd(load().brute_attn_bwd, q, k, v, do, causal, sm_scale)
    return (dq, dk, dv, delta) if with_delta else (dq, dk, dv)


def bwd_emul(q, k, v, do, causal, sm_scale=None):
    """fp64 backward with the reference kernel's bf16 rounding points (P before
    dV, P (dP - Delta) sm_scale before dK / dQ, Delta from the bf16 forward
    output) -> (dq, dk, dv, delta)."""
    return _bwd(load().brute_attn_bwd_emul, q, k, v, do, causal, sm_scale)


def bf16(x: float) -> float:
    """Round-to-nearest-even to bfloat16 precision (the C routine the emulation uses)."""
    return load().brute_bf16(float(x))
