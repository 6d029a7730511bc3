"""ctypes binding of the C ABI declared in include/mm1_attn.h.

The library is built in-tree by ``mimansm1_v1_amd.build`` (hipcc, gfx950).  It
is the only compute path of this package: if it is missing, every entry point
raises -- there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path


# Every symbol include/mm1_attn.h declares, with its ctypes signature.
_c_int, _c_float, _c_size, _vp = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p
SHAPE = [_c_int] * 5                       # B, S, H, Hkv, D
SHAPE_CS = SHAPE + [_c_int, _c_float]       # ..., causal, sm_scale
SIGNATURES = {
    "mm1_attn_version": (_c_int, []),
    "mm1_attn_fwd_state_size": (_c_size, SHAPE),
    "mm1_attn_fwd": (_c_int, [_vp] * 5 + [_vp, _c_size] + SHAPE_CS + [_vp]),
    "mm1_attn_fwd_tiles": (_c_int, [_vp] * 5 + [_vp, _c_size] + SHAPE_CS + [_c_int, _vp]),
    "mm1_attn_fwd_f32": (_c_int, [_vp] * 5 + [_vp, _c_size] + SHAPE_CS + [_c_int, _vp]),
    "mm1_attn_prep": (_c_int, [_vp] * 3 + [_vp, _c_size] + SHAPE + [_vp]),
    "mm1_attn_tile_count": (_c_int, [_c_int]),
    "mm1_attn_tile_desc": (ctypes.c_char_p, [_c_int, _c_int]),
    "mm1_attn_delta": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "mm1_attn_bwd_workspace_size": (_c_size, SHAPE),
    "mm1_attn_bwd_prep": (_c_int, [_vp, _vp, _vp, _vp, _c_size, _vp, _c_size] + SHAPE + [_c_float, _vp]),
    "mm1_attn_bwd_prep_delta": (_c_int, [_vp, _vp, _vp, _vp, _c_size, _vp, _c_size] + SHAPE + [_c_float, _vp]),
    "mm1_attn_bwd": (_c_int, [_vp, _vp, _vp, _vp, _c_size, _vp, _vp, _vp, _vp, _c_size] + SHAPE_CS + [_vp]),
    "mm1_attn_bwd_tiles": (_c_int, [_vp, _vp, _vp, _vp, _c_size, _vp, _vp, _vp, _vp, _c_size] + SHAPE_CS
                           + [_c_int, _c_int, _vp]),
    "mm1_attn_bwd_f32_tiles": (_c_int, [_vp, _vp, _vp, _vp, _c_size, _vp, _vp, _vp, _vp, _c_size] + SHAPE_CS
                               + [_c_int, _c_int, _vp]),
    "mm1_attn_bwd_noalloc": (_c_int, [_vp, _vp, _vp, _vp, _c_size, _vp, _vp, _vp] + SHAPE_CS + [_vp]),
    "mm1_attn_bwd_noalloc_scratch_size": (_c_size, SHAPE + [_c_int]),
    "mm1_attn_bwd_dkdv_tiles": (_c_int, [_vp, _c_size, _vp, _vp, _vp, _c_size] + SHAPE_CS + [_c_int, _vp]),
    "mm1_attn_bwd_dkdv_reduce_tiles": (_c_int, [_vp, _c_size, _vp, _vp] + SHAPE + [_c_int, _c_int, _vp]),
    "mm1_attn_bwd_dq_tiles": (_c_int, [_vp, _c_size, _vp, _vp, _c_size] + SHAPE_CS + [_c_int, _vp]),
    "mm1_attn_bwd_dq_reduce_tiles": (_c_int, [_vp, _c_size, _vp, _vp, _vp, _vp, _c_size] + SHAPE_CS
                                     + [_c_int, _c_int, _vp]),
    "mm1_attn_dispatch_order": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                         _c_int, _vp, _c_int]),
    "mm1_attn_dkdv_plan": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _vp]),
    "mm1_qknorm_rope_fwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float, _vp]),
    "mm1_qknorm_rope_bwd_workspace_size": (_c_size, []),
    "mm1_qknorm_rope_bwd": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _c_size, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                     _c_float, _vp]),
    "mm1_swiglu_gate_up": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "mm1_swiglu_grad": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, ctypes.c_long, _vp]),
    "mm1_lm_head_workspace_size": (_c_size, [_c_int, _c_int]),
    "mm1_lm_head_lse": (_c_int, [_vp, _vp, _vp, ctypes.c_longlong, _vp, _vp, _vp, _vp, _c_size,
                                 _c_int, _c_int, _c_int, _vp]),
    "mm1_lm_head_dlogits": (_c_int, [_vp, _vp, _vp, ctypes.c_longlong, _vp, _vp, _vp, ctypes.c_long,
                                     _c_int, _c_int, _c_int, _c_int, _c_int, _vp]),
    "mm1_attn_strerror": (ctypes.c_char_p, [_c_int]),
}

_lock = threading.Lock()
_lib = None


class LibraryMissing(RuntimeError):
    pass


def library_path() -> Path:
    """The in-tree build, or the file MM1_ATTN_LIB names (to compare builds)."""
    override = os.environ.get("MM1_ATTN_LIB")
    if override:
        return Path(override).resolve()
    from . import build   # imported here: `python -m mimansm1_v1_amd.build` must not find it loaded
    return build.library_path()


def load() -> ctypes.CDLL:
    """Load (once) and return the attention library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = library_path()
            if not path.exists():
                raise LibraryMissing(
                    f"{path} is not built; run `python -m mimansm1_v1_amd.build` "
                    "(hipcc, gfx950) first")
            lib = ctypes.CDLL(str(path))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


class AttnError(RuntimeError):
    """A nonzero return code of the C ABI."""

    def __init__(self, code: int, where: str):
        self.code = code
        msg = load().mm1_attn_strerror(code).decode()
        super().__init__(f"{where}: {msg} (code {code})")


def check(code: int, where: str) -> None:
    if code != 0:
        raise AttnError(code, where)
