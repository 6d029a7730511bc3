"""The C-ABI library: loads, exports every declared symbol, validates its
arguments before touching a device.  No GPU needed (and none is touched: every
call here returns from the argument checks)."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

from mimansm1_v1_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mm1_attn.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))
FAKE = 1 << 20  # aligned, non-null; never dereferenced (calls fail validation first)


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(mm1_\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_library_built_in_tree(lib):
    path = _lib.library_path()
    assert path.exists() and ROOT in path.parents


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 8
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mm1_\w+)", out))
    assert set(names) <= exported, set(names) - exported
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"
    for n in names:
        getattr(lib, n)


def test_probe_library_apart_from_the_abi(lib):
    """The matrix-core probe bench.py --mfma-ceiling runs is its own library:
    built in-tree beside the attention library, exporting only its entry
    point, which the attention library does not carry."""
    from mimansm1_v1_amd import build as B
    path = B.probe_path()
    assert path.exists() and ROOT in path.parents
    probe = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True,
                           check=True).stdout
    assert set(re.findall(r"\bT (mm1_\w+)", probe)) == {"mm1_probe_mfma_ceiling"}
    attn = subprocess.run(["nm", "-D", "--defined-only", str(_lib.library_path())], capture_output=True,
                          text=True, check=True).stdout
    assert "mm1_probe_mfma_ceiling" not in attn


def test_version_matches_header(lib):
    m = re.search(r"#define MM1_ATTN_VERSION (\d+)", HEADER.read_text())
    assert lib.mm1_attn_version() == int(m.group(1))


def test_error_codes_and_messages(lib):
    codes = dict(re.findall(r"#define (MM1_E_\w+) \((-\d+)\)", HEADER.read_text()))
    assert len(codes) == 9
    for name, code in codes.items():
        msg = lib.mm1_attn_strerror(int(code)).decode()
        assert msg.startswith("mm1_attn:") and "unknown" not in msg, name
    assert lib.mm1_attn_strerror(0) == b"success"
    assert b"unknown" in lib.mm1_attn_strerror(-99)


def _state_bytes(lib, B=1, S=64, H=10, Hkv=2):
    return lib.mm1_attn_fwd_state_size(B, S, H, Hkv, 128)


def fwd(lib, q=FAKE, k=FAKE, v=FAKE, o=FAKE, lse=FAKE, st=FAKE, st_bytes=None, B=1, S=64, H=10, Hkv=2, D=128,
        causal=1, scale=0.088):
    nb = _state_bytes(lib, B, S, H, Hkv) if st_bytes is None else st_bytes
    return lib.mm1_attn_fwd(q, k, v, o, lse, st, nb, B, S, H, Hkv, D, causal, scale, None)


def test_state_and_workspace_sizes(lib):
    """The forward state holds fp16 Q, K, V (2 bytes a value), the O residual
    (1 byte) and the max|V| partials; the backward workspace fp16 dO, the
    scaled Delta, lse2 - log2(sm_scale), the dO maxima and scale, and 2 * G
    fp32 slots of partial sums (none when G == 1).  Every region is 256-byte
    aligned."""
    up = lambda x: (x + 255) // 256 * 256
    B, S, H, Hkv = 2, 100, 10, 2
    nq, nkv = B * S * H * 128, B * S * Hkv * 128
    assert lib.mm1_attn_fwd_state_size(B, S, H, Hkv, 128) == up(2 * nq) + 2 * up(2 * nkv) + up(nq) + up(512 * 4)
    base = up(2 * nq) + 2 * up(4 * B * H * S) + up(1024 * 4) + 256
    assert lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, 128) == base + up(2 * 5 * nkv * 4)
    assert lib.mm1_attn_bwd_workspace_size(B, S, 4, 4, 128) == up(2 * B * S * 4 * 128) + 2 * up(4 * B * 4 * S) \
        + up(1024 * 4) + 256
    assert lib.mm1_attn_bwd_workspace_size(B, S, 10, 3, 128) == 0   # invalid shape
    assert lib.mm1_attn_fwd_state_size(B, S, 10, 2, 64) == 0


def test_fwd_argument_errors(lib):
    assert fwd(lib, q=None) == -1
    assert fwd(lib, lse=None) == -1
    assert fwd(lib, st=None) == -1
    assert fwd(lib, H=10, Hkv=3) == -2
    assert fwd(lib, B=0) == -2
    assert fwd(lib, S=0) == -2
    assert fwd(lib, D=64) == -3
    assert fwd(lib, st_bytes=_state_bytes(lib) - 1) == -4
    assert fwd(lib, scale=0.0) == -5
    assert fwd(lib, scale=float("nan")) == -5
    assert fwd(lib, q=FAKE + 8) == -6
    assert fwd(lib, st=FAKE + 4) == -6
    nb = _state_bytes(lib)
    assert lib.mm1_attn_fwd_f32(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, nb, 1, 64, 10, 2, 128, 1, 0.1, 9, None) == -7
    assert lib.mm1_attn_fwd_f32(FAKE, FAKE, FAKE, None, FAKE, FAKE, nb, 1, 64, 10, 2, 128, 1, 0.1, 0, None) == -1
    assert lib.mm1_attn_prep(FAKE, FAKE, None, FAKE, nb, 1, 64, 10, 2, 128, None) == -1
    assert lib.mm1_attn_prep(FAKE, FAKE, FAKE, FAKE, nb - 256, 1, 64, 10, 2, 128, None) == -4
    assert lib.mm1_attn_prep(FAKE, FAKE, FAKE, FAKE, nb, 1, 64, 10, 2, 64, None) == -3


def test_bwd_argument_errors(lib):
    B, S, H, Hkv = 2, 100, 10, 2
    need = lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, 128)
    nst = _state_bytes(lib, B, S, H, Hkv)

    def bwd(o=FAKE, st=FAKE, st_bytes=None, ws=FAKE, ws_bytes=None, dq=FAKE, **kw):
        a = dict(B=B, S=S, H=H, Hkv=Hkv, D=128, causal=1, scale=0.088)
        a.update(kw)
        return lib.mm1_attn_bwd(o, FAKE, FAKE, st, nst if st_bytes is None else st_bytes, dq, FAKE, FAKE, ws,
                                need if ws_bytes is None else ws_bytes, a["B"], a["S"], a["H"], a["Hkv"], a["D"],
                                a["causal"], a["scale"], None)

    assert bwd(o=None) == -1
    assert bwd(dq=None) == -1
    assert bwd(st=None) == -1
    assert bwd(ws=None) == -1
    assert bwd(ws_bytes=need - 1) == -4
    assert bwd(st_bytes=nst - 1) == -4
    assert bwd(D=256) == -3
    assert bwd(H=9) == -2
    assert bwd(scale=-1.0) == -5
    assert bwd(ws=FAKE + 4) == -6
    assert bwd(dq=FAKE + 2) == -6
    sz = (B, S, H, Hkv, 128)
    assert lib.mm1_attn_bwd_prep(None, FAKE, FAKE, FAKE, nst, FAKE, need, *sz, 0.1, None) == -1
    assert lib.mm1_attn_bwd_prep(FAKE, FAKE, None, FAKE, nst, FAKE, need, *sz, 0.1, None) == -1
    assert lib.mm1_attn_bwd_prep(FAKE, FAKE, FAKE, FAKE, nst, FAKE, need - 8, *sz, 0.1, None) == -4
    assert lib.mm1_attn_bwd_prep(FAKE, FAKE, FAKE, FAKE, nst, FAKE, need, *sz, 0.0, None) == -5
    assert lib.mm1_attn_bwd_prep_delta(FAKE, None, FAKE, FAKE, nst, FAKE, need, *sz, 0.1, None) == -1
    assert lib.mm1_attn_bwd_prep_delta(FAKE, FAKE, None, FAKE, nst, FAKE, need, *sz, 0.1, None) == -1
    assert lib.mm1_attn_bwd_prep_delta(FAKE + 2, FAKE, FAKE, FAKE, nst, FAKE, need, *sz, 0.1, None) == -6
    cs = sz + (1, 0.1)
    assert lib.mm1_attn_bwd_dq_tiles(FAKE, nst, None, FAKE, need, *cs, 0, None) == -1
    assert lib.mm1_attn_bwd_dkdv_tiles(FAKE, nst, None, FAKE, FAKE, need, *cs, 0, None) == -1
    assert lib.mm1_attn_bwd_dq_reduce_tiles(FAKE, nst, FAKE, FAKE, None, FAKE, need, *cs, 0, 0, None) == -1
    assert lib.mm1_attn_bwd_dq_reduce_tiles(FAKE, nst, FAKE, FAKE, FAKE, None, 0, *cs, 0, 0, None) == -1
    assert lib.mm1_attn_bwd_dq_reduce_tiles(FAKE, nst, FAKE, FAKE, FAKE, FAKE + 4, need, *cs, 0, 0,
                                            None) == -6
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(None, 0, FAKE, FAKE, *sz, 1, 0, None) == -1
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(FAKE, need - 1, FAKE, FAKE, *sz, 1, 0, None) == -4
    # nothing to reduce without groups: success without a device call
    need1 = lib.mm1_attn_bwd_workspace_size(1, 64, 4, 4, 128)
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(FAKE, need1, FAKE, FAKE, 1, 64, 4, 4, 128, 1, 0, None) == 0
    f32 = lib.mm1_attn_bwd_f32_tiles
    assert f32(FAKE, FAKE, FAKE, FAKE, nst, FAKE, FAKE, FAKE, FAKE, need, *cs, 5, 0, None) == -7
    assert f32(FAKE, FAKE, FAKE, FAKE, nst, FAKE, None, FAKE, FAKE, need, *cs, 0, 0, None) == -1


def test_reduce_refuses_a_workspace_without_matching_partials(lib):
    """The calls that sum dK/dV partials check the layout record of the
    workspace (written by a successful mm1_attn_bwd_dkdv_tiles launch) and
    return MM1_E_LAYOUT, launching nothing, when there is none for that
    address -- here no dK/dV call ever ran on it.  On the GPU the
    mismatched-tiling and mismatched-shape cases are checked after real dK/dV
    launches."""
    E_LAYOUT = -8
    B, S, H, Hkv = 2, 100, 10, 2
    need = lib.mm1_attn_bwd_workspace_size(B, S, H, Hkv, 128)
    nst = _state_bytes(lib, B, S, H, Hkv)
    ws = FAKE + (1 << 20)
    cs = (B, S, H, Hkv, 128, 1, 0.1)
    for t in range(lib.mm1_attn_tile_count(1)):
        assert lib.mm1_attn_bwd_dkdv_reduce_tiles(ws, need, FAKE, FAKE, B, S, H, Hkv, 128, 1, t, None) == E_LAYOUT
        assert lib.mm1_attn_bwd_dq_reduce_tiles(FAKE, nst, FAKE, FAKE, FAKE, ws, need, *cs, t, 0,
                                                None) == E_LAYOUT
    # argument errors still come first, and a tiling out of range is MM1_E_TILES
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(ws, need, FAKE, FAKE, B, S, H, Hkv, 128, 1, 99, None) == -7
    assert lib.mm1_attn_bwd_dkdv_reduce_tiles(None, 0, FAKE, FAKE, B, S, H, Hkv, 128, 1, 0, None) == -1
    # the dQ call without the sum needs no record
    assert lib.mm1_attn_bwd_dq_tiles(FAKE, nst, FAKE, ws, need, *cs, 9, None) == -7
    assert lib.mm1_attn_bwd_dkdv_tiles(FAKE, nst, FAKE, FAKE, ws, need, *cs, 9, None) == -7


def test_layout_record_is_keyed_by_address_only():
    """The layout record behind MM1_E_LAYOUT is host state keyed by the
    workspace address (include/mm1_attn.h: a workspace freed and reallocated
    at the same address with no dK/dV call since passes the check).  This
    test reads the behaviour from the source of the check, which it cannot
    exercise without a device: the record holds no allocation identity."""
    src = (ROOT / "mimansm1_v1_amd" / "csrc" / "attn_capi.hip").read_text()
    fields = re.search(r"struct WsLayout \{(.*?)\};", src, flags=re.S).group(1)
    assert "const void* ws;" in fields
    same = re.search(r"bool same\(const WsLayout& o\) const \{(.*?)\}", fields, flags=re.S).group(1)
    assert "ws" not in re.sub(r"\bo\.", "", same).split()          # the address is the key, not compared
    assert "a workspace freed and reallocated" in re.sub(r"\s*\n \*\s*", " ", HEADER.read_text())


def test_noalloc_refuses_shapes_beyond_its_scratch(lib):
    """mm1_attn_bwd_noalloc checks its arguments and the static scratch's
    size before any device call: MM1_E_SCRATCH for a shape whose backward
    workspace exceeds MM1_NOALLOC_SCRATCH_BYTES, the usual codes otherwise."""
    cap = 256 << 20
    assert f"(size_t)256 << 20" in HEADER.read_text()
    need = lib.mm1_attn_bwd_noalloc_scratch_size
    for B, S in ((8, 2048), (2, 8192), (4, 4096), (1, 16384)):
        assert 0 < need(B, S, 10, 2, 128, 1) <= cap, (B, S)
    # G = 1: no partials, only fp16 dO, Delta, the maxima and the scale
    assert need(2, 8192, 4, 4, 128, 1) == lib.mm1_attn_bwd_workspace_size(2, 8192, 4, 4, 128)
    assert need(1, 32768, 10, 2, 128, 1) > cap
    nst = _state_bytes(lib, 1, 32768, 10, 2)
    args = (FAKE,) * 3
    assert lib.mm1_attn_bwd_noalloc(*args, FAKE, nst, FAKE, FAKE, FAKE, 1, 32768, 10, 2, 128, 1, 0.1, None) == -9
    nst = _state_bytes(lib, 2, 64, 10, 2)
    assert lib.mm1_attn_bwd_noalloc(None, *args[1:], FAKE, nst, FAKE, FAKE, FAKE, 2, 64, 10, 2, 128, 1, 0.1,
                                    None) == -1
    assert lib.mm1_attn_bwd_noalloc(*args, FAKE, nst, FAKE, FAKE, FAKE, 2, 64, 10, 3, 128, 1, 0.1, None) == -2
    assert lib.mm1_attn_bwd_noalloc(*args, FAKE, nst, FAKE, FAKE, FAKE, 2, 64, 10, 2, 128, 1, 0.0, None) == -5
    assert lib.mm1_attn_bwd_noalloc(*args, FAKE, nst - 1, FAKE, FAKE, FAKE, 2, 64, 10, 2, 128, 1, 0.1, None) == -4
    assert b"static scratch" in lib.mm1_attn_strerror(-9)


def test_no_environment_switch_changes_the_tiling(lib, monkeypatch):
    """The library reads no tiling or chunk switch from the environment: the
    chunk plan and the layout of the partial sums depend on the shape, the
    tiling argument and the CU count only."""
    import ctypes
    plan = (ctypes.c_int * 5)()
    assert lib.mm1_attn_dkdv_plan(2, 8192, 10, 2, 1, 256, plan) == 0
    before = list(plan)
    for name, val in (("MM1_DKDV_CHUNK", "300"), ("MM1_DKDV_VARIANT", "1"), ("MM1_DQ_VARIANT", "1"),
                      ("MM1_FWD_VARIANT", "2")):
        monkeypatch.setenv(name, val)
    assert lib.mm1_attn_dkdv_plan(2, 8192, 10, 2, 1, 256, plan) == 0
    assert list(plan) == before
    assert lib.mm1_attn_delta(FAKE, None, FAKE, 1, 64, 10, 128, None) == -1
    assert lib.mm1_attn_delta(FAKE, FAKE, FAKE, 1, 64, 10, 64, None) == -3


def test_python_error_wrapper(lib):
    with pytest.raises(_lib.AttnError, match="head_dim must be 128"):
        _lib.check(-3, "mm1_attn_fwd")


def test_qknorm_rope_argument_errors_without_device(lib):
    """The sublayer prologue entries reject bad arguments before any launch."""
    fwd = lib.mm1_qknorm_rope_fwd
    ok = dict(B=1, S=64, H=10, Hkv=2, D=128, rot=64, eps=1e-5)

    def call(qkv=FAKE, wq=FAKE, wk=FAKE, q=FAKE, **kw):
        a = dict(ok, **kw)
        return fwd(qkv, wq, wk, FAKE, FAKE, q, FAKE, FAKE, a["B"], a["S"], a["H"], a["Hkv"], a["D"],
                   a["rot"], a["eps"], None)

    assert call(qkv=None) == -1
    assert call(wk=None) == -1            # both norm weights or neither
    assert call(D=64) == -3
    assert call(H=9) == -2
    assert call(rot=63) == -2             # tables shorter than the sequence
    assert call(eps=0.0) == -5
    assert call(q=FAKE + 8) == -6
    ws = lib.mm1_qknorm_rope_bwd_workspace_size()
    assert ws > 0
    bwd = lib.mm1_qknorm_rope_bwd
    args = [FAKE] * 11
    assert bwd(*args, None, ws, 1, 64, 10, 2, 128, 64, 1e-5, None) == -4
    assert bwd(*args, FAKE, ws - 4, 1, 64, 10, 2, 128, 64, 1e-5, None) == -4
    assert bwd(*args[:9], None, FAKE, FAKE, ws, 1, 64, 10, 2, 128, 64, 1e-5, None) == -1


def test_tilings_queries_and_errors_without_device(lib):
    """The compiled tilings are enumerable; an index out of range is refused
    before any launch, from both explicit-tiling entries."""
    counts = [lib.mm1_attn_tile_count(kind) for kind in (0, 1, 2)]
    assert counts[0] >= 3 and counts[1] >= 2 and counts[2] >= 2
    assert lib.mm1_attn_tile_count(3) == 0 and lib.mm1_attn_tile_count(-1) == 0
    for kind, n in enumerate(counts):
        descs = [lib.mm1_attn_tile_desc(kind, i).decode() for i in range(n)]
        assert len(set(descs)) == n
        for d in descs:
            keys = [item.split("=")[0] for item in d.split()]
            assert keys == ["block_M", "block_N", "waves", "stages", "schedule"], d
        assert lib.mm1_attn_tile_desc(kind, n) is None
        assert lib.mm1_attn_tile_desc(kind, -1) is None

    def fwd_t(tiles, **kw):
        a = dict(q=FAKE, B=1, S=64, H=10, Hkv=2, D=128)
        a.update(kw)
        nb = lib.mm1_attn_fwd_state_size(1, 64, 10, 2, 128)
        return lib.mm1_attn_fwd_tiles(a["q"], FAKE, FAKE, FAKE, FAKE, FAKE, nb, a["B"], a["S"], a["H"],
                                      a["Hkv"], a["D"], 1, 0.088, tiles, None)

    assert fwd_t(counts[0]) == -7
    assert fwd_t(-2) == -7
    assert fwd_t(counts[0], q=None) == -1          # argument checks come first
    assert fwd_t(0, D=64) == -3
    need = lib.mm1_attn_bwd_workspace_size(2, 100, 10, 2, 128)
    nst = lib.mm1_attn_fwd_state_size(2, 100, 10, 2, 128)

    def bwd_t(dkdv, dq, dq_ptr=FAKE, ws=FAKE):
        return lib.mm1_attn_bwd_tiles(FAKE, FAKE, FAKE, FAKE, nst, dq_ptr, FAKE, FAKE, ws,
                                      need, 2, 100, 10, 2, 128, 1, 0.088, dkdv, dq, None)

    assert bwd_t(counts[1], 0) == -7
    assert bwd_t(0, counts[2]) == -7               # refused before the first launch
    assert bwd_t(0, 0, dq_ptr=None) == -1
    assert bwd_t(0, 0, dq_ptr=FAKE + 2) == -6
    assert bwd_t(0, 0, ws=None) == -1
    assert b"tiling" in lib.mm1_attn_strerror(-7)


def test_swiglu_argument_errors_without_device(lib):
    """The SwiGLU entries reject bad arguments before any launch."""
    def gu(x=FAKE, gate=FAKE, up=FAKE, act=FAKE, T=256, d=1280, F=3328, mode=2):
        return lib.mm1_swiglu_gate_up(x, FAKE, FAKE, gate, up, act, T, d, F, mode, None)

    assert gu(x=None) == -1
    assert gu(act=None) == -1                 # the training mode writes act
    assert gu(gate=None, mode=1) == -1
    assert gu(d=1000) == -2                   # d_model not a multiple of 128
    assert gu(F=3300) == -2                   # ffn not a multiple of 128
    assert gu(F=3264) == -2
    assert gu(T=0) == -2
    assert gu(mode=3) == -2
    assert gu(up=FAKE + 2, mode=1) == -6
    # unused outputs may be NULL and are not checked
    assert gu(gate=None, up=None, act=FAKE + 2, mode=0) == -6

    def grad(ld=3328, **kw):
        a = dict(da=FAKE, dg=FAKE, T=256, F=3328)
        a.update(kw)
        return lib.mm1_swiglu_grad(a["da"], FAKE, FAKE, a["dg"], FAKE, a["T"], a["F"], ld, None)

    assert grad(da=None) == -1
    assert grad(ld=3320) == -2                # ld_out < ffn
    assert grad(ld=6660) == -2                # not a multiple of 8
    assert grad(F=3324) == -2
    assert grad(dg=FAKE + 8) == -6


def test_lm_head_argument_errors_without_device(lib):
    """The cross-entropy head entries reject bad arguments before any launch."""
    ws = lib.mm1_lm_head_workspace_size(256, 49152)
    assert ws >= 256 * 768 * 8 + 256 * 4
    assert lib.mm1_lm_head_workspace_size(256, 100) == 0       # vocab not a multiple of 128

    def lse(h=FAKE, tg=FAKE, lse_=FAKE, tl=FAKE, ws_=FAKE, nb=None, T=256, d=1280, V=49152):
        return lib.mm1_lm_head_lse(h, FAKE, tg, -100, lse_, tl, FAKE, ws_, ws if nb is None else nb,
                                   T, d, V, None)

    assert lse(h=None) == -1
    assert lse(lse_=None) == -1
    assert lse(tg=None) == -1                 # target_logit / loss need targets
    assert lse(d=1000) == -2
    assert lse(V=49000) == -2
    assert lse(ws_=None) == -4
    assert lse(nb=ws - 8) == -4
    assert lse(h=FAKE + 2) == -6

    def dl(v0=0, vn=4096, ld=4096, out=FAKE, V=49152):
        return lib.mm1_lm_head_dlogits(FAKE, FAKE, FAKE, -100, FAKE, FAKE, out, ld, 256, 1280, V, v0, vn, None)

    assert dl(out=None) == -1
    assert dl(v0=64) == -2                    # chunk start not a multiple of 128
    assert dl(vn=100) == -2
    assert dl(v0=49152 - 128, vn=256) == -2   # past the vocabulary
    assert dl(ld=4000) == -2                  # row stride shorter than the chunk
    assert dl(out=FAKE + 8) == -6


# ---------------------------------------------------------------------------
# Workgroup dispatch order of the causal grids (host-side model, no device).

def _order(lib, kind, tiles, B, S, H=10, Hkv=2, causal=1, cus=256):
    import ctypes
    n = lib.mm1_attn_dispatch_order(kind, tiles, B, S, H, Hkv, causal, cus, None, 0)
    if n <= 0:
        return n, []
    buf = (ctypes.c_ushort * n)()
    assert lib.mm1_attn_dispatch_order(kind, tiles, B, S, H, Hkv, causal, cus, buf, n) == n
    return n, list(buf)


def _items_and_costs(kind, tiles, B, S, H=10, Hkv=2):
    """Default numbering and relative work of a grid's items: forward / dQ row
    blocks walk their causal key tiles (64 keys), dK/dV key tiles their query
    tiles (32 queries); the kernels' own index arithmetic."""
    G = H // Hkv
    if kind == 1:
        nbh, nkt = B * H, (S + 127) // 128
        return [(S - (j // nbh) * 128 + 31) // 32 for j in range(nkt * nbh)]
    bm = 128 if tiles == (1 if kind == 0 else 0) else 256
    nbg, R = B * Hkv, G * S
    nt = (R + bm - 1) // bm
    out = []
    for j in range(nt * nbg):
        tile = nt - 1 - j // nbg
        last = min(tile * bm + bm, R) - 1
        out.append(min(S - 1, last // G) // 64 + 1)
    return out


def _makespan(order, costs, slots_per_se):
    """Dispatch as measured on gfx950: launch slot b goes to XCD b % 8; an
    XCD hands its k-th workgroup to shader engine k % 4 and waits, in order,
    for a free slot there (item cost + 1 fixed unit per workgroup)."""
    import heapq
    worst = 0
    for x in range(8):
        free = [[0] * slots_per_se for _ in range(4)]
        last = 0
        for k, b in enumerate(range(x, len(order), 8)):
            t = max(heapq.heappop(free[k % 4]), last)
            last = t
            heapq.heappush(free[k % 4], t + (costs[order[b]] + 1 if order[b] != 0xFFFF else 0))
        worst = max(worst, max(max(f) for f in free))
    return worst


# (kind, tiling): forward 0-2, the per-head dK/dV tiling 1 (the grouped
# tiling 0 has its own plan test below), dQ 0-1
GRIDS = [(0, 0), (0, 1), (0, 2), (1, 1), (2, 0), (2, 1)]
SHAPES = [(2, 8192), (8, 2048), (4, 4096), (1, 1000), (3, 777)]


@pytest.mark.parametrize("kind,tiles", GRIDS)
@pytest.mark.parametrize("B,S", SHAPES)
def test_dispatch_order_is_a_balanced_permutation(lib, kind, tiles, B, S):
    costs = _items_and_costs(kind, tiles, B, S)
    n, order = _order(lib, kind, tiles, B, S)
    table = n > 0
    if not table:                    # launched in the default order
        n, order = len(costs), list(range(len(costs)))
    assert len(costs) <= n <= len(costs) + 8 * 4 and (n % 8 == 0 or n == len(costs))
    items = [i for i in order if i != 0xFFFF]
    assert sorted(items) == list(range(len(costs)))          # every item exactly once
    assert all(i % 8 == b % 8 for b, i in enumerate(order) if i != 0xFFFF)   # XCD kept
    slots = 8 * (2 if (kind == 0 and tiles == 1) or (kind == 2 and tiles == 0) else 1)
    default = list(range(len(costs)))
    new_span, old_span = _makespan(order, costs, slots), _makespan(default, costs, slots)
    bound = max(max(costs), -(-sum(c + 1 for c in costs) // (8 * 4 * slots)))
    assert new_span <= old_span * 1.01 + 2, (new_span, old_span, bound)
    if table:
        assert new_span <= 1.10 * bound + 4, (new_span, old_span, bound)


def test_dispatch_order_defaults_and_errors(lib, monkeypatch):
    import ctypes
    # non-causal grids (equal items) and grids beyond the table run in the default order
    assert lib.mm1_attn_dispatch_order(0, 0, 2, 8192, 10, 2, 0, 256, None, 0) == 0
    assert lib.mm1_attn_dispatch_order(0, 0, 16, 8192, 10, 2, 1, 256, None, 0) == 0   # 5120 blocks
    assert lib.mm1_attn_dispatch_order(1, 1, 2, 8192, 10, 2, 1, 256, None, 0) == 0    # per-head dK/dV
    monkeypatch.setenv("MM1_DISPATCH_ORDER", "0")
    assert lib.mm1_attn_dispatch_order(0, 0, 2, 8192, 10, 2, 1, 256, None, 0) == 0
    monkeypatch.delenv("MM1_DISPATCH_ORDER")
    n = lib.mm1_attn_dispatch_order(0, 0, 2, 8192, 10, 2, 1, 256, None, 0)
    assert n >= 640
    buf = (ctypes.c_ushort * 8)()
    assert lib.mm1_attn_dispatch_order(0, 0, 2, 8192, 10, 2, 1, 256, buf, 8) == n
    _, full = _order(lib, 0, 0, 2, 8192)
    assert list(buf) == full[:8]
    # a device with fewer CUs gets its own table; two workgroups per CU: default order
    _, small = _order(lib, 0, 0, 2, 8192, cus=128)
    assert small != full and sorted(small) == sorted(full)
    assert lib.mm1_attn_dispatch_order(0, 1, 2, 8192, 10, 2, 1, 256, None, 0) == 0
    assert lib.mm1_attn_dispatch_order(2, 0, 2, 8192, 10, 2, 1, 256, None, 0) == 0
    E_TILES, E_SHAPE, E_NULL, E_HEAD = -7, -2, -1, -3
    assert lib.mm1_attn_dispatch_order(3, 0, 2, 8192, 10, 2, 1, 256, None, 0) == E_TILES
    assert lib.mm1_attn_dispatch_order(0, 9, 2, 8192, 10, 2, 1, 256, None, 0) == E_TILES
    assert lib.mm1_attn_dispatch_order(0, 0, 0, 8192, 10, 2, 1, 256, None, 0) == E_SHAPE
    assert lib.mm1_attn_dispatch_order(0, 0, 2, 8192, 10, 3, 1, 256, None, 0) == E_SHAPE
    assert lib.mm1_attn_dispatch_order(0, 0, 2, 8192, 10, 2, 1, 0, None, 0) == E_SHAPE
    assert lib.mm1_attn_dispatch_order(0, 0, 2, 8192, 10, 2, 1, 256, None, 4) == E_NULL
    assert E_HEAD != E_SHAPE


# ---------------------------------------------------------------------------
# Grouped dK/dV tiling: work plan and dispatch table (host-side, no device).

GROUPED = [(2, 8192, 10, 2, 1), (8, 2048, 10, 2, 1), (4, 4096, 10, 2, 1), (2, 7777, 10, 2, 1),
           (3, 1000, 10, 2, 1), (2, 2048, 10, 2, 0), (1, 4096, 8, 1, 1), (1, 333, 6, 3, 0),
           (1, 16384, 10, 2, 1), (1, 64, 10, 2, 1), (1, 3001, 16, 1, 1), (2, 1111, 16, 1, 0)]


def _grouped_items(B, S, H, Hkv, causal, L, C):
    """Default numbering of the grouped dK/dV grid, j = (kt*C + c)*B*Hkv + bg,
    with each item's query tiles in the position-major walk of its key tile
    (None for an empty item), as the header states the plan."""
    G, nkt, nbg = H // Hkv, (S + 127) // 128, B * Hkv
    out = []
    for kt in range(nkt):
        ln = G * ((S - (128 * kt if causal else 0) + 31) // 32)
        nc = min(C, max(1, -(-ln // L)))
        for c in range(C):
            for bg in range(nbg):
                out.append((kt, bg, ln, nc, list(range(c, ln, nc)) if c < nc else None))
    return out


@pytest.mark.parametrize("B,S,H,Hkv,causal", GROUPED,
                         ids=[f"B{b}S{s}G{h // kv}{'c' if c else 'f'}" for b, s, h, kv, c in GROUPED])
def test_grouped_dkdv_plan(lib, B, S, H, Hkv, causal):
    """The plan's chunks cover every (position tile, head) of every key tile
    exactly once, split only the key tiles below split_keys, fit the G
    workspace slots; its table runs every non-empty item once on the XCD of
    its default slot, with a modelled span no worse than the default order."""
    import ctypes
    plan = (ctypes.c_int * 5)()
    assert lib.mm1_attn_dkdv_plan(B, S, H, Hkv, causal, 256, plan) == 0
    L, C, split_keys, n_items, n_table = list(plan)
    G, nkt = H // Hkv, (S + 127) // 128
    assert C == G and L >= 1 and n_items == nkt * C * B * Hkv
    items = _grouped_items(B, S, H, Hkv, causal, L, C)
    by_tile = {}
    for kt, bg, ln, nc, tiles in items:
        assert nc <= C
        assert (nc > 1) == (128 * kt < split_keys), (kt, nc, split_keys)
        if tiles is not None:
            by_tile.setdefault((kt, bg), []).extend(tiles)
    for (kt, bg), tiles in by_tile.items():
        ln = items[(kt * C) * B * Hkv + bg][2]
        assert sorted(tiles) == list(range(ln))
    assert split_keys % 128 == 0 or split_keys == S
    n, order = _order(lib, 1, 0, B, S, H=H, Hkv=Hkv, causal=causal)
    assert n == n_table
    live = [j for j, it in enumerate(items) if it[4] is not None]
    if n == 0:
        return
    assert sorted(i for i in order if i != 0xFFFF) == live
    assert all(i % 8 == b % 8 for b, i in enumerate(order) if i != 0xFFFF)
    costs = [len(it[4]) if it[4] is not None else 0 for it in items]
    default = [j if items[j][4] is not None else 0xFFFF for j in range(len(items))]
    assert _makespan(order, costs, 8) <= _makespan(default, costs, 8) * 1.01 + 8


def test_grouped_dkdv_plan_errors_and_dispatch_switch(lib, monkeypatch):
    import ctypes
    plan = (ctypes.c_int * 5)()
    assert lib.mm1_attn_dkdv_plan(2, 8192, 10, 2, 1, 256, None) == -1
    assert lib.mm1_attn_dkdv_plan(2, 8192, 10, 3, 1, 256, plan) == -2
    assert lib.mm1_attn_dkdv_plan(2, 8192, 10, 2, 1, 0, plan) == -2
    # the dK/dV tiling index is checked by the dispatch-order query
    assert lib.mm1_attn_dispatch_order(1, lib.mm1_attn_tile_count(1), 2, 8192, 10, 2, 1, 256, None, 0) == -7
    assert lib.mm1_attn_dispatch_order(1, 1, 2, 8192, 10, 2, 1, 256, None, 0) == 0
    monkeypatch.setenv("MM1_DISPATCH_ORDER", "0")
    assert lib.mm1_attn_dkdv_plan(2, 8192, 10, 2, 1, 256, plan) == 0
    assert plan[4] == 0
