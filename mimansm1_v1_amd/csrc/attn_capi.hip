// extern "C" entry points: argument checks, then the kernel launchers.
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include <mutex>

#include "../../include/mm1_attn.h"
#include "../../include/mm1_swiglu.h"
#include "../../include/mm1_lm_head.h"
#include "attn_layout.h"
#include "dispatch_order.h"
#include "mm1_common.h"

namespace mm1 {
hipError_t launch_fwd(const void* q, const void* k, const void* v, void* o, float* lse2, bool f32,
                      _Float16* q16, _Float16* k16, _Float16* v16, uint8_t* o_lo, float* vmax, bool save,
                      int B, int S, int H, int Hkv, bool causal, float sm_scale, int variant, hipStream_t stream);
hipError_t launch_cvt_kv(const void* k, const void* v, _Float16* k16, _Float16* v16, float* kmax, float* vmax,
                         long n, hipStream_t stream);
hipError_t launch_cvt16(const void* x, _Float16* x16, long n, hipStream_t stream);
hipError_t launch_delta(const void* o, const void* dO, float* delta, int B, int S, int H,
                        hipStream_t stream);
hipError_t launch_bwd_prep(const void* o, const uint8_t* o_lo, const void* dO, const float* delta_in,
                           const float* lse2, const float* vmax, char* ws, int B, int S, int H, int Hkv,
                           float sm_scale, hipStream_t stream);
hipError_t launch_bwd_dkdv(const char* state, char* ws, void* dk, void* dv, bool f32, int B, int S, int H,
                           int Hkv, bool causal, float sm_scale, int variant, hipStream_t stream);
hipError_t launch_bwd_reduce(const char* ws, void* dk, void* dv, bool f32, int B, int S, int H, int Hkv,
                             bool causal, int dkdv_variant, hipStream_t stream);
hipError_t launch_bwd_dq(const char* state, char* ws, void* dq, bool reduce, void* dk, void* dv, bool f32,
                         int B, int S, int H, int Hkv, bool causal, float sm_scale, int variant, int dkdv_variant,
                         hipStream_t stream);
size_t bwd_partials_bytes(int B, int S, int H, int Hkv, bool causal, int variant);
size_t qknorm_bwd_workspace_bytes();
hipError_t launch_qknorm_fwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                             const float* sin_t, void* q, void* k, void* v, int B, int S, int H, int Hkv,
                             float eps, hipStream_t stream);
hipError_t launch_swiglu_gate_up(const void* x, const void* wg, const void* wu, void* gate, void* up,
                                 void* act, int T, int d, int F, int mode, hipStream_t stream);
hipError_t launch_swiglu_grad(const void* dact, const void* gate, const void* up, void* dgate, void* dup,
                              int T, int F, long ld_out, hipStream_t stream);
size_t lm_head_workspace_bytes(int T, int V);
hipError_t launch_lm_lse(const void* hidden, const void* weight, const long long* targets, long long ignore_index,
                         float* lse, float* tlogit_out, float* loss, void* workspace, int T, int d, int V,
                         hipStream_t stream);
hipError_t launch_lm_dlogits(const void* hidden, const void* weight, const long long* targets,
                             long long ignore_index, const float* lse, const float* scale, void* dlogits, long ld,
                             int T, int d, int V, int v0, int vn, hipStream_t stream);
hipError_t launch_qknorm_bwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                             const float* sin_t, const void* dq, const void* dk, const void* dv,
                             void* dqkv, float* dwq, float* dwk, void* workspace, int B, int S, int H,
                             int Hkv, float eps, hipStream_t stream);
}  // namespace mm1

namespace {

// Largest sizes the 32-bit index arithmetic inside the kernels allows.
constexpr long kMaxRows = 1L << 30;

int check_shape(int B, int S, int H, int Hkv, int D) {
  if (B < 1 || S < 1 || H < 1 || Hkv < 1 || H % Hkv != 0) return MM1_E_SHAPE;
  if ((long)B * S * H > kMaxRows || (long)(H / Hkv) * S > kMaxRows) return MM1_E_SHAPE;
  if (D != mm1::HD) return MM1_E_HEAD_DIM;
  return MM1_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Tilings compiled into the library (the `variant` argument of launch_fwd,
// launch_bwd_dkdv and launch_bwd_dq).  block_M / block_N name the stationary
// and the streamed block: query rows x key rows for the forward and dQ, key
// rows x query rows for dK/dV.
const char* const kFwdTiles[] = {
    "block_M=256 block_N=64 waves=8 stages=2 schedule=pingpong",
    "block_M=128 block_N=64 waves=4 stages=2 schedule=ring",
    "block_M=256 block_N=64 waves=8 stages=3 schedule=ring",
};
const char* const kDkdvTiles[] = {
    "block_M=128 block_N=32 waves=8 stages=7 schedule=group",
    "block_M=128 block_N=32 waves=8 stages=7 schedule=pipelined",
};
const char* const kDqTiles[] = {
    "block_M=128 block_N=64 waves=4 stages=2 schedule=ring",
    "block_M=256 block_N=64 waves=8 stages=3 schedule=ring",
};

template <size_t N>
constexpr int count(const char* const (&)[N]) { return static_cast<int>(N); }

int tile_count(int kind) {
  switch (kind) {
    case MM1_TILES_FWD: return count(kFwdTiles);
    case MM1_TILES_DKDV: return count(kDkdvTiles);
    case MM1_TILES_DQ: return count(kDqTiles);
    default: return 0;
  }
}

// The tiling to launch: `tiles` itself when >= 0, index 0 (the default) for
// -1; -1 when out of range.
int pick_tiles(int kind, int tiles) {
  if (tiles == -1) tiles = 0;
  return (tiles >= 0 && tiles < tile_count(kind)) ? tiles : -1;
}

// ---------------------------------------------------------------------------
// Layout of the dK/dV partial sums a workspace holds.  mm1_attn_bwd_dkdv*
// records, per workspace address, the layout its launch wrote; the calls that
// sum the partials (mm1_attn_bwd_dkdv_reduce*, mm1_attn_bwd_dq_reduce*) work
// out the layout their own tiling and shape read and refuse (MM1_E_LAYOUT) a
// workspace whose record differs or is missing, instead of summing the wrong
// slots.  The record is host state only (nothing is written to the device);
// it holds the last few workspaces in use.
struct WsLayout {
  const void* ws;
  int grouped;                 // chunked (grouped tilings) or one slot per head
  int L, C, split_keys;        // grouped: the chunk plan (dkdv_plan)
  int B, S, H, Hkv, causal;
  bool same(const WsLayout& o) const {
    return grouped == o.grouped && L == o.L && C == o.C && split_keys == o.split_keys && B == o.B &&
           S == o.S && H == o.H && Hkv == o.Hkv && causal == o.causal;
  }
};

WsLayout layout_of(const void* ws, int dkdv_variant, int B, int S, int H, int Hkv, bool causal) {
  WsLayout l{};
  l.ws = ws;
  l.B = B, l.S = S, l.H = H, l.Hkv = Hkv;
  if (mm1::dkdv_grouped(dkdv_variant)) {
    const mm1::DkdvPlan& plan = mm1::dkdv_plan(B, S, H, Hkv, causal);
    l.grouped = 1;
    l.L = plan.L, l.C = plan.C, l.split_keys = plan.split_keys;
    l.causal = causal ? 1 : 0;
  }
  return l;
}

constexpr int kLayoutSlots = 64;
std::mutex g_layout_mu;
WsLayout g_layouts[kLayoutSlots];
int g_layout_next = 0;

void record_layout(const WsLayout& l) {
  std::lock_guard<std::mutex> lock(g_layout_mu);
  for (WsLayout& e : g_layouts) {
    if (e.ws == l.ws) {
      e = l;
      return;
    }
  }
  g_layouts[g_layout_next] = l;
  g_layout_next = (g_layout_next + 1) % kLayoutSlots;
}

bool layout_matches(const WsLayout& want) {
  std::lock_guard<std::mutex> lock(g_layout_mu);
  for (const WsLayout& e : g_layouts)
    if (e.ws == want.ws) return e.same(want);
  return false;
}

int from_hip(hipError_t e) { return e == hipSuccess ? MM1_OK : static_cast<int>(e); }

// ---------------------------------------------------------------------------
// Scratch of mm1_attn_bwd_noalloc: the backward workspace of the default
// tilings (fp16 dO, Delta, the dK/dV partial sums) lives in this static
// device array instead of a buffer the caller allocates.  Every device the
// library runs on holds its own copy (MM1_NOALLOC_SCRATCH_BYTES) until the
// process ends.  In host code `scratch` is only a handle: its device address
// on the current device comes from hipGetSymbolAddress, taken once per
// device and kept in g_scratch_addr.
static __device__ __align__(256) char scratch[MM1_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices];

// The current device's address of `scratch` (MM1_OK), or an error code.
int scratch_addr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return from_hip(e);
  if (dev < 0 || dev >= kMaxDevices) return MM1_E_SHAPE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return from_hip(e);
    if (!p) return MM1_E_NULL;
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return MM1_OK;
}

bool bad_scale(float sm_scale) { return !(sm_scale > 0.f) || !isfinite(sm_scale); }

// Bytes of the backward workspace when its partial sums are those of dK/dV
// tiling `variant` (the regions before them are fixed).
size_t ws_bytes_for(int B, int S, int H, int Hkv, bool causal, int variant) {
  return mm1::bwd_ws(B, S, H, Hkv).partials + mm1::bwd_partials_bytes(B, S, H, Hkv, causal, variant);
}

// Argument checks shared by the calls that read a forward state and a
// prepared backward workspace.
int check_state_ws(const void* state, size_t state_bytes, const void* ws, size_t ws_bytes, int B, int S, int H,
                   int Hkv) {
  if (!state || !ws) return MM1_E_NULL;
  if (state_bytes < mm1::fwd_state(B, S, H, Hkv).bytes || ws_bytes < mm1::bwd_ws(B, S, H, Hkv).bytes)
    return MM1_E_WORKSPACE;
  if (!aligned16(state) || !aligned16(ws)) return MM1_E_ALIGN;
  return MM1_OK;
}

int fwd_any(const void* q, const void* k, const void* v, void* o, float* lse2, bool f32, void* state,
            size_t state_bytes, int B, int S, int H, int Hkv, int D, int causal, float sm_scale, int tiles,
            void* stream) {
  if (!q || !k || !v || !o || !lse2 || !state) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (bad_scale(sm_scale)) return MM1_E_SCALE;
  if (state_bytes < mm1::fwd_state(B, S, H, Hkv).bytes) return MM1_E_WORKSPACE;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(state)) return MM1_E_ALIGN;
  const int variant = pick_tiles(MM1_TILES_FWD, tiles);
  if (variant < 0) return MM1_E_TILES;
  const mm1::FwdState f = mm1::fwd_state(B, S, H, Hkv);
  char* st = static_cast<char*>(state);
  return from_hip(mm1::launch_fwd(q, k, v, o, lse2, f32, reinterpret_cast<_Float16*>(st + f.q16),
                                  reinterpret_cast<_Float16*>(st + f.k16), reinterpret_cast<_Float16*>(st + f.v16),
                                  reinterpret_cast<uint8_t*>(st + f.olo), reinterpret_cast<float*>(st + f.vmax), true,
                                  B, S, H, Hkv, causal != 0, sm_scale, variant, static_cast<hipStream_t>(stream)));
}

int bwd_prep_any(const void* o, const void* dO, const float* delta_in, const float* lse2, const void* state,
                 size_t state_bytes, void* ws, size_t ws_bytes, int B, int S, int H, int Hkv, int D, float sm_scale,
                 void* stream) {
  if (!dO || !lse2) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (bad_scale(sm_scale)) return MM1_E_SCALE;
  if ((rc = check_state_ws(state, state_bytes, ws, ws_bytes, B, S, H, Hkv))) return rc;
  if (!aligned16(dO) || (o && !aligned16(o))) return MM1_E_ALIGN;
  const mm1::FwdState f = mm1::fwd_state(B, S, H, Hkv);
  const char* st = static_cast<const char*>(state);
  return from_hip(mm1::launch_bwd_prep(o, reinterpret_cast<const uint8_t*>(st + f.olo), dO, delta_in, lse2,
                                       reinterpret_cast<const float*>(st + f.vmax), static_cast<char*>(ws), B, S,
                                       H, Hkv, sm_scale, static_cast<hipStream_t>(stream)));
}

int bwd_dkdv(const void* state, size_t state_bytes, void* dk, void* dv, bool f32, void* ws, size_t ws_bytes,
             int B, int S, int H, int Hkv, int D, int causal, float sm_scale, int tiles, void* stream) {
  if (!dk || !dv) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (bad_scale(sm_scale)) return MM1_E_SCALE;
  if ((rc = check_state_ws(state, state_bytes, ws, ws_bytes, B, S, H, Hkv))) return rc;
  if (!aligned16(dk) || !aligned16(dv)) return MM1_E_ALIGN;
  const int variant = pick_tiles(MM1_TILES_DKDV, tiles);
  if (variant < 0) return MM1_E_TILES;
  rc = from_hip(mm1::launch_bwd_dkdv(static_cast<const char*>(state), static_cast<char*>(ws), dk, dv, f32, B, S,
                                     H, Hkv, causal != 0, sm_scale, variant, static_cast<hipStream_t>(stream)));
  if (rc == MM1_OK && H / Hkv > 1) record_layout(layout_of(ws, variant, B, S, H, Hkv, causal != 0));
  return rc;
}

// dq, and with `reduce` the group sum of the dK/dV partials in the same launch.
int bwd_dq(const void* state, size_t state_bytes, void* dq, void* dk, void* dv, bool reduce, bool f32, void* ws,
           size_t ws_bytes, int B, int S, int H, int Hkv, int D, int causal, float sm_scale, int tiles,
           int dkdv_tiles, void* stream) {
  if (!dq) return MM1_E_NULL;
  if (reduce && (!dk || !dv)) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (bad_scale(sm_scale)) return MM1_E_SCALE;
  if ((rc = check_state_ws(state, state_bytes, ws, ws_bytes, B, S, H, Hkv))) return rc;
  if (!aligned16(dq) || (reduce && (!aligned16(dk) || !aligned16(dv)))) return MM1_E_ALIGN;
  const int variant = pick_tiles(MM1_TILES_DQ, tiles);
  const int dkdv_variant = pick_tiles(MM1_TILES_DKDV, dkdv_tiles);
  if (variant < 0 || dkdv_variant < 0) return MM1_E_TILES;
  if (reduce && H / Hkv > 1 && !layout_matches(layout_of(ws, dkdv_variant, B, S, H, Hkv, causal != 0)))
    return MM1_E_LAYOUT;
  return from_hip(mm1::launch_bwd_dq(static_cast<const char*>(state), static_cast<char*>(ws), dq, reduce, dk, dv,
                                     f32, B, S, H, Hkv, causal != 0, sm_scale, variant, dkdv_variant,
                                     static_cast<hipStream_t>(stream)));
}

int bwd_reduce(void* ws, size_t ws_bytes, void* dk, void* dv, int B, int S, int H, int Hkv, int D, int causal,
               int dkdv_tiles, void* stream) {
  if (!ws || !dk || !dv) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  const int dkdv_variant = pick_tiles(MM1_TILES_DKDV, dkdv_tiles);
  if (dkdv_variant < 0) return MM1_E_TILES;
  if (ws_bytes < mm1::bwd_ws(B, S, H, Hkv).bytes) return MM1_E_WORKSPACE;
  if (!aligned16(ws) || !aligned16(dk) || !aligned16(dv)) return MM1_E_ALIGN;
  if (H / Hkv <= 1) return MM1_OK;
  if (!layout_matches(layout_of(ws, dkdv_variant, B, S, H, Hkv, causal != 0))) return MM1_E_LAYOUT;
  return from_hip(mm1::launch_bwd_reduce(static_cast<const char*>(ws), dk, dv, false, B, S, H, Hkv, causal != 0,
                                         dkdv_variant, static_cast<hipStream_t>(stream)));
}

// The whole backward: prep, dK/dV, dQ with the partial sum in its tail.
int bwd_all(const void* o, const void* dO, const float* lse2, const void* state, size_t state_bytes, void* dq,
            void* dk, void* dv, bool f32, void* ws, size_t ws_bytes, int B, int S, int H, int Hkv, int D,
            int causal, float sm_scale, int dkdv_tiles, int dq_tiles, void* stream) {
  // what only the later launches check is checked first, so that an
  // argument error launches nothing
  if (!o || !dO || !lse2 || !dq || !dk || !dv) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (bad_scale(sm_scale)) return MM1_E_SCALE;
  if ((rc = check_state_ws(state, state_bytes, ws, ws_bytes, B, S, H, Hkv))) return rc;
  if (!aligned16(o) || !aligned16(dO) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv)) return MM1_E_ALIGN;
  if (pick_tiles(MM1_TILES_DQ, dq_tiles) < 0 || pick_tiles(MM1_TILES_DKDV, dkdv_tiles) < 0) return MM1_E_TILES;
  if ((rc = bwd_prep_any(o, dO, nullptr, lse2, state, state_bytes, ws, ws_bytes, B, S, H, Hkv, D, sm_scale,
                         stream)))
    return rc;
  if ((rc = bwd_dkdv(state, state_bytes, dk, dv, f32, ws, ws_bytes, B, S, H, Hkv, D, causal, sm_scale, dkdv_tiles,
                     stream)))
    return rc;
  return bwd_dq(state, state_bytes, dq, dk, dv, true, f32, ws, ws_bytes, B, S, H, Hkv, D, causal, sm_scale,
                dq_tiles, dkdv_tiles, stream);
}

}  // namespace

extern "C" {

int mm1_attn_version(void) { return MM1_ATTN_VERSION; }

size_t mm1_attn_fwd_state_size(int B, int S, int H, int Hkv, int D) {
  if (check_shape(B, S, H, Hkv, D) != MM1_OK) return 0;
  return mm1::fwd_state(B, S, H, Hkv).bytes;
}

int mm1_attn_fwd_tiles(const void* q, const void* k, const void* v, void* o, float* lse2, void* state,
                       size_t state_bytes, int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                       int tiles, void* stream) {
  return fwd_any(q, k, v, o, lse2, false, state, state_bytes, B, S, H, Hkv, D, causal, sm_scale, tiles, stream);
}

int mm1_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse2, void* state,
                 size_t state_bytes, int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                 void* stream) {
  return fwd_any(q, k, v, o, lse2, false, state, state_bytes, B, S, H, Hkv, D, causal, sm_scale, -1, stream);
}

int mm1_attn_fwd_f32(const void* q, const void* k, const void* v, float* o, float* lse2, void* state,
                     size_t state_bytes, int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                     int tiles, void* stream) {
  return fwd_any(q, k, v, o, lse2, true, state, state_bytes, B, S, H, Hkv, D, causal, sm_scale, tiles, stream);
}

int mm1_attn_prep(const void* q, const void* k, const void* v, void* state, size_t state_bytes,
                  int B, int S, int H, int Hkv, int D, void* stream) {
  if (!q || !k || !v || !state) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (state_bytes < mm1::fwd_state(B, S, H, Hkv).bytes) return MM1_E_WORKSPACE;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(state)) return MM1_E_ALIGN;
  const mm1::FwdState f = mm1::fwd_state(B, S, H, Hkv);
  char* st = static_cast<char*>(state);
  const hipStream_t sm = static_cast<hipStream_t>(stream);
  rc = from_hip(mm1::launch_cvt_kv(k, v, reinterpret_cast<_Float16*>(st + f.k16),
                                   reinterpret_cast<_Float16*>(st + f.v16), nullptr,
                                   reinterpret_cast<float*>(st + f.vmax), (long)B * S * Hkv * mm1::HD, sm));
  if (rc) return rc;
  return from_hip(mm1::launch_cvt16(q, reinterpret_cast<_Float16*>(st + f.q16), (long)B * S * H * mm1::HD, sm));
}

int mm1_attn_tile_count(int kind) { return tile_count(kind); }

const char* mm1_attn_tile_desc(int kind, int index) {
  if (index < 0 || index >= tile_count(kind)) return nullptr;
  switch (kind) {
    case MM1_TILES_FWD: return kFwdTiles[index];
    case MM1_TILES_DKDV: return kDkdvTiles[index];
    default: return kDqTiles[index];
  }
}

int mm1_attn_delta(const void* o, const void* dO, float* delta, int B, int S, int H, int D,
                   void* stream) {
  if (!o || !dO || !delta) return MM1_E_NULL;
  int rc = check_shape(B, S, H, 1, D);
  if (rc) return rc;
  if (!aligned16(o) || !aligned16(dO)) return MM1_E_ALIGN;
  return from_hip(mm1::launch_delta(o, dO, delta, B, S, H, static_cast<hipStream_t>(stream)));
}

size_t mm1_attn_bwd_workspace_size(int B, int S, int H, int Hkv, int D) {
  if (check_shape(B, S, H, Hkv, D) != MM1_OK) return 0;
  return mm1::bwd_ws(B, S, H, Hkv).bytes;
}

int mm1_attn_bwd_prep(const void* o, const void* dO, const float* lse2, const void* state, size_t state_bytes,
                      void* workspace, size_t workspace_bytes, int B, int S, int H, int Hkv, int D, float sm_scale,
                      void* stream) {
  if (!o) return MM1_E_NULL;
  return bwd_prep_any(o, dO, nullptr, lse2, state, state_bytes, workspace, workspace_bytes, B, S, H, Hkv, D,
                      sm_scale, stream);
}

int mm1_attn_bwd_prep_delta(const void* dO, const float* delta, const float* lse2, const void* state,
                            size_t state_bytes, void* workspace, size_t workspace_bytes, int B, int S, int H, int Hkv,
                            int D, float sm_scale, void* stream) {
  if (!delta) return MM1_E_NULL;
  return bwd_prep_any(nullptr, dO, delta, lse2, state, state_bytes, workspace, workspace_bytes, B, S, H, Hkv, D,
                      sm_scale, stream);
}

int mm1_attn_bwd_dkdv_tiles(const void* state, size_t state_bytes, void* dk, void* dv, void* workspace,
                            size_t workspace_bytes, int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                            int dkdv_tiles, void* stream) {
  return bwd_dkdv(state, state_bytes, dk, dv, false, workspace, workspace_bytes, B, S, H, Hkv, D, causal, sm_scale,
                  dkdv_tiles, stream);
}

int mm1_attn_bwd_dkdv_reduce_tiles(void* workspace, size_t workspace_bytes, void* dk, void* dv, int B, int S,
                                   int H, int Hkv, int D, int causal, int dkdv_tiles, void* stream) {
  return bwd_reduce(workspace, workspace_bytes, dk, dv, B, S, H, Hkv, D, causal, dkdv_tiles, stream);
}

int mm1_attn_bwd_dq_tiles(const void* state, size_t state_bytes, void* dq, void* workspace, size_t workspace_bytes,
                          int B, int S, int H, int Hkv, int D, int causal, float sm_scale, int dq_tiles, void* stream) {
  return bwd_dq(state, state_bytes, dq, nullptr, nullptr, false, false, workspace, workspace_bytes, B, S, H, Hkv, D,
                causal, sm_scale, dq_tiles, -1, stream);
}

int mm1_attn_bwd_dq_reduce_tiles(const void* state, size_t state_bytes, void* dq, void* dk, void* dv,
                                 void* workspace, size_t workspace_bytes, int B, int S, int H, int Hkv, int D,
                                 int causal, float sm_scale, int dkdv_tiles, int dq_tiles, void* stream) {
  return bwd_dq(state, state_bytes, dq, dk, dv, true, false, workspace, workspace_bytes, B, S, H, Hkv, D, causal,
                sm_scale, dq_tiles, dkdv_tiles, stream);
}

int mm1_attn_bwd_tiles(const void* o, const void* dO, const float* lse2, const void* state, size_t state_bytes,
                       void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, int B, int S, int H,
                       int Hkv, int D, int causal, float sm_scale, int dkdv_tiles, int dq_tiles, void* stream) {
  return bwd_all(o, dO, lse2, state, state_bytes, dq, dk, dv, false, workspace, workspace_bytes, B, S, H, Hkv, D,
                 causal, sm_scale, dkdv_tiles, dq_tiles, stream);
}

int mm1_attn_bwd(const void* o, const void* dO, const float* lse2, const void* state, size_t state_bytes, void* dq,
                 void* dk, void* dv, void* workspace, size_t workspace_bytes, int B, int S, int H, int Hkv, int D,
                 int causal, float sm_scale, void* stream) {
  return bwd_all(o, dO, lse2, state, state_bytes, dq, dk, dv, false, workspace, workspace_bytes, B, S, H, Hkv, D,
                 causal, sm_scale, -1, -1, stream);
}

int mm1_attn_bwd_f32_tiles(const void* o, const void* dO, const float* lse2, const void* state, size_t state_bytes,
                           float* dq, float* dk, float* dv, void* workspace, size_t workspace_bytes, int B, int S,
                           int H, int Hkv, int D, int causal, float sm_scale, int dkdv_tiles, int dq_tiles,
                           void* stream) {
  return bwd_all(o, dO, lse2, state, state_bytes, dq, dk, dv, true, workspace, workspace_bytes, B, S, H, Hkv, D,
                 causal, sm_scale, dkdv_tiles, dq_tiles, stream);
}

int mm1_attn_bwd_noalloc(const void* o, const void* dO, const float* lse2, const void* state, size_t state_bytes,
                         void* dq, void* dk, void* dv, int B, int S, int H, int Hkv, int D, int causal,
                         float sm_scale, void* stream) {
  if (!o || !dO || !lse2 || !state || !dq || !dk || !dv) return MM1_E_NULL;
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (bad_scale(sm_scale)) return MM1_E_SCALE;
  if (state_bytes < mm1::fwd_state(B, S, H, Hkv).bytes) return MM1_E_WORKSPACE;
  if (!aligned16(o) || !aligned16(dO) || !aligned16(state) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv))
    return MM1_E_ALIGN;
  const size_t need = ws_bytes_for(B, S, H, Hkv, causal != 0, 0);
  if (need > MM1_NOALLOC_SCRATCH_BYTES) return MM1_E_SCRATCH;
  void* ws = nullptr;
  if ((rc = scratch_addr(&ws)) != MM1_OK) return rc;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const mm1::FwdState f = mm1::fwd_state(B, S, H, Hkv);
  const char* sp = static_cast<const char*>(state);
  char* wp = static_cast<char*>(ws);
  rc = from_hip(mm1::launch_bwd_prep(o, reinterpret_cast<const uint8_t*>(sp + f.olo), dO, nullptr, lse2,
                                     reinterpret_cast<const float*>(sp + f.vmax), wp, B, S, H, Hkv, sm_scale, st));
  if (rc) return rc;
  rc = from_hip(mm1::launch_bwd_dkdv(sp, wp, dk, dv, false, B, S, H, Hkv, causal != 0, sm_scale, 0, st));
  if (rc) return rc;
  return from_hip(mm1::launch_bwd_dq(sp, wp, dq, true, dk, dv, false, B, S, H, Hkv, causal != 0, sm_scale, 0, 0,
                                     st));
}

size_t mm1_attn_bwd_noalloc_scratch_size(int B, int S, int H, int Hkv, int D, int causal) {
  if (check_shape(B, S, H, Hkv, D) != MM1_OK) return 0;
  return ws_bytes_for(B, S, H, Hkv, causal != 0, 0);
}

int mm1_attn_dispatch_order(int kind, int tiles, int B, int S, int H, int Hkv, int causal, int cus,
                            unsigned short* out, int cap) {
  if (kind < MM1_TILES_FWD || kind > MM1_TILES_DQ) return MM1_E_TILES;
  const int variant = pick_tiles(kind, tiles);
  if (variant < 0) return MM1_E_TILES;
  if (const int rc = check_shape(B, S, H, Hkv, mm1::HD)) return rc;
  if (cus < 1 || cap < 0) return MM1_E_SHAPE;
  if (cap > 0 && !out) return MM1_E_NULL;
  if (kind == MM1_TILES_DKDV && !mm1::dkdv_grouped(variant)) return 0;   // per-head grids: default order
  const mm1::DispatchOrder& ord =
      kind == MM1_TILES_DKDV ? mm1::dkdv_plan_for(B, S, H, Hkv, causal != 0, cus).order
      : kind == MM1_TILES_DQ ? mm1::dispatch_order_for(mm1::dq_grid(variant, B, S, H, Hkv), causal != 0, cus)
                             : mm1::dispatch_order_for(mm1::row_block_grid(variant, B, S, H, Hkv), causal != 0, cus);
  for (int i = 0; i < ord.n && i < cap; ++i) out[i] = ord.item[i];
  return ord.n;
}

int mm1_attn_dkdv_plan(int B, int S, int H, int Hkv, int causal, int cus, int* out) {
  if (!out) return MM1_E_NULL;
  if (const int rc = check_shape(B, S, H, Hkv, mm1::HD)) return rc;
  if (cus < 1) return MM1_E_SHAPE;
  const mm1::DkdvPlan& plan = mm1::dkdv_plan_for(B, S, H, Hkv, causal != 0, cus);
  out[0] = plan.L;
  out[1] = plan.C;
  out[2] = plan.split_keys;
  out[3] = plan.n_items;
  out[4] = plan.order.n;
  return MM1_OK;
}

static int check_qknorm(int B, int S, int H, int Hkv, int D, int rot_len, float eps, bool norm) {
  int rc = check_shape(B, S, H, Hkv, D);
  if (rc) return rc;
  if (S > rot_len) return MM1_E_SHAPE;
  if (norm && !(eps > 0.f && isfinite(eps))) return MM1_E_SCALE;
  return MM1_OK;
}

int mm1_qknorm_rope_fwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                        const float* sin_t, void* q, void* k, void* v,
                        int B, int S, int H, int Hkv, int D, int rot_len, float eps, void* stream) {
  if (!qkv || !cos_t || !sin_t || !q || !k || !v || (!wq) != (!wk)) return MM1_E_NULL;
  int rc = check_qknorm(B, S, H, Hkv, D, rot_len, eps, wq != nullptr);
  if (rc) return rc;
  if (!aligned16(qkv) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(cos_t) ||
      !aligned16(sin_t))
    return MM1_E_ALIGN;
  return from_hip(mm1::launch_qknorm_fwd(qkv, wq, wk, cos_t, sin_t, q, k, v, B, S, H, Hkv, eps,
                                         static_cast<hipStream_t>(stream)));
}

size_t mm1_qknorm_rope_bwd_workspace_size(void) { return mm1::qknorm_bwd_workspace_bytes(); }

int mm1_qknorm_rope_bwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                        const float* sin_t, const void* dq, const void* dk, const void* dv,
                        void* dqkv, float* dwq, float* dwk, void* workspace, size_t workspace_bytes,
                        int B, int S, int H, int Hkv, int D, int rot_len, float eps, void* stream) {
  if (!qkv || !cos_t || !sin_t || !dq || !dk || !dv || !dqkv || (!wq) != (!wk)) return MM1_E_NULL;
  if (wq && (!dwq || !dwk)) return MM1_E_NULL;
  int rc = check_qknorm(B, S, H, Hkv, D, rot_len, eps, wq != nullptr);
  if (rc) return rc;
  if (wq && (!workspace || workspace_bytes < mm1::qknorm_bwd_workspace_bytes())) return MM1_E_WORKSPACE;
  if (!aligned16(qkv) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) || !aligned16(dqkv) ||
      !aligned16(cos_t) || !aligned16(sin_t))
    return MM1_E_ALIGN;
  return from_hip(mm1::launch_qknorm_bwd(qkv, wq, wk, cos_t, sin_t, dq, dk, dv, dqkv, dwq, dwk,
                                         workspace, B, S, H, Hkv, eps, static_cast<hipStream_t>(stream)));
}

// Largest token count: keeps T * ffn / 8 and the row arithmetic well inside
// the kernels' integer ranges.
constexpr long kMaxTokens = 1L << 26;

static int check_swiglu_shape(int T, int d, int F) {
  if (T < 1 || (long)T > kMaxTokens || d < 128 || d % 128 != 0 || F < 128 || F % 128 != 0)
    return MM1_E_SHAPE;
  // 32-bit byte offsets inside x and the weights (the kernel's DMA addressing)
  if ((long)T * d >= (1L << 30) || (long)d * F >= (1L << 30) || (long)T * F > (1L << 40)) return MM1_E_SHAPE;
  return MM1_OK;
}

int mm1_swiglu_gate_up(const void* x, const void* w_gate, const void* w_up, void* gate, void* up,
                       void* act, int T, int d_model, int ffn, int mode, void* stream) {
  if (mode < MM1_SWIGLU_ACT || mode > MM1_SWIGLU_TRAIN) return MM1_E_SHAPE;
  const bool split = mode != MM1_SWIGLU_ACT, with_act = mode != MM1_SWIGLU_SPLIT;
  if (!x || !w_gate || !w_up || (split && (!gate || !up)) || (with_act && !act)) return MM1_E_NULL;
  int rc = check_swiglu_shape(T, d_model, ffn);
  if (rc) return rc;
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || (split && (!aligned16(gate) || !aligned16(up))) ||
      (with_act && !aligned16(act)))
    return MM1_E_ALIGN;
  return from_hip(mm1::launch_swiglu_gate_up(x, w_gate, w_up, gate, up, act, T, d_model, ffn, mode,
                                             static_cast<hipStream_t>(stream)));
}

int mm1_swiglu_grad(const void* d_act, const void* gate, const void* up, void* d_gate, void* d_up,
                    int T, int ffn, long ld_out, void* stream) {
  if (!d_act || !gate || !up || !d_gate || !d_up) return MM1_E_NULL;
  if (T < 1 || (long)T > kMaxTokens || ffn < 8 || ffn % 8 != 0 || ld_out < ffn || ld_out % 8 != 0)
    return MM1_E_SHAPE;
  if (!aligned16(d_act) || !aligned16(gate) || !aligned16(up) || !aligned16(d_gate) || !aligned16(d_up))
    return MM1_E_ALIGN;
  return from_hip(mm1::launch_swiglu_grad(d_act, gate, up, d_gate, d_up, T, ffn, ld_out,
                                          static_cast<hipStream_t>(stream)));
}

static int check_lm_shape(int T, int d, int V) {
  if (T < 1 || (long)T > kMaxTokens || d < 128 || d % 128 != 0 || V < 128 || V % 128 != 0) return MM1_E_SHAPE;
  // 32-bit byte offsets inside hidden and a 64-row slab of the weight
  if ((long)T * d >= (1L << 30) || 64L * V >= (1L << 30)) return MM1_E_SHAPE;
  return MM1_OK;
}

size_t mm1_lm_head_workspace_size(int T, int vocab) {
  if (check_lm_shape(T, 128, vocab) != MM1_OK) return 0;
  return mm1::lm_head_workspace_bytes(T, vocab);
}

int mm1_lm_head_lse(const void* hidden, const void* weight, const long long* targets, long long ignore_index,
                    float* lse, float* target_logit, float* loss, void* workspace, size_t workspace_bytes,
                    int T, int d_model, int vocab, void* stream) {
  if (!hidden || !weight || !lse) return MM1_E_NULL;
  if (!targets && (target_logit || loss)) return MM1_E_NULL;
  int rc = check_lm_shape(T, d_model, vocab);
  if (rc) return rc;
  if (!workspace || workspace_bytes < mm1::lm_head_workspace_bytes(T, vocab)) return MM1_E_WORKSPACE;
  if (!aligned16(hidden) || !aligned16(weight) || !aligned16(workspace)) return MM1_E_ALIGN;
  return from_hip(mm1::launch_lm_lse(hidden, weight, targets, ignore_index, lse, target_logit, loss, workspace,
                                     T, d_model, vocab, static_cast<hipStream_t>(stream)));
}

int mm1_lm_head_dlogits(const void* hidden, const void* weight, const long long* targets, long long ignore_index,
                        const float* lse, const float* scale, void* d_logits, long ld,
                        int T, int d_model, int vocab, int v0, int vn, void* stream) {
  if (!hidden || !weight || !targets || !lse || !scale || !d_logits) return MM1_E_NULL;
  int rc = check_lm_shape(T, d_model, vocab);
  if (rc) return rc;
  if (v0 < 0 || vn < 128 || v0 % 128 != 0 || vn % 128 != 0 || (long)v0 + vn > vocab || ld < vn || ld % 8 != 0)
    return MM1_E_SHAPE;
  if (!aligned16(hidden) || !aligned16(weight) || !aligned16(d_logits)) return MM1_E_ALIGN;
  return from_hip(mm1::launch_lm_dlogits(hidden, weight, targets, ignore_index, lse, scale, d_logits, ld, T,
                                         d_model, vocab, v0, vn, static_cast<hipStream_t>(stream)));
}

const char* mm1_attn_strerror(int code) {
  switch (code) {
    case MM1_OK: return "success";
    case MM1_E_NULL: return "mm1_attn: a required pointer is NULL";
    case MM1_E_SHAPE: return "mm1_attn: bad shape (need B, S, H, Hkv >= 1 and H % Hkv == 0)";
    case MM1_E_HEAD_DIM: return "mm1_attn: head_dim must be 128";
    case MM1_E_WORKSPACE: return "mm1_attn: workspace smaller than mm1_attn_bwd_workspace_size()";
    case MM1_E_SCALE: return "mm1_attn: sm_scale must be a positive finite number";
    case MM1_E_ALIGN: return "mm1_attn: tensor pointers must be 16-byte aligned";
    case MM1_E_TILES: return "mm1_attn: tiling index out of range (see mm1_attn_tile_count)";
    case MM1_E_SCRATCH:
      return "mm1_attn: the dK/dV partial sums of this shape exceed the static scratch of "
             "mm1_attn_bwd_noalloc (MM1_NOALLOC_SCRATCH_BYTES); use mm1_attn_bwd with a workspace";
    case MM1_E_LAYOUT:
      return "mm1_attn: the workspace holds no dK/dV partial sums of this shape and dK/dV tiling "
             "(run mm1_attn_bwd_dkdv with the same arguments first)";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "mm1_attn: unknown error";
}

}  // extern "C"
