// Causal / full GQA flash-attention backward for gfx950.
//
// The reference computes the backward as one KV-stationary kernel that pushes
// dQ, dK and dV out with fp32 atomics (flash_delta / flash_bwd,
// CODE/mimans/model/attention_tilelang.py:192-217 and :242-323).  The
// arithmetic kept from it:
//   Delta_i = sum_d O_id dO_id                     (:212-214)
//   P_ij    = exp2(s_ij * scale2 - lse2_i)         (:297), zero above the diagonal (:298-301)
//   dP_ij   = dO_i . V_j                           (:304)
//   dV_j   += sum_i P_ij dO_i                      (:307)
//   dS_ij   = P_ij (dP_ij - Delta_i) sm_scale      (:310)
//   dK_j   += sum_i dS_ij Q_i                       (:311)
//   dQ_i   += sum_j dS_ij K_j                       (:314)
// The reference rounds P and dS to bf16 before their products and takes
// Delta from its bf16 O; here P and dS are rounded to fp16 (11 significant
// bits), Delta is formed from 15 significant bits of the forward's O (the
// bf16 O and its residual byte), and all products run on fp16 copies of Q,
// K, V and of dO scaled by a power of two 2^E (attn_delta16_kernel,
// attn_do16_kernel).  sm_scale enters through lse = lse2 - log2(sm_scale):
// exp2(s scale2 - lse) = P sm_scale, so dS is one multiply.
//
// The decomposition here is atomic-free and deterministic:
//   * attn_delta16_kernel / attn_do16_kernel : Delta, fp16 dO and its scale
//     (attn_delta_kernel is the reference's flash_delta on the bf16 O).
//   * attn_dkdv_pipe_kernel : key-stationary.  Each wave pair keeps 32 keys
//     of K and V and their dK/dV accumulators in registers while it walks
//     query tiles, which arrive in LDS by DMA (row-major; transposed operands
//     are read with the LDS transpose read).  The default (grouped) tiling
//     gives a workgroup one 128-key tile of one KV head and walks the query
//     tiles of all G heads of the group, so the group sum stays in
//     registers; only the long key tiles of a causal grid are split into
//     chunks, whose fp32 partials go to a workspace [chunk][B][S][Hkv][D].
//     The per-head tiling gives a workgroup one (128-key tile, query head)
//     and writes a partial per head.  The partials are summed in a fixed
//     order and rounded once (in the dQ launch's tail, or
//     attn_dkdv_reduce_kernel).
//   * attn_dq_kernel      : query-stationary over the packed GQA row space
//     (as in the forward): K/V tiles in LDS serve all G heads of a group and
//     dQ is written once in bf16 -- no fp32 scratch and no un-swizzle pass.
#include <type_traits>

#include "dispatch_order.h"
#include "attn_layout.h"
#include "mm1_common.h"

// k-steps by which the dQ kernel's K / V row reads run ahead of their
// products (1: dQ 2% faster than 0; 2 measured no faster than 1).
#ifndef MM1_DQ_PREFETCH
#define MM1_DQ_PREFETCH 1
#endif

// Products by which the dK/dV kernel's LDS operand reads run ahead of their
// products: Q / dO row fragments of the S / dP products, transposed dO / Q
// fragments (two reads each) of the dV^T / dK^T accumulations.
#ifndef MM1_DKDV_PF_ROWS
#define MM1_DKDV_PF_ROWS 2
#endif
#ifndef MM1_DKDV_PF_TR
#define MM1_DKDV_PF_TR 2
#endif

namespace mm1 {

// ---------------------------------------------------------------------------
// Delta = rowsum(O * dO) in fp32.  A 16-lane group reads two consecutive
// (b, s, h) rows (512 contiguous bytes of each tensor), so every lane has four
// 16-byte loads in flight.
__global__ __launch_bounds__(256) void attn_delta_kernel(
    const __bf16* __restrict__ o, const __bf16* __restrict__ dO, float* __restrict__ delta,
    int B, int S, int H) {
  const long nrows = (long)B * S * H;
  const long row0 = (((long)blockIdx.x * 256 + threadIdx.x) >> 4) * 2;
  const int c = threadIdx.x & 15;
  if (row0 >= nrows) return;   // whole 16-lane groups leave together
  const long row1 = min(row0 + 1, nrows - 1);
  const bf16x8 a0 = *reinterpret_cast<const bf16x8*>(o + row0 * HD + 8 * c);
  const bf16x8 d0 = *reinterpret_cast<const bf16x8*>(dO + row0 * HD + 8 * c);
  const bf16x8 a1 = *reinterpret_cast<const bf16x8*>(o + row1 * HD + 8 * c);
  const bf16x8 d1 = *reinterpret_cast<const bf16x8*>(dO + row1 * HD + 8 * c);
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    acc0 = fmaf((float)a0[t], (float)d0[t], acc0);
    acc1 = fmaf((float)a1[t], (float)d1[t], acc1);
  }
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) {
    acc0 += __shfl_xor(acc0, m);
    acc1 += __shfl_xor(acc1, m);
  }
  if (c == 0) {
    auto put = [&](long row, float v) {
      const int hh = (int)(row % H);
      const long bs = row / H;
      const int sp = (int)(bs % S);
      const int bb = (int)(bs / S);
      delta[((long)bb * H + hh) * S + sp] = v;
    };
    put(row0, acc0);
    if (row0 + 1 < nrows) put(row0 + 1, acc1);
  }
}

// ---------------------------------------------------------------------------
// Backward preprocess of the state-based backward (mm1_attn_bwd_prep).
//
// dO is used by the products as do16 = fp16(2^E dO), with E from max|dO| and
// max|V| (do_scale_exp).  E = 0 whenever that is safe, so the common case
// converts dO in the same pass that computes Delta and finds max|dO|; a
// second launch (attn_do16_kernel) reconverts dO with 2^E only when E != 0.
//
// attn_delta16_kernel:
//   Delta_i = sum_d O_id dO_id in fp32, O from the bf16 output and its
//   residual byte (lo8_decode: 15 significant bits of the forward's fp32 O);
//   with o == nullptr the caller's Delta is copied (mm1_attn_bwd_prep_delta).
//   It stores -Delta (the products accumulate dP - Delta onto it) and
//   lse = lse2 - log2(sm_scale) (so exp2(s scale2 - lse) is P sm_scale, the
//   scaled softmax weight dS is formed from), both per (b, h, s) row.
//   do16 = fp16(dO) (E = 0), and max|dO| of the workgroup's rows in
//   part_max[blockIdx.x].  16 lanes per (b, s, h) row, grid-stride over pairs
//   of rows.
__global__ __launch_bounds__(256) void attn_delta16_kernel(
    const __bf16* __restrict__ o, const uint8_t* __restrict__ o_lo, const __bf16* __restrict__ dO,
    const float* __restrict__ delta_in, const float* __restrict__ lse2, float log2_sm_scale,
    float* __restrict__ ndelta, float* __restrict__ lse, _Float16* __restrict__ do16,
    float* __restrict__ part_max, int B, int S, int H) {
  const long nrows = (long)B * S * H;
  const int c = threadIdx.x & 15;
  float mx = 0.f;
  for (long row0 = (((long)blockIdx.x * 256 + threadIdx.x) >> 4) * 2; row0 < nrows;
       row0 += (long)gridDim.x * 32) {
    const long row1 = min(row0 + 1, nrows - 1);
    const bf16x8 d0 = *reinterpret_cast<const bf16x8*>(dO + row0 * HD + 8 * c);
    const bf16x8 d1 = *reinterpret_cast<const bf16x8*>(dO + row1 * HD + 8 * c);
    f16x8 h0, h1;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float f0 = (float)d0[t], f1 = (float)d1[t];
      mx = fmaxf(mx, fmaxf(fabsf(f0), fabsf(f1)));
      h0[t] = (_Float16)f0;
      h1[t] = (_Float16)f1;
    }
    *reinterpret_cast<f16x8*>(do16 + row0 * HD + 8 * c) = h0;
    if (row0 + 1 < nrows) *reinterpret_cast<f16x8*>(do16 + row1 * HD + 8 * c) = h1;
    float acc0 = 0.f, acc1 = 0.f;
    if (o) {
      const u32x4 a0 = *reinterpret_cast<const u32x4*>(o + row0 * HD + 8 * c);
      const u32x4 a1 = *reinterpret_cast<const u32x4*>(o + row1 * HD + 8 * c);
      const uint2 b0 = *reinterpret_cast<const uint2*>(o_lo + row0 * HD + 8 * c);
      const uint2 b1 = *reinterpret_cast<const uint2*>(o_lo + row1 * HD + 8 * c);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t ob0 = (a0[t >> 1] >> (16 * (t & 1))) & 0xffffu;
        const uint32_t ob1 = (a1[t >> 1] >> (16 * (t & 1))) & 0xffffu;
        const uint32_t q0 = ((t < 4 ? b0.x : b0.y) >> (8 * (t & 3))) & 0xffu;
        const uint32_t q1 = ((t < 4 ? b1.x : b1.y) >> (8 * (t & 3))) & 0xffu;
        acc0 = fmaf(lo8_decode(ob0, q0), (float)d0[t], acc0);
        acc1 = fmaf(lo8_decode(ob1, q1), (float)d1[t], acc1);
      }
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) {
        acc0 += __shfl_xor(acc0, m);
        acc1 += __shfl_xor(acc1, m);
      }
    }
    if (c == 0) {
      auto put = [&](long row, float v) {
        const int hh = (int)(row % H);
        const long bs = row / H;
        const int sp = (int)(bs % S);
        const int bb = (int)(bs / S);
        const long i = ((long)bb * H + hh) * S + sp;
        ndelta[i] = -(o ? v : delta_in[i]);
        lse[i] = lse2[i] - log2_sm_scale;
      };
      put(row0, acc0);
      if (row0 + 1 < nrows) put(row0 + 1, acc1);
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  __shared__ float wmax[4];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) part_max[blockIdx.x] = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}

// The power of two 2^E that dO is scaled by before its fp16 rounding, from
// mdo = max|dO| and mv = max|V|.  dS = P (dP - Delta) sm_scale, with
// |dP_ij| <= D mdo mv and |Delta_i| <= max_j |dP_ij|, is bounded by
// bound = 2 D sm_scale mdo mv; the fp16 values must stay below 2^15.
//   * E = 0 when 2^-8 <= mdo <= 2^8 and bound < 2^15: dO's largest values
//     keep 11 significant bits, and values below fp16's normal range (2^-14,
//     at most 2^-6 of the largest) lose at most 2^-25 absolutely;
//   * otherwise E = -ilogb(mdo) (2^E mdo in [1, 2)), lowered until 2^E
//     bound < 2^15.  E reaches 133 for the smallest bf16 (subnormal) dO;
//     2^E is applied as two factors of at most 2^67 each (exact).
// mdo == 0 (or a non-finite maximum, which the results then carry): E = 0.
__device__ __forceinline__ int do_scale_exp(float mdo, float mv, float sm_scale) {
  if (!(mdo > 0.f) || !isfinite(mdo) || !isfinite(mv)) return 0;
  const float bound = 2.f * HD * sm_scale * mdo * mv;
  const bool bound_ok = !(bound >= 32768.f);
  if (mdo >= 0x1p-8f && mdo <= 0x1p8f && bound_ok) return 0;
  int e = -ilogbf(mdo);
  if (bound > 0.f && isfinite(bound)) e = min(e, 14 - ilogbf(bound));
  return max(-126, min(134, e));
}

// x * 2^e for |e| <= 134, as two exact power-of-two multiplies.
__device__ __forceinline__ float scale_pow2(float x, int e) {
  return x * ldexpf(1.f, e / 2) * ldexpf(1.f, e - e / 2);
}

// E from the partial maxima; scale[0] = 2^-E, scale[1] = 2^E (the kernels
// that consume the scaled values multiply their dQ / dK / dV by scale[0]:
// exact, a power of two).  With E != 0 it reconverts dO -> fp16(2^E dO) and
// scales -Delta by 2^E in place; with E == 0 (attn_delta16_kernel's
// conversion stands) every workgroup leaves after reading the maxima.  Each
// workgroup reduces the n_dmax + n_vmax partial maxima itself (a few KiB,
// L2-resident), so no other launch sits between the maxima and the
// conversion.
__global__ __launch_bounds__(256) void attn_do16_kernel(
    const __bf16* __restrict__ dO, _Float16* __restrict__ do16, float* __restrict__ delta,
    const float* __restrict__ dmax, int n_dmax, const float* __restrict__ vmax, int n_vmax,
    float* __restrict__ scale, float sm_scale, long n_do, long n_delta) {
  float md = 0.f, mv = 0.f;
  for (int i = threadIdx.x; i < n_dmax; i += 256) md = fmaxf(md, dmax[i]);
  for (int i = threadIdx.x; i < n_vmax; i += 256) mv = fmaxf(mv, vmax[i]);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    md = fmaxf(md, __shfl_xor(md, m));
    mv = fmaxf(mv, __shfl_xor(mv, m));
  }
  __shared__ float wm[2][4];
  if ((threadIdx.x & 63) == 0) {
    wm[0][threadIdx.x >> 6] = md;
    wm[1][threadIdx.x >> 6] = mv;
  }
  __syncthreads();
  md = fmaxf(fmaxf(wm[0][0], wm[0][1]), fmaxf(wm[0][2], wm[0][3]));
  mv = fmaxf(fmaxf(wm[1][0], wm[1][1]), fmaxf(wm[1][2], wm[1][3]));
  const int e = do_scale_exp(md, mv, sm_scale);
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    scale[0] = ldexpf(1.f, -e);                 // 2^-134 .. 2^126: subnormal at the far end
    scale[1] = e < 128 ? ldexpf(1.f, e) : INFINITY;
  }
  if (e == 0) return;
  const long stride = (long)gridDim.x * 256;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n_do / 8; i += stride) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(dO + 8 * i);
    f16x8 r;
#pragma unroll
    for (int t = 0; t < 8; ++t) r[t] = (_Float16)scale_pow2((float)x[t], e);
    *reinterpret_cast<f16x8*>(do16 + 8 * i) = r;
  }
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n_delta; i += stride) delta[i] = scale_pow2(delta[i], e);
}

// ---------------------------------------------------------------------------
// Work item of a per-head dK/dV workgroup: key tile kt = item / (B*H) of query head
// bh = item % (B*H), or -1 for a launch slot without one.  Slot b runs on XCD
// b % 8.  The slots are dealt so that each XCD owns whole query heads, and
// the workgroups it runs at one time share the Q/dO tiles they stream.  Each
// head's key tiles are split by kt mod q into q parts, q = 8 / gcd(B*H, 8),
// so that the 8 XCDs get m = B*H*q/8 parts each.  XCD x runs its parts
// x*m .. x*m+m-1 interleaved, key tiles ascending (longest first).  When 8
// divides B*H (q = 1) every XCD holds whole heads.  (The plain b -> (b /
// (B*H), b % (B*H)) order spreads each head over several XCDs unless 8
// divides B*H; at B*H = 20 that fetched 2.3x the bytes from beyond L2.)
struct KeyTileOrder {
  int q, m;   // parts per head, parts per XCD
};

inline KeyTileOrder key_tile_order(int nbh) {
  int g = 8;
  while (nbh % g) g >>= 1;   // gcd(nbh, 8)
  const int q = 8 / g;
  return {q, nbh * q / 8};
}

__device__ __forceinline__ int key_tile_item(int slot, int nbh, int n_kt, KeyTileOrder o) {
  const int x = slot & 7, r = slot >> 3;
  const int part = x * o.m + r % o.m;
  const int kt = o.q * (r / o.m) + part % o.q;
  return kt < n_kt ? kt * nbh + part / o.q : -1;
}

template <int V>
using ic = std::integral_constant<int, V>;
template <class T>
struct is_ic : std::false_type {};
template <int V>
struct is_ic<std::integral_constant<int, V>> : std::true_type {};

// Calls f(integral_constant<J>) for J = 0 .. N-1 while it returns true.
template <int J, int N, class F>
__device__ __forceinline__ void unroll_while(F&& f) {
  if constexpr (J < N) {
    if (f(std::integral_constant<int, J>{})) unroll_while<J + 1, N>(f);
  }
}

// ---------------------------------------------------------------------------
// dK, dV, software-pipelined across the two roles of a pair.
//
// One workgroup per 128-key tile, 8 waves in 4 pairs, one pair per SIMD; a
// pair owns 32 keys of the tile and splits the work by role: the P wave
// keeps K (B operand) and the dV^T accumulators, the dS wave V and dK^T.  P
// goes from the P wave to the dS wave through a two-slot LDS mailbox, as the
// fp16 values the P wave's dV^T product takes (half the LDS bytes of fp32,
// which the kernel's LDS traffic is the tightest limit on).
// The query tiles are 32 rows (Q, dO row-major; the transposed operands of
// dV^T and dK^T come from the LDS transpose read), and the work on a tile is
// spread over four segments:
//   segment s, P wave : S(s+1) = Q(s+1) K^T                 | P'(s) = exp2(S(s) scale2 - lse) = P sm_scale -> mailbox | dV^T += dO(s-1)^T P'(s-1)
//   segment s, dS wave: dP(s) - Delta = -Delta + dO(s) V^T   | dS(s-1) = fp16(P'(s-1)) (dP(s-1) - Delta)               | dK^T += Q(s-2)^T dS(s-2)
// Within a segment each wave's VALU work (middle column) depends on no
// product of the same segment, so it runs under the wave's own products
// (and, with two waves per SIMD, the other wave's), and the pair meets at one
// barrier per segment, which also publishes the DMA ring.  S(s+1), P(s-1)
// (fp16) stay in the P wave's registers, dP(s-1) and dS(s-2) (fp16) in the
// dS wave's.  Each wave starts its segment with the accumulation product
// (the P wave runs dV^T before S(s+1)), whose tile was published segments
// earlier: its first operand fragments and the wave's lse / -Delta vector
// are read before the previous barrier, so right after a barrier the waves
// issue products instead of all waiting on the LDS together.
//
// Operands: the fp16 copies q16, k16, v16 of the forward state and do16 =
// fp16(2^E dO) with -Delta scaled alike (attn_do16_kernel), so dP, dS and
// the accumulators carry the factor 2^E; the epilogue multiplies dK by
// scale[0] = 2^-E.  The P wave's exponentials take lse = lse2 -
// log2(sm_scale) and give P' = P sm_scale, which is rounded to fp16 for
// dV^T and for the mailbox (dS = fp16(P') (dP - Delta) in fp32, rounded to
// fp16 for dK^T): the epilogue multiplies dV by 2^-E / sm_scale.  F32OUT: dk / dv (and the partials)
// are fp32, the values the bf16 path rounds.
//
// Tile x of the ring lives in slot x % NSTAGE; it is first read in segment
// x-1 and last in segment x+2, so segment s refills slot (s-3) % NSTAGE with
// tile s + NSTAGE - 3 and waits for tile s+2 before its barrier (NSTAGE - 5
// segments of lead).  Tiles whose queries all precede a pair's keys (causal)
// are computed with the mask (P = 0): the pair would otherwise only wait at
// the barrier.
template <int NSTAGE, bool CAUSAL, bool GROUP, bool RAGGED, bool F32OUT>
__global__ __launch_bounds__(512, 1) void attn_dkdv_pipe_kernel(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    const _Float16* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ ndelta,
    const float* __restrict__ scale, float* __restrict__ ws_dk, float* __restrict__ ws_dv,
    void* __restrict__ dk, void* __restrict__ dv,
    int B, int S, int H, int Hkv, int G, float scale2, float sm_scale, KeyTileOrder order,
    int chunk_tiles, int max_chunks, const DispatchOrder ord, int ws_rows) {
  static_assert(NSTAGE >= 6, "ring depth: at least 6");
  constexpr int KB = 1;                   // 32-key blocks per wave
  constexpr int NW = 8;                   // waves per workgroup
  constexpr int NP = NW / 2;              // pairs
  // Waves that copy the ring's tiles: the P waves (the dS waves, which carry
  // the longer chain of the segment, issue no copies and wait for none).
  constexpr int DW = NP;
  constexpr int QPW = 8 / DW;             // row quads of a 32-row tile each copying wave copies
  constexpr int BQ = 32;                  // query positions per tile
  constexpr int QT = BQ * HD * 2;         // one 32 x 128 fp16 operand tile
  // LDS: three rings of NSTAGE slots -- Q tiles, dO tiles, [lse x 32 |
  // -Delta x 32] vectors -- then the mailboxes.  Every read of a Q tile lies
  // below 64 KiB (it takes the per-lane bases of make_lds_bases plus a
  // constant in the offset field); dO tiles and vectors are read through
  // per-lane bases that hold their ring's offset (below).
  constexpr int QR = 0;                   // Q ring
  constexpr int DR = NSTAGE * QT;         // dO ring
  constexpr int VR = 2 * NSTAGE * QT;     // vector ring
  constexpr int VSLOT = 256;
  constexpr int MB0 = VR + NSTAGE * VSLOT;
  constexpr int MBOX = 32 * 32 * 2;       // one 32 x 32 fp16 P block
  static_assert(QR + NSTAGE * QT + 4096 <= 0x10000, "Q reads must reach every Q slot by the offset field");
  __shared__ __attribute__((aligned(1024))) char smem[MB0 + NP * 2 * KB * MBOX];

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index (uniform)
  const int pair = w % NP;
  const bool pwave = w < NP;
  const int n_kt = (S + 127) / 128;
  // The work of this workgroup: key tile kt of (b, g) and the n_u query
  // tiles u0, u0 + ustep, u0 + 2*ustep, ... of the position-major walk over
  // HW heads (tile u: position tile u / HW counted from the sequence end,
  // head hbase + u % HW of the group).  The chunks of a split key tile
  // interleave, so every workgroup starts at the sequence end and those that
  // run together stream the same rows.  The sums go to partial slot `part`
  // of `nparts`, or straight to dk/dv when nparts == 1.  A workspace slot
  // holds ws_rows key rows per batch element: S for the per-head tilings,
  // split_keys (the keys of split key tiles, the only ones with partials)
  // for the grouped ones.
  int b, g, kt, n_qt, u0, n_u, ustep, part, nparts, hbase, HW;
  if constexpr (GROUP) {
    const int j = dispatch_item(ord);
    if (j < 0) return;
    const int nbg = B * Hkv;
    const int bg = j % nbg, r = j / nbg;
    kt = r / max_chunks;                  // heaviest key tiles first
    const int c = r - kt * max_chunks;
    if (kt >= n_kt) return;
    b = bg / Hkv;
    g = bg - b * Hkv;
    n_qt = dkdv_n_qt(S, kt, CAUSAL);
    const int len = G * n_qt;
    nparts = dkdv_chunks(len, chunk_tiles, max_chunks);
    if (c >= nparts) return;              // an empty item of the default numbering
    u0 = c;
    ustep = nparts;   // <= max_chunks <= G: one wrap of the head index at most
    n_u = (len - c + nparts - 1) / nparts;
    part = c;
    hbase = 0;
    HW = G;
  } else {
    const int nbh = B * H;
    const int item = key_tile_item(blockIdx.x, nbh, n_kt, order);
    if (item < 0) return;
    kt = item / nbh;                      // heaviest key tiles first
    const int bh = item % nbh;
    b = bh / H;
    const int hq = bh % H;
    g = hq / G;
    const int hh = hq % G;
    n_qt = dkdv_n_qt(S, kt, CAUSAL);
    u0 = 0;
    ustep = 1;
    n_u = n_qt;
    part = hh;
    nparts = G;
    hbase = hh;
    HW = 1;
  }
  const int kw0 = kt * 128 + 32 * KB * pair;   // this pair's first key
  // mailbox of this pair: two slots of KB blocks; a block is
  // [register half j][lane] x 8 fp16 (registers 8j .. 8j+7 of the lane's P'
  // block), so each 16-byte access of a wave is one contiguous 1 KiB row
  _Float16* const mbox = reinterpret_cast<_Float16*>(smem + MB0 + pair * 2 * KB * MBOX) + lane * 8;

  const int q_begin = CAUSAL ? kt * 128 : 0;
  const long qstride = (long)H * HD;
  // walk head hh: Q / dO rows at grp_rows + hh*HD, lse / -Delta at
  // vec_src + hh*S (lanes 0-31 lse, lanes 32-63 -Delta)
  const long grp_rows = ((long)b * S * H + g * G + hbase) * HD;
  const float* vec_src = (h ? ndelta : lse) + ((long)b * H + g * G + hbase) * S + l32;

  // Position tiles are walked from the sequence end down to q_begin, so the
  // workgroups that start together read the same rows together; the first
  // position tile can be partial (S % 32 != 0).  Tile cursors (walk head,
  // position tile) advance one tile at a time.
  auto tile_p0 = [&](int t) MM1_INLINE { return q_begin + (n_qt - 1 - t) * BQ; };
  auto advance = [&](int& hh, int& t) MM1_INLINE {
    hh += ustep;
    if (hh >= HW) {
      hh -= HW;
      ++t;
    }
  };
  // LDS DMA, per copying wave and tile: row quads w, w + DW, ... of Q and of dO;
  // wave 0 adds the lse | -Delta vector.  (quad & 3) == (w & 3) for every quad
  // of the wave, so one per-lane offset serves all of them.
  const uint32_t dma_off = tile_lane_off(qstride, tid);
  const uint32_t lds_smem = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  // Only position tile 0 can be partial, and only when S % 32 != 0
  // (RAGGED); the walks without partial tiles carry no code for them.
  auto issue = [&](int slot, int hh, int t, auto may_be_partial) MM1_INLINE {
    if (w >= DW) return;
    const int p0 = tile_p0(t);
    const long rows = grp_rows + (long)hh * HD + (long)p0 * qstride;
    const float* vs = vec_src + (long)hh * S;
    const uint32_t lq = lds_smem + QR + slot * QT, ld = lds_smem + DR + slot * QT;
    const uint32_t lv = lds_smem + VR + slot * VSLOT;
    if (!decltype(may_be_partial)::value || p0 + BQ <= S) {
#pragma unroll
      for (int i = 0; i < QPW; ++i) {
        const int quad = w + DW * i;
        dma16_sbase(dma_off, q + rows + (long)(4 * quad) * qstride, lq + quad * 1024);
        dma16_sbase(dma_off, dO + rows + (long)(4 * quad) * qstride, ld + quad * 1024);
      }
      if (w == 0) dma4(vs + p0, lv);
    } else {   // same DMA count per wave as a full tile
      const int L = tid & 63;
#pragma unroll
      for (int i = 0; i < QPW; ++i) {
        const int quad = w + DW * i;
        const int row = 4 * quad + (L >> 4);
        const int chunk = (L & 15) ^ swz(row);
        const long src = rows + (long)min(row, S - p0 - 1) * qstride + 8 * chunk;
        dma16(q + src, lq + quad * 1024);
        dma16(dO + src, ld + quad * 1024);
      }
      if (w == 0) dma4(vs + min(p0, S - 1 - l32), lv);
    }
  };
  int itl = u0 / HW, ih = u0 - itl * HW;      // issue cursor
  int ch = ih, ctl = itl;                     // compute cursor (tile s of the walk)
  for (int it = 0; it < NSTAGE - 3 && it < n_u; ++it) {
    issue(it, ih, itl, std::bool_constant<RAGGED>{});
    advance(ih, itl);
  }

  // This lane's key rows of K (P wave) or V (dS wave) as the B operands,
  // one per key block.  The dP product accumulates onto -Delta and gives
  // dP - Delta, and the mailbox carries P sm_scale, so dS = P (dP - Delta)
  // sm_scale is one multiply.
  f16x8 breg[KB][8];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int kk = min(kw0 + 32 * kb + l32, S - 1);
    const _Float16* src = (pwave ? k : v) + ((long)(b * S + kk) * Hkv + g) * HD + 8 * h;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) breg[kb][ks] = *reinterpret_cast<const f16x8*>(src + 16 * ks);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) pin(breg[kb][ks]);
  }

  f32x16 acc[KB][4];   // dV^T (P wave) or dK^T (dS wave), per key block
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[kb][db] = zero16();
  }
  auto accumulate = [&](f32x16& c, const f16x8& a, const f16x8& bb) MM1_INLINE { c = mfma32h(a, bb, c); };
  // The P wave computes S one segment ahead (snext), so that its
  // exponentials run between the products of the next S.  The dS wave
  // computes dS(s-1) between the products of dK^T += Q^T dS(s-2) and dP(s)
  // last, for the next segment.
  f16x8 pb[KB][2];     // P wave: P(s-1) as the B operand of dV^T
  f32x16 snext[KB];    // P wave: S(s), computed one segment ahead
  f32x16 dpp[KB];      // dS wave: dP(s-1)
  f16x8 sbp[KB][2];    // dS wave: dS(s-2) as the B operand of dK^T
  const LdsBases lb = make_lds_bases(lane);
  // Reads.  The ring slots of the walk's segments are compile-time constants
  // (the walk is unrolled by the ring depth), so each read is a per-lane
  // base plus a constant in the ds instruction's 16-bit offset field.  The
  // dO and vector rings lie past 64 KiB: their reads take per-lane bases
  // that hold the ring's offset, opaque to the compiler (it would otherwise
  // fold the offset into the constant and add it back with a VALU
  // instruction per read).  Each role sets the bases it reads with: the P
  // wave dO^T (transposed) and the lse vector, the dS wave dO rows and the
  // -Delta vector.  The last two segments, whose slots depend on the walk's
  // length, take a run-time slot and plain addresses.
  using lds_cp = const MM1_LDS char*;
  lds_cp dbase[8], vbase;
  auto set_bases = [&](bool pw) MM1_INLINE {
    const lds_cp d = (lds_cp)smem + DR;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dbase[i] = d + (pw ? lb.tr[i >> 1][i & 1] : (lb.row ^ (32 * i)));
      __asm__ volatile("" : "+v"(dbase[i]));
    }
    vbase = (lds_cp)smem + VR + 16 * h;
    __asm__ volatile("" : "+v"(vbase));
  };
  // fragments of the tile in ring slot `sl` (an integral_constant): rows of Q
  // / dO (the A operands of S / dP), transposed fragments (blk, ks) of Q / dO
  // (the A operands of dK^T / dV^T), 4 of a lane's 16 per-row vector values
  // (byte offset `vec`: 0 lse, 4*BQ -Delta; rows 8*a4 + 4*h .. +3)
  auto slot_of = [](auto sl) MM1_INLINE { return (int)sl; };
  auto q_rows = [&](auto sl, int ks) MM1_INLINE { return rows_a(smem + QR + slot_of(sl) * QT, lb, 0, ks); };
  auto q_tr = [&](auto sl, int blk, int ks) MM1_INLINE {
    return tr_a(smem + QR + slot_of(sl) * QT, lb, blk, ks);
  };
  auto do_rows = [&](auto sl, int ks) MM1_INLINE {
    if constexpr (is_ic<decltype(sl)>::value)
      return *reinterpret_cast<const MM1_LDS f16x8*>(dbase[ks] + decltype(sl)::value * QT);
    else
      return rows_a(smem + DR + sl * QT, lb, 0, ks);
  };
  auto do_tr = [&](auto sl, int blk, int ks) MM1_INLINE {
    if constexpr (is_ic<decltype(sl)>::value) {
      f16x8 out;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const f16x4 v4 = __builtin_bit_cast(
            f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                       (MM1_LDS fp16x4_tr*)(dbase[2 * blk + r] + (decltype(sl)::value * QT + 4096 * ks))));
#pragma unroll
        for (int e = 0; e < 4; ++e) out[4 * r + e] = v4[e];
      }
      return out;
    } else {
      return tr_a(smem + DR + sl * QT, lb, blk, ks);
    }
  };
  auto vec4 = [&](auto sl, int vec, int a4) MM1_INLINE {
    if constexpr (is_ic<decltype(sl)>::value)
      return *reinterpret_cast<const MM1_LDS f32x4*>(vbase + (decltype(sl)::value * VSLOT + vec + 32 * a4));
    else
      return *reinterpret_cast<const f32x4*>(smem + VR + sl * VSLOT + vec + 32 * a4 + 16 * h);
  };
  wait_dma();
  __syncthreads();
  // S = Q K^T / dP = dO V^T of one tile, per key block (D layout: register r
  // holds query 8*(r/4) + 4*h + (r%4) of the tile, lane l32 holds key
  // kw0 + 32*kb + l32); each row fragment (rows(ks)) is read once for all
  // key blocks (accumulated onto c0)
  auto product_onto = [&](auto&& rows, f32x16 (&sacc)[KB], const f32x16& c0,
                          auto&& between) MM1_INLINE {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) sacc[kb] = c0;
    mfma_chain<8, MM1_DKDV_PF_ROWS>(
        [&](int ks) MM1_INLINE { return rows(ks); },
        [&](int ks, const f16x8& fa) MM1_INLINE {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) sacc[kb] = mfma32h(fa, breg[kb][ks], sacc[kb]);
        },
        between);
  };
  auto product = [&](auto&& rows, f32x16 (&sacc)[KB], auto&& between) MM1_INLINE {
    product_onto(rows, sacc, zero16(), between);
  };
  // dV^T += dO^T P (P wave) / dK^T += Q^T dS (dS wave) of one tile: product
  // i = 4*kh + db takes the transposed fragment tr(i) = (db, kh) of the tile
  // and the B operand bop[kb][kh]; its first PFT fragments were read before
  // the segment's barrier (first)
  constexpr int PFT = MM1_DKDV_PF_TR;
  auto accumulate_tile = [&](const f16x8 (&first)[PFT], auto&& tr, const f16x8 (&bop)[KB][2],
                             auto&& between) MM1_INLINE {
    mfma_chain_from<8, PFT>(
        first, [&](int i) MM1_INLINE { return tr(i); },
        [&](int i, const f16x8& a) MM1_INLINE {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) accumulate(acc[kb][i & 3], a, bop[kb][i >> 2]);
        },
        between);
  };
  // What a wave's next segment starts with, read at the end of this one
  // from tiles published by earlier barriers, so that after the barrier the
  // first product waits for no LDS read: the first PFT transposed fragments
  // of the accumulation product (P wave: dO(s) for dV^T; dS wave: Q(s-1) for
  // dK^T) and, for the P wave, the lse vector of tile s+1 (its
  // exponentials).  The dS wave reads Delta of tile s just before its dP
  // product, which starts from it (holding it across the barrier cost more
  // registers than the read).
  f16x8 nfa[PFT];
  f32x4 nvec[4];
  auto read_first = [&](auto&& tr) MM1_INLINE {
#pragma unroll
    for (int i = 0; i < PFT; ++i) nfa[i] = tr(i);
  };
  auto read_lse = [&](auto sl) MM1_INLINE {
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) nvec[a4] = vec4(sl, 0, a4);
  };
  auto nothing = [](int) MM1_INLINE {};

  // Segment s, its tile in ring slot cs = s % NSTAGE, an integral_constant
  // or (the last two segments) an int; tn, tc, tp, tp2: the slots of tiles
  // s+1, s, s-1, s-2.  CUR: s < n_u; PREV: tile s-1 exists; PREV2: tile s-2
  // exists; SYNC: a later segment reads what this one publishes (mailbox,
  // ring).  In the last segment with CUR, S(s+1) reads a slot holding
  // another tile (or nothing yet) and is discarded, as is the lse read for
  // segment s+1: every read stays inside the ring.
  auto shift = [](auto sl, auto d) MM1_INLINE {
    if constexpr (is_ic<decltype(sl)>::value)
      return ic<(decltype(sl)::value + decltype(d)::value) % NSTAGE>{};
    else
      return (sl + decltype(d)::value) % NSTAGE;
  };
  auto segment = [&](auto cslot, int s, auto role, auto cur, auto prev, auto prev2, auto sync) MM1_INLINE {
    const auto tn = shift(cslot, ic<1>{});
    const auto tc = cslot;
    const auto tp = shift(cslot, ic<NSTAGE - 1>{});
    const auto tp2 = shift(cslot, ic<NSTAGE - 2>{});
    const int refill = slot_of(shift(cslot, ic<NSTAGE - 3>{}));
    constexpr bool PW = decltype(role)::value;
    constexpr bool CUR = decltype(cur)::value, PREV = decltype(prev)::value;
    constexpr bool PREV2 = decltype(prev2)::value, SYNC = decltype(sync)::value;
    if (CUR && s + NSTAGE - 3 < n_u) {
      // a per-head walk meets position tile 0 only in the prologue
      issue(refill, ih, itl, std::bool_constant<RAGGED && GROUP>{});
      advance(ih, itl);
    }
    if constexpr (PW) {
      f32x16 sv[KB];
      f32x4 lse4[4];
      if constexpr (CUR) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) lse4[a4] = nvec[a4];
      }
      // P' = exp2(S*scale2 - lse) = P sm_scale of register r of every key block
      auto exp_at = [&](int r) MM1_INLINE {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          float x = exp2_fast(fmaf(sv[kb][r], scale2, -lse4[r >> 2][r & 3]));
          pin(x);   // computed here, not sunk towards its first use
          sv[kb][r] = x;
        }
      };
      // causal / past-the-end mask, only in the tiles that need it
      auto mask = [&]() MM1_INLINE {
        const int p0 = tile_p0(ctl);
        if ((CAUSAL && p0 < kw0 + 32 * KB - 1) || p0 + BQ > S) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
            const int key = kw0 + 32 * kb + l32;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int qpos = p0 + 8 * (r >> 2) + 4 * h + (r & 3);
              sv[kb][r] = ((CAUSAL && key > qpos) || qpos >= S) ? 0.f : sv[kb][r];
            }
          }
        }
      };
      // fp16 P(s), the B operand of the next segment's dV^T product: registers
      // 2j, 2j+1 of each key block
      f16x8 pbn[KB][2];
      auto pack_at = [&](int j) MM1_INLINE {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
          for (int e = 0; e < 2; ++e) pbn[kb][j >> 2][2 * (j & 3) + e] = (_Float16)sv[kb][2 * j + e];
          if ((j & 3) == 3) pin(pbn[kb][j >> 2]);
        }
      };
      // dV^T += dO(s-1)^T P(s-1) first (its operands were read before the
      // barrier), with the exponentials of S(s) between its products; then
      // S(s+1) from the tile the barrier published, with the fp16 pack of
      // P(s) between its products
      if constexpr (CUR) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) sv[kb] = snext[kb];
      }
      if constexpr (PREV) {
        accumulate_tile(nfa, [&](int i) MM1_INLINE { return do_tr(tp, i & 3, i >> 2); }, pb, [&](int i) MM1_INLINE {
          if constexpr (CUR) {
            exp_at(2 * i);
            exp_at(2 * i + 1);
          }
        });
      } else if constexpr (CUR) {
#pragma unroll
        for (int r = 0; r < 16; ++r) exp_at(r);
      }
      if constexpr (CUR) {
        mask();
        // the fp16 P'(s) of the dV^T product goes to the mailbox as well, each
        // half as soon as it is packed (spreading the writes over the product)
        _Float16* mb = mbox + (s & 1) * (KB * MBOX / 2);
        product([&](int ks) MM1_INLINE { return q_rows(tn, ks); }, snext, [&](int ks) MM1_INLINE {
          pack_at(ks);
          if ((ks & 3) == 3) {
#pragma unroll
            for (int kb = 0; kb < KB; ++kb)
              *reinterpret_cast<f16x8*>(mb + kb * (MBOX / 2) + 512 * (ks >> 2)) = pbn[kb][ks >> 2];
          }
        });
      }
      if constexpr (CUR) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          pb[kb][0] = pbn[kb][0];
          pb[kb][1] = pbn[kb][1];
        }
        read_first([&](int i) MM1_INLINE { return do_tr(tc, i & 3, i >> 2); });
        read_lse(tn);
      }
    } else {
      // dS(s-1) = P'(s-1) (dP(s-1) - Delta) from the mailbox's fp16
      // P' = P sm_scale, between the products of dK^T += Q(s-2)^T dS(s-2)
      f32x16 dsv[KB];
      f16x8 pm[KB][2];   // P'(s-1) in fp16, as the P wave's dV^T product takes it
      if constexpr (PREV) {
        const _Float16* mb = mbox + ((s - 1) & 1) * (KB * MBOX / 2);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
          for (int j = 0; j < 2; ++j) pm[kb][j] = *reinterpret_cast<const f16x8*>(mb + kb * (MBOX / 2) + 512 * j);
        }
      }
      auto ds_at = [&](int r) MM1_INLINE {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          // one v_fma_mix_f32: the fp16 operand is widened inside the fma
          float x = fmaf((float)pm[kb][r >> 3][r & 7], dpp[kb][r], 0.f);
          pin(x);
          dsv[kb][r] = x;
        }
      };
      f16x8 sbn[KB][2];
      auto dspack_at = [&](int j) MM1_INLINE {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
          for (int e = 0; e < 2; ++e) sbn[kb][j >> 2][2 * (j & 3) + e] = (_Float16)dsv[kb][2 * j + e];
          if ((j & 3) == 3) pin(sbn[kb][j >> 2]);
        }
      };
      if constexpr (PREV2) {
        accumulate_tile(nfa, [&](int i) MM1_INLINE { return q_tr(tp2, i & 3, i >> 2); }, sbp, [&](int i) MM1_INLINE {
          if constexpr (PREV) {
            ds_at(2 * i);
            ds_at(2 * i + 1);
            dspack_at(i);
          }
        });
      } else if constexpr (PREV) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          ds_at(2 * j);
          ds_at(2 * j + 1);
          dspack_at(j);
        }
      }
      if constexpr (PREV) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          sbp[kb][0] = sbn[kb][0];
          sbp[kb][1] = sbn[kb][1];
        }
      }
      // dP(s) - Delta = -Delta + dO(s) V^T, used by the next segment
      if constexpr (CUR) {
        f32x16 dlt;   // -Delta of tile s in the D layout (register r: query 8*(r/4) + 4*h + r%4)
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          const f32x4 d4 = vec4(tc, 4 * BQ, a4);
#pragma unroll
          for (int c = 0; c < 4; ++c) dlt[4 * a4 + c] = d4[c];
        }
        product_onto([&](int ks) MM1_INLINE { return do_rows(tc, ks); }, dpp, dlt, nothing);
      }
      if constexpr (PREV) read_first([&](int i) MM1_INLINE { return q_tr(tp, i & 3, i >> 2); });
    }
    if constexpr (CUR) advance(ch, ctl);
    if constexpr (SYNC) {
      // tile s+2 must have landed; the newer prefetches stay in flight
      // (2 * QPW copies per tile and copying wave, wave 0 one more).  A wave
      // that copies nothing waits for nothing.
      if (w < DW) {
        if (s + NSTAGE - 3 < n_u) {
          if (w == 0) __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"((2 * QPW + 1) * (NSTAGE - 5)) : "memory");
          else __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * QPW * (NSTAGE - 5)) : "memory");
        } else {
          wait_dma();
        }
      }
      lds_barrier();
    }
  };

  // Each role runs its own specialised copy of the loop (same barriers).
  // Segments 2 .. n_u-1 are unrolled NSTAGE at a time so that every ring
  // slot, and so every LDS offset, is a compile-time constant.
  using T = std::true_type;
  using F = std::false_type;
  auto run = [&](auto role) MM1_INLINE {
    set_bases(decltype(role)::value);
    if constexpr (decltype(role)::value) {
      product([&](int ks) MM1_INLINE { return q_rows(ic<0>{}, ks); }, snext, nothing);
      read_lse(ic<0>{});        // lse of tile 0
    }
    if (n_u == 1) {
      segment(ic<0>{}, 0, role, T{}, F{}, F{}, T{});
      segment(ic<1>{}, 1, role, F{}, T{}, F{}, F{});
      segment(ic<2>{}, 2, role, F{}, F{}, T{}, F{});
      return;
    }
    segment(ic<0>{}, 0, role, T{}, F{}, F{}, T{});
    segment(ic<1>{}, 1, role, T{}, T{}, F{}, T{});
    for (int b0 = 2; b0 < n_u; b0 += NSTAGE) {
      unroll_while<0, NSTAGE>([&](auto j) MM1_INLINE {
        const int s = b0 + decltype(j)::value;
        if (s >= n_u) return false;
        segment(ic<(2 + decltype(j)::value) % NSTAGE>{}, s, role, T{}, T{}, T{}, T{});
        return true;
      });
    }
    segment(n_u % NSTAGE, n_u, role, F{}, T{}, T{}, F{});
    segment((n_u + 1) % NSTAGE, n_u + 1, role, F{}, F{}, T{}, F{});
  };
  if (pwave) run(std::true_type{});
  else run(std::false_type{});

  // D layout of dK^T / dV^T: register r of block db holds column
  // d = 32*db + 8*(r/4) + 4*h + (r%4) of this lane's key row.  The sums
  // carry the factor 2^E of do16 (dV also sm_scale, from P'): times 2^-E
  // (and 1 / sm_scale) they are dK, dV.
  const float unscale = pwave ? scale[0] / sm_scale : scale[0];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = kw0 + 32 * kb + l32;
    if (key >= S) continue;
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[kb][db] *= unscale;
    if (nparts == 1) {
      const long row = ((long)(b * S + key) * Hkv + g) * HD;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          if constexpr (F32OUT) {
            f32x4 o4;
#pragma unroll
            for (int c = 0; c < 4; ++c) o4[c] = acc[kb][db][4 * a4 + c];
            *reinterpret_cast<f32x4*>(static_cast<float*>(pwave ? dv : dk) + row + 32 * db + 8 * a4 + 4 * h) = o4;
          } else {
            bf16x4 o4;
#pragma unroll
            for (int c = 0; c < 4; ++c) o4[c] = (__bf16)acc[kb][db][4 * a4 + c];
            *reinterpret_cast<bf16x4*>(static_cast<__bf16*>(pwave ? dv : dk) + row + 32 * db + 8 * a4 + 4 * h) = o4;
          }
        }
      }
    } else {
      const long slot = (long)part * B * ws_rows * Hkv * HD;
      float* row = (pwave ? ws_dv : ws_dk) + slot + ((long)(b * ws_rows + key) * Hkv + g) * HD;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          f32x4 o4;
#pragma unroll
          for (int c = 0; c < 4; ++c) o4[c] = acc[kb][db][4 * a4 + c];
          *reinterpret_cast<f32x4*>(row + 32 * db + 8 * a4 + 4 * h) = o4;
        }
      }
    }
  }
}

// The dK/dV partial sums to reduce, and where the reduction runs.  Two
// layouts, fp32, dK's slots then dV's:
//   per-head dK/dV (chunk_tiles == 0): [G][B][S][Hkv][D], slot = query head
//     of the group; every element sums its G slots;
//   grouped dK/dV (chunk_tiles > 0): [C][B][split_keys][Hkv][D], slot = chunk
//     of the key tile; only keys [0, split_keys) of each batch are split,
//     and a key of tile kt sums its
//     dkdv_chunks(G * dkdv_n_qt(S, kt), chunk_tiles, max_chunks) slots (the
//     other keys were written as bf16 by the dK/dV kernel itself).
// The dQ kernel folds the reduction in: the last n_red workgroups of its grid
// each reduce one contiguous slice after their own work (with n_red = the
// grid size, a small slice per workgroup, spread over the whole launch).
struct TailReduce {
  const float* ws_dk;
  const float* ws_dv;
  __bf16* dk;
  __bf16* dv;
  float* dk32;      // non-null: write the sums in fp32 here instead (fp32 backward)
  float* dv32;
  long n;           // elements of one slot: B*S*Hkv*D (per-head), B*split_keys*Hkv*D (grouped)
  int G;
  int n_red;        // 0: no reduction in this launch
  int chunk_tiles;  // grouped dK/dV: the plan's chunk length; 0: per-head
  int max_chunks;
  int split_keys;
  int S, Hkv;
  int causal;
};

// Elements of the reduction (a multiple of 4).
__host__ __device__ inline long reduce_len(const TailReduce& red) { return red.n; }

// Sum the slots of reduction elements i .. i+3 in slot order and round to
// bf16 once, so the result does not depend on which thread or kernel does it.
__device__ __forceinline__ void reduce_at(const TailReduce& red, long i) {
  long e = i;          // element of dk / dv; i is the element of a slot
  int slots = red.G;
  if (red.chunk_tiles > 0) {
    const long row = (long)red.Hkv * HD;
    const long per_b = red.split_keys * row;
    const long bb = i / per_b;
    const long r = i - bb * per_b;
    e = bb * red.S * row + r;
    const int kt = (int)(r / row) >> 7;
    slots = dkdv_chunks(red.G * dkdv_n_qt(red.S, kt, red.causal != 0), red.chunk_tiles, red.max_chunks);
    if (slots <= 1) return;
  }
  f32x4 sk = *reinterpret_cast<const f32x4*>(red.ws_dk + i);
  f32x4 sv = *reinterpret_cast<const f32x4*>(red.ws_dv + i);
  for (int j = 1; j < slots; ++j) {
    sk += *reinterpret_cast<const f32x4*>(red.ws_dk + (long)j * red.n + i);
    sv += *reinterpret_cast<const f32x4*>(red.ws_dv + (long)j * red.n + i);
  }
  if (red.dk32) {
    *reinterpret_cast<f32x4*>(red.dk32 + e) = sk;
    *reinterpret_cast<f32x4*>(red.dv32 + e) = sv;
    return;
  }
  bf16x4 ok, ov;
#pragma unroll
  for (int c = 0; c < 4; ++c) { ok[c] = (__bf16)sk[c]; ov[c] = (__bf16)sv[c]; }
  *reinterpret_cast<bf16x4*>(red.dk + e) = ok;
  *reinterpret_cast<bf16x4*>(red.dv + e) = ov;
}

__global__ __launch_bounds__(256) void attn_dkdv_reduce_kernel(const TailReduce red) {
  const long i = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= reduce_len(red)) return;
  reduce_at(red, i);
}

// The slice of launch slot blockIdx.x (slices go to the last n_red slots).
__device__ __forceinline__ void tail_reduce(const TailReduce& red, int tid, int nthreads) {
  const int slice = (int)blockIdx.x - ((int)gridDim.x - red.n_red);
  if (slice < 0) return;
  const long len = reduce_len(red);
  const long per = ((len + red.n_red - 1) / red.n_red + 3) & ~3L;
  const long end = min(len, per * (slice + 1));
  for (long i = per * slice + 4L * tid; i < end; i += 4L * nthreads) reduce_at(red, i);
}

// ---------------------------------------------------------------------------
// dQ: one workgroup per NW*32 packed query rows (32 per wave); K and V tiles
// of 64 keys arrive by LDS DMA (row-major) in an NSTAGE-deep ring; K^T for
// dQ^T = K^T dS^T is read transposed from the same K tile.  Operands are the
// fp16 q16, k16, v16 and do16 = fp16(2^E dO) (Delta scaled alike); dQ is
// multiplied by scale[0] = 2^-E on the way out.
// F32OUT: dq is fp32 (the values the bf16 path rounds), else bf16.
template <int NW, int NSTAGE, bool CAUSAL, bool F32OUT = false>
__global__ __launch_bounds__(NW * 64, 8 / NW) void attn_dq_kernel(
    const _Float16* __restrict__ q, const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    const _Float16* __restrict__ dO, const float* __restrict__ lse, const float* __restrict__ ndelta,
    const float* __restrict__ scale, void* __restrict__ dq_out,
    int B, int S, int H, int Hkv, int G, float scale2, float sm_scale, int n_tiles, TailReduce red,
    const DispatchOrder ord) {
  constexpr int BM = NW * 32;
  constexpr int BN = TILE_ROWS;
  // LDS: a ring of K tiles, then a ring of V tiles.  The K reads (rows and
  // transposed) stay below 64 KiB, where a ds instruction's offset field
  // reaches every slot from the per-lane bases; when the V ring ends past 64
  // KiB its row reads take per-lane bases that hold the ring's offset (VHI).
  constexpr int KR = 0, VR = NSTAGE * TILE_BYTES;
  constexpr bool VHI = VR + NSTAGE * TILE_BYTES > 0x10000;
  constexpr int DMA_PER_TILE = 2 * (16 / NW);
  static_assert(2 * NSTAGE * TILE_BYTES >= NW * 8192, "the epilogue stages 8 KiB per wave in the ring");
  static_assert(VR <= 0x10000, "K reads must reach every K slot by the offset field");
  __shared__ __attribute__((aligned(1024))) char smem[2 * NSTAGE * TILE_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index (uniform)
  const int nbg = B * Hkv;
  const int item = dispatch_item(ord);    // default order: blockIdx.x
  if (item < 0) {                         // a launch slot without rows still sums its slice
    tail_reduce(red, tid, NW * 64);
    return;
  }
  int tile = item / nbg;
  if (CAUSAL) tile = n_tiles - 1 - tile;
  const int bg = item % nbg;
  const int b = bg / Hkv, g = bg % Hkv;
  const int R = G * S;
  const int r0 = tile * BM;
  const int rw0 = r0 + 32 * w;
  const bool wave_active = rw0 < R;

  const int last_row_wg = min(r0 + BM, R) - 1;
  const int n_kt = CAUSAL ? (min(S - 1, last_row_wg / G) / BN + 1) : (S + BN - 1) / BN;
  const int pw_lo = rw0 / G;
  const int pw_hi = wave_active ? min(S - 1, (min(rw0 + 32, R) - 1) / G) : -1;

  const long kvstride = (long)Hkv * HD;
  const _Float16* kbase = k + ((long)b * S * Hkv + g) * HD;
  const _Float16* vbase = v + ((long)b * S * Hkv + g) * HD;
  const uint32_t dma_off = tile_lane_off(kvstride, tid);
  auto issue_tile = [&](int slot, int kt) {
    const int nk = kt * BN;
    tile_dma<NW>(smem + KR + slot * TILE_BYTES, kbase + (long)nk * kvstride, kvstride, S - nk, dma_off, tid);
    tile_dma<NW>(smem + VR + slot * TILE_BYTES, vbase + (long)nk * kvstride, kvstride, S - nk, dma_off, tid);
  };
#pragma unroll
  for (int st = 0; st < NSTAGE - 1; ++st)
    if (st < n_kt) issue_tile(st, st);

  const int rr = rw0 + l32;
  const int qp = rr / G;
  const int hh = rr - qp * G;
  const bool row_valid = rr < R;
  const long roff = ((long)(b * S + qp) * H + g * G + hh) * HD;
  f16x8 qreg[8], doreg[8];
  float lse_i = INFINITY, dl_i = 0.f;
  if (row_valid) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qreg[ks] = *reinterpret_cast<const f16x8*>(q + roff + 16 * ks + 8 * h);
      doreg[ks] = *reinterpret_cast<const f16x8*>(dO + roff + 16 * ks + 8 * h);
    }
    const long li = ((long)b * H + g * G + hh) * S + qp;
    // P sm_scale = exp2(s scale2 - lse), lse = lse2 - log2 sm_scale (from the
    // workspace): dS comes out scaled, and is rounded to fp16 with the scale
    // in it, as the reference's
    lse_i = lse[li];
    dl_i = ndelta[li];   // -Delta
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) { pin(qreg[ks]); pin(doreg[ks]); }
    __asm__ volatile("" : "+v"(lse_i), "+v"(dl_i));
  } else {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
      for (int t = 0; t < 8; ++t) { qreg[ks][t] = (_Float16)0.f; doreg[ks][t] = (_Float16)0.f; }
    }
  }

  f32x16 negdl;   // the initial accumulator of every dP^T block: -Delta
#pragma unroll
  for (int r = 0; r < 16; ++r) negdl[r] = dl_i;
  f32x16 dqacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) dqacc[db] = zero16();
  const LdsBases lb = make_lds_bases(lane);
  using lds_cp = const MM1_LDS char*;
  lds_cp vrow[8];   // VHI: per-lane bases of the V row reads, VR included, opaque to the compiler
  if constexpr (VHI) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      vrow[ks] = (lds_cp)smem + VR + (lb.row ^ (32 * ks));
      __asm__ volatile("" : "+v"(vrow[ks]));
    }
  }
  // row fragment (jb, ks) of the V tile in slot P
  auto v_rows = [&](auto slot, int jb, int ks) MM1_INLINE {
    constexpr int P = decltype(slot)::value;
    if constexpr (VHI)
      return *reinterpret_cast<const MM1_LDS f16x8*>(vrow[ks] + (P * TILE_BYTES + jb * 8192));
    else
      return rows_a(smem + VR + P * TILE_BYTES, lb, jb, ks);
  };
  wait_dma();
  __syncthreads();

  auto step = [&](auto slot, int kt) {
    constexpr int P = decltype(slot)::value;
    const char* kl = smem + KR + P * TILE_BYTES;
    const bool prefetch = kt + NSTAGE - 1 < n_kt;
    if (prefetch) issue_tile((P + NSTAGE - 1) % NSTAGE, kt + NSTAGE - 1);
    const int k0 = kt * BN;
    if (wave_active && (!CAUSAL || k0 <= pw_hi)) {
      const bool need_mask = CAUSAL ? (k0 + BN - 1 > pw_lo) : (k0 + BN > S);
      // one 32-key block at a time keeps S^T/dP^T at 32 registers
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        // dP^T accumulates onto -Delta: the products give dP - Delta directly
        f32x16 sv = zero16(), dp = negdl;
        // the wave issuing products goes first; the other wave of the SIMD
        // fills the gaps with its dS arithmetic
        wave_prio<1>();
        // K / V fragments read PF k-steps ahead of their products
        constexpr int PF = MM1_DQ_PREFETCH;
        f16x8 ka[PF + 1], va[PF + 1];
#pragma unroll
        for (int ks = 0; ks < PF; ++ks) {
          ka[ks] = rows_a(kl, lb, jb, ks);
          va[ks] = v_rows(slot, jb, ks);
        }
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          if (ks + PF < 8) {
            ka[(ks + PF) % (PF + 1)] = rows_a(kl, lb, jb, ks + PF);
            va[(ks + PF) % (PF + 1)] = v_rows(slot, jb, ks + PF);
          }
          // keep the reads ahead: the scheduler would otherwise sink them
          // to their products and expose the LDS latency on every pair
          __builtin_amdgcn_sched_barrier(0);
          sv = mfma32h(ka[ks % (PF + 1)], qreg[ks], sv);
          dp = mfma32h(va[ks % (PF + 1)], doreg[ks], dp);
          __builtin_amdgcn_sched_barrier(0);
        }
        // dS^T = P^T (dP^T - Delta), masked only in the tiles that need it,
        // as separate straight-line code
        auto dscore = [&](auto masked) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float pr = exp2_fast(fmaf(sv[r], scale2, -lse_i));
            if constexpr (decltype(masked)::value) {
              const int key = k0 + 32 * jb + 8 * (r >> 2) + 4 * h + (r & 3);
              pr = (CAUSAL ? (key > qp) : (key >= S)) ? 0.f : pr;
            }
            sv[r] = pr * dp[r];
          }
        };
        wave_prio<0>();
        if (need_mask) dscore(std::true_type{});
        else dscore(std::false_type{});
        wave_prio<1>();
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const f16x8 sb = pack8(sv, 8 * kh);
#pragma unroll
          for (int db = 0; db < 4; ++db)
            dqacc[db] = mfma32h(tr_a(kl, lb, db, 2 * jb + kh), sb, dqacc[db]);
        }
      }
    }
    if (NSTAGE > 2 && prefetch) {
      __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(DMA_PER_TILE * (NSTAGE - 2)) : "memory");
    } else {
      wait_dma();
    }
    lds_barrier();
  };
  for (int kt = 0; kt < n_kt; kt += NSTAGE) {
    step(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < n_kt) step(std::integral_constant<int, 1>{}, kt + 1);
    if constexpr (NSTAGE > 2) {
      if (kt + 2 < n_kt) step(std::integral_constant<int, 2>{}, kt + 2);
    }
  }

  const float unscale = scale[0];   // 2^-E of do16
  if constexpr (!F32OUT) {
    // every slot is free after the last step's barrier: each wave's rows go
    // out through 8 KiB of it (store_tile_bf16)
    if (wave_active)
      store_tile_bf16(dqacc, unscale, smem + w * 8192, lane, [&](int i) -> __bf16* {
        const int r = rw0 + i;
        if (r >= R) return nullptr;
        const int p = r / G;
        return static_cast<__bf16*>(dq_out) + ((long)(b * S + p) * H + g * G + (r - p * G)) * HD;
      });
  } else if (row_valid) {
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        if constexpr (F32OUT) {
          f32x4 val;
#pragma unroll
          for (int c = 0; c < 4; ++c) val[c] = dqacc[db][4 * a4 + c] * unscale;
          *reinterpret_cast<f32x4*>(static_cast<float*>(dq_out) + roff + 32 * db + 8 * a4 + 4 * h) = val;
        } else {
          bf16x4 val;
#pragma unroll
          for (int c = 0; c < 4; ++c) val[c] = (__bf16)(dqacc[db][4 * a4 + c] * unscale);
          *reinterpret_cast<bf16x4*>(static_cast<__bf16*>(dq_out) + roff + 32 * db + 8 * a4 + 4 * h) = val;
        }
      }
    }
  }

  // dK/dV group sum slice (the partials were completed by an earlier launch)
  tail_reduce(red, tid, NW * 64);
}

// ---------------------------------------------------------------------------
hipError_t launch_delta(const void* o, const void* dO, float* delta, int B, int S, int H,
                        hipStream_t stream) {
  const long rows = (long)B * S * H;
  const long blocks = ((rows + 1) / 2 * 16 + 255) / 256;   // 16 lanes per pair of rows
  hipLaunchKernelGGL(attn_delta_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const __bf16*>(o), static_cast<const __bf16*>(dO), delta, B, S, H);
  return hipGetLastError();
}

// Delta (from o + o_lo, or the caller's delta_in when o is null), max|dO|,
// then do16 = fp16(2^E dO), Delta *= 2^E and the scale cells: what the
// dK/dV and dQ kernels read from the workspace.
hipError_t launch_bwd_prep(const void* o, const uint8_t* o_lo, const void* dO, const float* delta_in,
                           const float* lse2, const float* vmax, char* ws, int B, int S, int H, int Hkv,
                           float sm_scale, hipStream_t stream) {
  const BwdWs w = bwd_ws(B, S, H, Hkv);
  float* delta = reinterpret_cast<float*>(ws + w.delta);
  float* dmax = reinterpret_cast<float*>(ws + w.dmax);
  hipLaunchKernelGGL(attn_delta16_kernel, dim3(kDeltaBlocks), dim3(256), 0, stream,
                     static_cast<const __bf16*>(o), o_lo, static_cast<const __bf16*>(dO), delta_in, lse2,
                     log2f(sm_scale), delta, reinterpret_cast<float*>(ws + w.lse),
                     reinterpret_cast<_Float16*>(ws + w.do16), dmax, B, S, H);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attn_do16_kernel, dim3(1024), dim3(256), 0, stream, static_cast<const __bf16*>(dO),
                     reinterpret_cast<_Float16*>(ws + w.do16), delta, dmax, kDeltaBlocks, vmax, kCvtBlocks,
                     reinterpret_cast<float*>(ws + w.scale), sm_scale, (long)B * S * H * HD, (long)B * H * S);
  return hipGetLastError();
}

// Where the partial sums of dK/dV tiling `variant` live in a workspace:
// `slots` slots of `rows` key rows per batch element (`stride` floats each),
// dK's slots first, then dV's.
WsSlots ws_slots(int B, int S, int H, int Hkv, bool causal, int variant) {
  if (dkdv_grouped(variant)) {
    const DkdvPlan& plan = dkdv_plan(B, S, H, Hkv, causal);
    return {(long)B * plan.split_keys * Hkv * HD, plan.split_keys, plan.C};
  }
  return {(long)B * S * Hkv * HD, S, H / Hkv};
}

// Bytes of the partial sums tiling `variant` writes (0 when it writes none).
size_t bwd_partials_bytes(int B, int S, int H, int Hkv, bool causal, int variant) {
  if (H / Hkv <= 1) return 0;
  const WsSlots w = ws_slots(B, S, H, Hkv, causal, variant);
  return (size_t)2 * w.slots * w.stride * sizeof(float);
}

// The reduction that follows dK/dV tiling `dkdv_variant` (n_red = 0 when
// there is nothing to sum); f32: the sums go to dk / dv as fp32.
TailReduce make_reduce(const float* partials, void* dk, void* dv, bool f32, int B, int S, int H, int Hkv,
                       bool causal, int dkdv_variant) {
  const int G = H / Hkv;
  TailReduce red{};
  red.G = G;
  red.S = S;
  red.Hkv = Hkv;
  red.causal = causal ? 1 : 0;
  if (!partials || G <= 1) return red;
  const WsSlots w = ws_slots(B, S, H, Hkv, causal, dkdv_variant);
  red.n = w.stride;
  red.ws_dk = partials;
  red.ws_dv = red.ws_dk + (long)w.slots * w.stride;
  if (f32) {
    red.dk32 = static_cast<float*>(dk);
    red.dv32 = static_cast<float*>(dv);
  } else {
    red.dk = static_cast<__bf16*>(dk);
    red.dv = static_cast<__bf16*>(dv);
  }
  if (dkdv_grouped(dkdv_variant)) {
    const DkdvPlan& plan = dkdv_plan(B, S, H, Hkv, causal);
    red.chunk_tiles = plan.L;
    red.max_chunks = plan.C;
    red.split_keys = plan.split_keys;
  }
  red.n_red = reduce_len(red) > 0 ? 1 << 30 : 0;
  return red;
}

// The fp16 operands and scaled values the dK/dV and dQ kernels read.
struct BwdOperands {
  const _Float16 *q, *k, *v, *dO;
  const float *lse, *ndelta, *scale;
};

BwdOperands bwd_operands(const char* state, const char* ws, int B, int S, int H, int Hkv) {
  const FwdState f = fwd_state(B, S, H, Hkv);
  const BwdWs w = bwd_ws(B, S, H, Hkv);
  BwdOperands o;
  o.q = reinterpret_cast<const _Float16*>(state + f.q16);
  o.k = reinterpret_cast<const _Float16*>(state + f.k16);
  o.v = reinterpret_cast<const _Float16*>(state + f.v16);
  o.dO = reinterpret_cast<const _Float16*>(ws + w.do16);
  o.lse = reinterpret_cast<const float*>(ws + w.lse);
  o.ndelta = reinterpret_cast<const float*>(ws + w.delta);
  o.scale = reinterpret_cast<const float*>(ws + w.scale);
  return o;
}

// The pipelined dK/dV kernel for one tiling: GROUP (one workgroup per key
// tile over the G heads of its KV group, chunked by dkdv_plan) or per head.
template <bool GROUP, bool F32OUT>
static void launch_dkdv_pipe(const BwdOperands& op, float* ws_dk, float* ws_dv, void* dk, void* dv, int B, int S,
                             int H, int Hkv, bool causal, float scale2, float sm_scale, hipStream_t stream) {
  const int G = H / Hkv;
  const bool ragged = S % 32 != 0;
  const KeyTileOrder order = key_tile_order(B * H);
  dim3 grid;
  int L = 0, C = G;
  const DispatchOrder* ord;
  if constexpr (GROUP) {
    const DkdvPlan& plan = dkdv_plan(B, S, H, Hkv, causal);
    grid = dim3(plan.order.n ? plan.order.n : plan.n_items);
    L = plan.L;
    C = plan.C;
    ord = &plan.order;
  } else {
    const int n_ktiles = (S + 127) / 128;
    grid = dim3(8 * order.m * ((n_ktiles + order.q - 1) / order.q));
    ord = &dispatch_order(row_block_grid(0, B, S, H, Hkv), false);   // unused: default order
  }
  const dim3 block(512);
  const int ws_rows = ws_slots(B, S, H, Hkv, causal, GROUP ? 0 : 1).rows;
#define MM1_DKDV_PIPE(CS, RG)                                                                              \
  hipLaunchKernelGGL((attn_dkdv_pipe_kernel<7, CS, GROUP, RG, F32OUT>), grid, block, 0, stream, op.q, op.k, op.v, \
                     op.dO, op.lse, op.ndelta, op.scale, ws_dk, ws_dv, dk, dv, B, S, H, Hkv, G, scale2,         \
                     sm_scale, order, L, C, *ord, ws_rows)
  if (causal) {
    if (ragged) MM1_DKDV_PIPE(true, true);
    else MM1_DKDV_PIPE(true, false);
  } else {
    if (ragged) MM1_DKDV_PIPE(false, true);
    else MM1_DKDV_PIPE(false, false);
  }
#undef MM1_DKDV_PIPE
}

// dK/dV from the state and a prepared workspace.  variant: 0 = over the
// whole GQA group per key tile (chunked by dkdv_plan), 1 = one workgroup per
// (key tile, query head).  f32: dk / dv are fp32.
hipError_t launch_bwd_dkdv(const char* state, char* ws, void* dk, void* dv, bool f32, int B, int S, int H,
                           int Hkv, bool causal, float sm_scale, int variant, hipStream_t stream) {
  const float scale2 = sm_scale * 1.4426950408889634f;
  const BwdOperands op = bwd_operands(state, ws, B, S, H, Hkv);
  const WsSlots w = ws_slots(B, S, H, Hkv, causal, variant);
  float* ws_dk = H / Hkv > 1 ? reinterpret_cast<float*>(ws + bwd_ws(B, S, H, Hkv).partials) : nullptr;
  float* ws_dv = ws_dk ? ws_dk + (long)w.slots * w.stride : nullptr;
  if (variant == 0) {
    if (f32) launch_dkdv_pipe<true, true>(op, ws_dk, ws_dv, dk, dv, B, S, H, Hkv, causal, scale2, sm_scale, stream);
    else launch_dkdv_pipe<true, false>(op, ws_dk, ws_dv, dk, dv, B, S, H, Hkv, causal, scale2, sm_scale, stream);
  } else {
    if (f32) launch_dkdv_pipe<false, true>(op, ws_dk, ws_dv, dk, dv, B, S, H, Hkv, causal, scale2, sm_scale, stream);
    else launch_dkdv_pipe<false, false>(op, ws_dk, ws_dv, dk, dv, B, S, H, Hkv, causal, scale2, sm_scale, stream);
  }
  return hipGetLastError();
}

hipError_t launch_bwd_reduce(const char* ws, void* dk, void* dv, bool f32, int B, int S, int H, int Hkv,
                             bool causal, int dkdv_variant, hipStream_t stream) {
  const float* partials = reinterpret_cast<const float*>(ws + bwd_ws(B, S, H, Hkv).partials);
  const TailReduce red = make_reduce(partials, dk, dv, f32, B, S, H, Hkv, causal, dkdv_variant);
  if (red.n_red == 0) return hipSuccess;
  const long blocks = (reduce_len(red) / 4 + 255) / 256;
  hipLaunchKernelGGL(attn_dkdv_reduce_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, red);
  return hipGetLastError();
}

template <int NW, int NSTAGE, bool F32OUT>
static void launch_dq_t(const BwdOperands& op, void* dq, int B, int S, int H, int Hkv, bool causal, float scale2,
                        float sm_scale, TailReduce red, const DispatchOrder& ord, hipStream_t stream) {
  const int G = H / Hkv;
  const int BM = NW * 32;
  const int n_qtiles = (G * S + BM - 1) / BM;
  const int n_blocks = ord.n ? ord.n : n_qtiles * B * Hkv;
  if (red.n_red > 0) red.n_red = min(red.n_red, n_blocks);
  dim3 grid(n_blocks), block(NW * 64);
  if (causal)
    hipLaunchKernelGGL((attn_dq_kernel<NW, NSTAGE, true, F32OUT>), grid, block, 0, stream, op.q, op.k, op.v, op.dO,
                       op.lse, op.ndelta, op.scale, dq, B, S, H, Hkv, G, scale2, sm_scale, n_qtiles, red, ord);
  else
    hipLaunchKernelGGL((attn_dq_kernel<NW, NSTAGE, false, F32OUT>), grid, block, 0, stream, op.q, op.k, op.v, op.dO,
                       op.lse, op.ndelta, op.scale, dq, B, S, H, Hkv, G, scale2, sm_scale, n_qtiles, red, ord);
}

// dQ from the state and a prepared workspace.  variant: 0 = 4 waves x
// 2-stage ring (two workgroups per CU), 1 = 8 waves x 3-stage ring (one per
// CU).  reduce: also sum the dK/dV partials that tiling dkdv_variant left in
// the workspace into dk, dv (what launch_bwd_reduce does), in the dQ grid's
// tail.  f32: dq (and dk, dv) are fp32.
hipError_t launch_bwd_dq(const char* state, char* ws, void* dq, bool reduce, void* dk, void* dv, bool f32,
                         int B, int S, int H, int Hkv, bool causal, float sm_scale, int variant, int dkdv_variant,
                         hipStream_t stream) {
  const float scale2 = sm_scale * 1.4426950408889634f;
  const BwdOperands op = bwd_operands(state, ws, B, S, H, Hkv);
  const float* partials = reduce ? reinterpret_cast<const float*>(ws + bwd_ws(B, S, H, Hkv).partials) : nullptr;
  // with n_red = 1 << 30 every workgroup of the grid takes a slice
  const TailReduce red = make_reduce(partials, dk, dv, f32, B, S, H, Hkv, causal, dkdv_variant);
  const DispatchOrder& ord = dispatch_order(dq_grid(variant, B, S, H, Hkv), causal);
  if (variant == 1) {
    if (f32) launch_dq_t<8, 3, true>(op, dq, B, S, H, Hkv, causal, scale2, sm_scale, red, ord, stream);
    else launch_dq_t<8, 3, false>(op, dq, B, S, H, Hkv, causal, scale2, sm_scale, red, ord, stream);
  } else {
    if (f32) launch_dq_t<4, 2, true>(op, dq, B, S, H, Hkv, causal, scale2, sm_scale, red, ord, stream);
    else launch_dq_t<4, 2, false>(op, dq, B, S, H, Hkv, causal, scale2, sm_scale, red, ord, stream);
  }
  return hipGetLastError();
}

}  // namespace mm1
