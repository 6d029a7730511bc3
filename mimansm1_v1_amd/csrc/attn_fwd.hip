// Causal / full GQA flash-attention forward for gfx950.
//
// Follows the algorithm of flash_fwd, CODE/mimans/model/attention_tilelang.py:110-190:
// online softmax in the exp2 domain with scale2 = log2(e)/sqrt(D) (:114, :164-176),
// O normalised by the running sum (:182-183) and lse2 = log2(l) + m*scale2 (:186-188).
//
// Work decomposition (MI355X-first, not the reference's):
//   * The G query heads that share one KV head are packed into one row space:
//     packed row r of KV head g is position r / G, query head g*G + r % G.
//     A workgroup owns BM = 32*NW consecutive packed rows (32 per wave), so
//     each K/V tile it stages in LDS serves all G heads at once.
//   * The product is computed transposed, S^T = K Q^T (keys on the MFMA M axis,
//     queries on N), so every lane owns one query column: the row max needs a
//     single cross-half exchange and P^T feeds the next product as a B operand
//     straight from the accumulator registers (pi order, see mm1_common.h).
//   * O^T = V^T P^T keeps the same one-query-per-lane layout for the rescale;
//     V^T is read transposed from the row-major V tile.
//   * K and V tiles arrive by LDS DMA into an NSTAGE-deep ring, one barrier
//     per key tile; no staging registers.
//   * The running max is only moved (and O, l rescaled) when a row's max
//     grows by more than 2^8 (log2 units); otherwise P = exp2(s - m_old) <= 256
//     stays exact in fp32 and within fp16's range, and the final
//     normalisation uses the same frame, so the result is unchanged.
//   * Operands are fp16: K and V come as fp16 copies (attn_cvt16_kernel, in
//     the forward state), Q is converted in registers, and P is rounded to
//     fp16 (11 significant bits) before O^T += V^T P^T.  The reference rounds
//     P to bf16 there (AT:178-180); the finer rounding keeps O, and the
//     backward's Delta = rowsum(O dO), within the stated tolerance of the
//     fp32 math also for peaky softmax rows.
//   * For the backward the forward also leaves, in the state, the fp16 copy
//     of Q and one byte per value of O (o_lo: the 8 fp32 mantissa bits after
//     the bf16 truncation, lo8_bits): Delta is then computed from 15
//     significant bits of O instead of the 8 of the bf16 output.
#include <type_traits>

#include "dispatch_order.h"
#include "attn_layout.h"
#include "mm1_common.h"

// 1: the forward stores its fp16 copy of Q after the prologue's wait
// (store_q16); 0: with the loads, before it.
#ifndef MM1_FWD_Q16_LATE
#define MM1_FWD_Q16_LATE 1
#endif

namespace mm1 {

constexpr float kRescaleThreshold = 8.0f;   // log2 units

// ---------------------------------------------------------------------------
// bf16 -> fp16 copies of K and V (blockIdx.y = tensor), with the largest |x|
// of each workgroup's share in part_max[y][blockIdx.x] (the backward sizes
// the scale of dO from max|V|).  8 values per thread per step, grid-stride.
struct Cvt16 {
  const __bf16* src[2];
  _Float16* dst[2];
  float* part_max[2];   // nullptr: no maxima
  long n[2];            // elements, a multiple of 8
};

__global__ __launch_bounds__(256) void attn_cvt16_kernel(const Cvt16 c) {
  const int y = blockIdx.y;
  const __bf16* src = c.src[y];
  _Float16* dst = c.dst[y];
  const long n8 = c.n[y] / 8;
  float mx = 0.f;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n8; i += (long)gridDim.x * 256) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(src + 8 * i);
    f16x8 r;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float f = (float)x[t];
      mx = fmaxf(mx, fabsf(f));
      r[t] = (_Float16)f;
    }
    *reinterpret_cast<f16x8*>(dst + 8 * i) = r;
  }
  if (!c.part_max[y]) return;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  __shared__ float wmax[4];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0)
    c.part_max[y][blockIdx.x] = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}

// Query operands of a wave (B of S^T = K Q^T): row rr of the packed row
// space, the 64 values 16*ks + 8*h .. +7 (ks = 0..7) of it, converted to
// fp16; with q16 != nullptr also stored there (the backward's copy of Q).
__device__ __forceinline__ void load_q16(f16x8 (&qreg)[8], const __bf16* q, _Float16* q16, long roff,
                                         bool valid, int h) {
  if (valid) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
      qreg[ks] = bf16_to_f16(*reinterpret_cast<const bf16x8*>(q + roff + 16 * ks + 8 * h));
    if (!MM1_FWD_Q16_LATE && q16) {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) *reinterpret_cast<f16x8*>(q16 + roff + 16 * ks + 8 * h) = qreg[ks];
    }
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) pin(qreg[ks]);
  } else {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
      for (int t = 0; t < 8; ++t) qreg[ks][t] = (_Float16)0.f;
    }
  }
}

// The fp16 copy of the wave's query rows (q16 != nullptr), stored after the
// prologue's wait for its K / V copies: the wait counts stores too, so a
// store issued before it would hold the first tile back.
__device__ __forceinline__ void store_q16(const f16x8 (&qreg)[8], _Float16* q16, long roff, bool valid, int h) {
  if (MM1_FWD_Q16_LATE && q16 && valid) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) *reinterpret_cast<f16x8*>(q16 + roff + 16 * ks + 8 * h) = qreg[ks];
  }
}

// The outputs of a wave's 32 rows: bf16 O through LDS (store_tile_bf16, with
// the residual bytes to o_lo when o_lo != nullptr), or fp32 O written
// directly (F32OUT: the values the bf16 output rounds; o_lo then holds their
// residual bytes as well); lse2 in both cases.
template <bool F32OUT>
__device__ __forceinline__ void store_fwd_rows(const f32x16 (&oacc)[4], float m_run, float l_run, float scale2,
                                               void* o_out, uint8_t* o_lo, float* lse2, char* lds, int lane,
                                               int b, int g, int S, int H, int G, int R, int rw0) {
  const int h = lane >> 5, l32 = lane & 31;
  const float l_tot = xhalf_sum(l_run);
  const float inv = 1.f / l_tot;
  const int rr = rw0 + l32;
  const int qpos = rr / G, hq = rr - qpos * G;
  if (rr < R && h == 0) lse2[((long)b * H + g * G + hq) * S + qpos] = m_run * scale2 + log2f(l_tot);
  auto row_of = [&](int i) -> long {
    const int r = rw0 + i;
    if (r >= R) return -1;
    const int p = r / G;
    return ((long)(b * S + p) * H + g * G + (r - p * G)) * HD;
  };
  if constexpr (!F32OUT) {
    auto dst = [&](int i) -> __bf16* {
      const long off = row_of(i);
      return off < 0 ? nullptr : static_cast<__bf16*>(o_out) + off;
    };
    if (o_lo) {
      store_tile_bf16_lo(oacc, inv, lds, lane, dst, [&](int i) -> uint8_t* {
        const long off = row_of(i);
        return off < 0 ? nullptr : o_lo + off;
      });
    } else {
      store_tile_bf16(oacc, inv, lds, lane, dst);
    }
  } else if (rr < R) {
    const long row = row_of(l32);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int a4 = 0; a4 < 4; ++a4) {
        f32x4 val;
        uint32_t lo = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          val[c] = oacc[db][4 * a4 + c] * inv;
          lo |= lo8_bits(val[c]) << (8 * c);
        }
        *reinterpret_cast<f32x4*>(static_cast<float*>(o_out) + row + 32 * db + 8 * a4 + 4 * h) = val;
        if (o_lo) *reinterpret_cast<uint32_t*>(o_lo + row + 32 * db + 8 * a4 + 4 * h) = lo;
      }
    }
  }
}

// NW waves x 32 packed query rows per workgroup; NSTAGE-deep K/V ring.
// F32OUT: O is written in fp32 (the values the bf16 output rounds).
template <int NW, int NSTAGE, bool CAUSAL, bool F32OUT = false>
__global__ __launch_bounds__(NW * 64, 8 / NW) void attn_fwd_kernel(
    const __bf16* __restrict__ q, const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    void* __restrict__ o_out, float* __restrict__ lse2, _Float16* __restrict__ q16, uint8_t* __restrict__ o_lo,
    int B, int S, int H, int Hkv, int G, float scale2, int n_tiles, const DispatchOrder ord) {
  constexpr int BM = NW * 32;     // packed rows per workgroup
  constexpr int BN = TILE_ROWS;   // keys per iteration
  constexpr int BUF = 2 * TILE_BYTES;
  constexpr int DMA_PER_TILE = 2 * (16 / NW);   // copies one wave issues per K/V tile
  static_assert(NSTAGE * BUF >= NW * 8192, "the epilogue stages 8 KiB per wave in the ring");
  __shared__ __attribute__((aligned(1024))) char smem[NSTAGE * BUF];

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index (uniform)
  const int nbg = B * Hkv;
  const int item = dispatch_item(ord);     // default order: blockIdx.x
  if (item < 0) return;
  int tile = item / nbg;
  if (CAUSAL) tile = n_tiles - 1 - tile;   // longest rows first
  const int bg = item % nbg;
  const int b = bg / Hkv, g = bg % Hkv;
  const int R = G * S;
  const int r0 = tile * BM;
  const int rw0 = r0 + w * 32;
  const bool wave_active = rw0 < R;

  const int last_row_wg = min(r0 + BM, R) - 1;
  const int n_kt = CAUSAL ? (min(S - 1, last_row_wg / G) / BN + 1) : (S + BN - 1) / BN;
  const int pw_lo = rw0 / G;
  const int pw_hi = wave_active ? min(S - 1, (min(rw0 + 32, R) - 1) / G) : -1;

  const long kvstride = (long)Hkv * HD;
  const _Float16* kbase = k + ((long)b * S * Hkv + g) * HD;
  const _Float16* vbase = v + ((long)b * S * Hkv + g) * HD;
  const uint32_t dma_off = tile_lane_off(kvstride, tid);
  auto issue_tile = [&](char* buf, int kt) {
    const int nk = kt * BN;
    tile_dma<NW>(buf, kbase + (long)nk * kvstride, kvstride, S - nk, dma_off, tid);
    tile_dma<NW>(buf + TILE_BYTES, vbase + (long)nk * kvstride, kvstride, S - nk, dma_off, tid);
  };
#pragma unroll
  for (int st = 0; st < NSTAGE - 1; ++st)
    if (st < n_kt) issue_tile(smem + st * BUF, st);

  // Query operands (B of S^T = K Q^T), loaded once.
  f16x8 qreg[8];
  const int rr = rw0 + l32;
  const int qpos = rr / G;
  const int hq = rr - qpos * G;
  const long qoff = ((long)(b * S + qpos) * H + g * G + hq) * HD;
  load_q16(qreg, q, q16, qoff, rr < R, h);

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  const LdsBases lb = make_lds_bases(lane);
  wait_dma();
  __syncthreads();
  store_q16(qreg, q16, qoff, rr < R, h);

  // One key tile; the loop below runs it NSTAGE times per trip so the ring
  // slot (and every LDS offset) is a compile-time constant.
  auto step = [&](auto slot, int kt) {
    constexpr int P = decltype(slot)::value;
    const char* kl = smem + P * BUF;
    const char* vl = kl + TILE_BYTES;
    const bool prefetch = kt + NSTAGE - 1 < n_kt;
    if (prefetch) issue_tile(smem + ((P + NSTAGE - 1) % NSTAGE) * BUF, kt + NSTAGE - 1);
    const int k0 = kt * BN;
    if (wave_active && (!CAUSAL || k0 <= pw_hi)) {
      f32x16 sacc[2];
      sacc[0] = zero16();
      sacc[1] = zero16();
      rows_chain2(kl, lb, qreg, sacc);
      const bool need_mask = CAUSAL ? (k0 + BN - 1 > pw_lo) : (k0 + BN > S);
      if (need_mask) {
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + 32 * jb + 8 * (r >> 2) + 4 * h + (r & 3);
            const bool masked = CAUSAL ? (key > qpos) : (key >= S);
            sacc[jb][r] = masked ? -INFINITY : sacc[jb][r];
          }
        }
      }
      // Row max of this tile; move the running max only when it grows by
      // more than the threshold (any lane of the wave -> whole wave rescales).
      float mx = -INFINITY;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[jb][r]);
      }
      mx = xhalf_max(mx);
      const float m_new = fmaxf(m_run, mx);
      if (__any(!((m_new - m_run) * scale2 <= kRescaleThreshold))) {
        const float alpha = (m_new == -INFINITY) ? 1.f : exp2_fast((m_run - m_new) * scale2);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
        m_run = m_new;
      }
      const float ms = (m_run == -INFINITY) ? 0.f : m_run * scale2;
      float sum = 0.f;
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pr = exp2_fast(fmaf(sacc[jb][r], scale2, -ms));
          sacc[jb][r] = pr;
          sum += pr;
        }
      }
      l_run += sum;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const f16x8 pb = pack8(sacc[ks >> 1], 8 * (ks & 1));
#pragma unroll
        for (int db = 0; db < 4; ++db) oacc[db] = mfma32h(tr_a(vl, lb, db, ks), pb, oacc[db]);
      }
    }
    // tile kt+1 must have landed; the newer prefetches stay in flight
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

  if (!wave_active) return;
  // every slot is free after the last step's barrier: each wave's rows go
  // out through 8 KiB of it
  store_fwd_rows<F32OUT>(oacc, m_run, l_run, scale2, o_out, o_lo, lse2, smem + w * 8192, lane, b, g, S, H, G,
                         R, rw0);
}

// Ping-pong forward: one workgroup of 8 waves per CU over 256 packed query
// rows.  Group A (waves 0-3) owns rows 0-127, group B (waves 4-7) rows
// 128-255, and the waves of the two groups pair up on the four SIMDs.  The
// work on a 64-key tile is split into
//   part 1: S^T = K Q^T, row max, lazy rescale, P = exp2(..), row sums;
//   part 2: O^T += V^T P^T,
// and group B runs half a tile behind group A, so in every phase (one
// barrier each) one wave of a SIMD runs part 1 while the other runs part 2:
// the SIMD sees 16 products from each wave, and the softmax VALU work of one
// wave runs under the other wave's products.
//   phase 2t  : A part 1 of tile t,  B part 2 of tile t-1
//   phase 2t+1: A part 2 of tile t,  B part 1 of tile t
// K(t) is read in phases 2t and 2t+1, V(t) in 2t+1 and 2t+2.  Two-slot rings
// for each: the group running part 2 issues the copies of the phase (B
// refills K(t+2) in phase 2t+2, A refills V(t+2) in phase 2t+3) and waits for
// them at the end of the next phase, two phases ahead of their first use.
template <bool CAUSAL, bool F32OUT = false>
__global__ __launch_bounds__(512, 1) void attn_fwd_pp_kernel(
    const __bf16* __restrict__ q, const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    void* __restrict__ o, float* __restrict__ lse2, _Float16* __restrict__ q16, uint8_t* __restrict__ o_lo,
    int B, int S, int H, int Hkv, int G, float scale2, int n_tiles, const DispatchOrder ord) {
  constexpr int BM = 256;         // packed rows per workgroup
  constexpr int BN = TILE_ROWS;   // keys per tile
  __shared__ __attribute__((aligned(1024))) char smem[4 * TILE_BYTES];   // K slots 0, 1; V slots 0, 1

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index (uniform)
  const int grp = w >> 2;                                    // 0 = A, 1 = B
  const int nbg = B * Hkv;
  const int item = dispatch_item(ord);     // default order: blockIdx.x
  if (item < 0) return;
  int tile = item / nbg;
  if (CAUSAL) tile = n_tiles - 1 - tile;   // longest rows first
  const int bg = item % nbg;
  const int b = bg / Hkv, g = bg % Hkv;
  const int R = G * S;
  const int r0 = tile * BM;
  const int rw0 = r0 + w * 32;
  const bool wave_active = rw0 < R;

  const int last_row_wg = min(r0 + BM, R) - 1;
  const int n_kt = CAUSAL ? (min(S - 1, last_row_wg / G) / BN + 1) : (S + BN - 1) / BN;
  const int pw_lo = rw0 / G;

  const long kvstride = (long)Hkv * HD;
  const _Float16* kbase = k + ((long)b * S * Hkv + g) * HD;
  const _Float16* vbase = v + ((long)b * S * Hkv + g) * HD;
  const uint32_t dma_off = tile_lane_off(kvstride, tid);
  auto kslot = [&](int j) { return smem + j * TILE_BYTES; };
  auto vslot = [&](int j) { return smem + (2 + j) * TILE_BYTES; };
  // all 8 waves (prologue) or the 4 waves of one group (in the loop; the
  // quad a wave copies depends on w & 3 only, as tile_dma<4> requires)
  auto copy8 = [&](char* dst, const _Float16* base, int kt) {
    const int nk = kt * BN;
    tile_dma<8>(dst, base + (long)nk * kvstride, kvstride, S - nk, dma_off, tid);
  };
  auto copy4 = [&](char* dst, const _Float16* base, int kt) {
    const int nk = kt * BN;
    tile_dma<4>(dst, base + (long)nk * kvstride, kvstride, S - nk, dma_off, tid & 255);
  };
  copy8(kslot(0), kbase, 0);
  copy8(vslot(0), vbase, 0);
  if (n_kt > 1) {
    copy8(kslot(1), kbase, 1);
    copy8(vslot(1), vbase, 1);
  }

  // Query operands (B of S^T = K Q^T), loaded once.
  f16x8 qreg[8];
  const int rr = rw0 + l32;
  const int qpos = rr / G;
  const int hq = rr - qpos * G;
  const long qoff = ((long)(b * S + qpos) * H + g * G + hq) * HD;
  load_q16(qreg, q, q16, qoff, rr < R, h);

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) oacc[db] = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  f16x8 pb[4];    // P(t) of part 1, the B operand of part 2
  const LdsBases lb = make_lds_bases(lane);
  wait_dma();
  __syncthreads();
  store_q16(qreg, q16, qoff, rr < R, h);

  // part 1 of tile kt from K slot J
  auto part1 = [&](auto jslot, int kt) {
    constexpr int J = decltype(jslot)::value;
    const char* kl = kslot(J);
    const int k0 = kt * BN;
    f32x16 sacc[2];
    sacc[0] = zero16();
    sacc[1] = zero16();
    rows_chain2(kl, lb, qreg, sacc);
    if (CAUSAL ? (k0 + BN - 1 > pw_lo) : (k0 + BN > S)) {
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 32 * jb + 8 * (r >> 2) + 4 * h + (r & 3);
          sacc[jb][r] = (CAUSAL ? (key > qpos) : (key >= S)) ? -INFINITY : sacc[jb][r];
        }
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[jb][r]);
    }
    mx = xhalf_max(mx);
    const float m_new = fmaxf(m_run, mx);
    if (__any(!((m_new - m_run) * scale2 <= kRescaleThreshold))) {
      const float alpha = (m_new == -INFINITY) ? 1.f : exp2_fast((m_run - m_new) * scale2);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] *= alpha;
      m_run = m_new;
    }
    const float ms = (m_run == -INFINITY) ? 0.f : m_run * scale2;
    float sum = 0.f;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = exp2_fast(fmaf(sacc[jb][r], scale2, -ms));
        sacc[jb][r] = pr;
        sum += pr;
      }
    }
    l_run += sum;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) pb[ks] = pack8(sacc[ks >> 1], 8 * (ks & 1));
  };
  // part 2 of a tile from V slot J
  auto part2 = [&](auto jslot) {
    constexpr int J = decltype(jslot)::value;
    const char* vl = vslot(J);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int db = 0; db < 4; ++db) oacc[db] = mfma32h(tr_a(vl, lb, db, ks), pb[ks], oacc[db]);
    }
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  if (grp == 0) {
    // phase 2t: part 1 (t); phase 2t+1: part 2 (t), refill V(t+1) when t >= 1
    // (V(0), V(1) come from the prologue); the refill is waited for at the
    // end of phase 2t+2.
    auto tile_a = [&](auto jslot, int t) {
      part1(jslot, t);
      if (t >= 2) wait_dma();          // V(t) refilled in phase 2t-1
      lds_barrier();
      if (t >= 1 && t + 1 < n_kt) copy4(vslot(decltype(jslot)::value ^ 1), vbase, t + 1);
      part2(jslot);
      lds_barrier();
    };
    for (int t = 0; t < n_kt; t += 2) {
      tile_a(I0{}, t);
      if (t + 1 < n_kt) tile_a(I1{}, t + 1);
    }
  } else {
    // phase 2t+1: part 1 (t); phase 2t+2: part 2 (t), refill K(t+2) (its slot
    // was last read in phase 2t+1), waited for at the end of phase 2t+3.
    lds_barrier();   // phase 0
    auto tile_b = [&](auto jslot, int t) {
      part1(jslot, t);
      if (t >= 1) wait_dma();          // K(t+1) refilled in phase 2t
      lds_barrier();
      if (t + 2 < n_kt) copy4(kslot(decltype(jslot)::value), kbase, t + 2);
      part2(jslot);
      if (t + 1 < n_kt) lds_barrier();
    };
    for (int t = 0; t < n_kt; t += 2) {
      tile_b(I0{}, t);
      if (t + 1 < n_kt) tile_b(I1{}, t + 1);
    }
  }
  wait_dma();

  // The rows go out through LDS (store_tile_bf16): group A's through the K
  // slots, free since B's last part 1 (before A's last barrier), while B
  // runs the last part 2; group B's through the V slots after a final
  // barrier.
  auto store_rows = [&](char* region) {
    if (!wave_active) return;
    store_fwd_rows<F32OUT>(oacc, m_run, l_run, scale2, o, o_lo, lse2, region + (w & 3) * 8192, lane, b, g, S,
                           H, G, R, rw0);
  };
  if (grp == 0) {
    store_rows(kslot(0));
    lds_barrier();
  } else {
    lds_barrier();
    store_rows(vslot(0));
  }
}

// K, V -> k16, v16 (with max|V| partials in vmax when it is not null).
hipError_t launch_cvt_kv(const void* k, const void* v, _Float16* k16, _Float16* v16, float* kmax, float* vmax,
                         long n, hipStream_t stream) {
  Cvt16 c{};
  c.src[0] = static_cast<const __bf16*>(k);
  c.src[1] = static_cast<const __bf16*>(v);
  c.dst[0] = k16;
  c.dst[1] = v16;
  c.part_max[0] = kmax;
  c.part_max[1] = vmax;
  c.n[0] = c.n[1] = n;
  hipLaunchKernelGGL(attn_cvt16_kernel, dim3(kCvtBlocks, 2), dim3(256), 0, stream, c);
  return hipGetLastError();
}

// One bf16 tensor -> fp16 (Q of a backward without a forward state).
hipError_t launch_cvt16(const void* x, _Float16* x16, long n, hipStream_t stream) {
  Cvt16 c{};
  c.src[0] = static_cast<const __bf16*>(x);
  c.dst[0] = x16;
  c.n[0] = n;
  hipLaunchKernelGGL(attn_cvt16_kernel, dim3(kCvtBlocks, 1), dim3(256), 0, stream, c);
  return hipGetLastError();
}

template <int NW, int NSTAGE, bool F32OUT>
static void launch_fwd_t(const __bf16* q, const _Float16* k, const _Float16* v, void* o, float* lse2,
                         _Float16* q16, uint8_t* o_lo, int B, int S, int H, int Hkv, bool causal, float scale2,
                         const DispatchOrder& ord, hipStream_t stream) {
  const int G = H / Hkv;
  const int BM = NW * 32;
  const int n_tiles = (G * S + BM - 1) / BM;
  dim3 grid(ord.n ? ord.n : n_tiles * B * Hkv), block(NW * 64);
  if (causal)
    hipLaunchKernelGGL((attn_fwd_kernel<NW, NSTAGE, true, F32OUT>), grid, block, 0, stream, q, k, v, o, lse2, q16,
                       o_lo, B, S, H, Hkv, G, scale2, n_tiles, ord);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<NW, NSTAGE, false, F32OUT>), grid, block, 0, stream, q, k, v, o, lse2,
                       q16, o_lo, B, S, H, Hkv, G, scale2, n_tiles, ord);
}

template <bool F32OUT>
static void launch_fwd_v(const __bf16* qp, const _Float16* kp, const _Float16* vp, void* o, float* lse2,
                         _Float16* q16, uint8_t* o_lo, int B, int S, int H, int Hkv, bool causal, float scale2,
                         int variant, hipStream_t stream) {
  const DispatchOrder& ord = dispatch_order(row_block_grid(variant, B, S, H, Hkv), causal);
  if (variant == 0) {
    const int G = H / Hkv;
    const int n_tiles = (G * S + 255) / 256;
    dim3 grid(ord.n ? ord.n : n_tiles * B * Hkv), block(512);
    if (causal)
      hipLaunchKernelGGL((attn_fwd_pp_kernel<true, F32OUT>), grid, block, 0, stream, qp, kp, vp, o, lse2, q16, o_lo,
                         B, S, H, Hkv, G, scale2, n_tiles, ord);
    else
      hipLaunchKernelGGL((attn_fwd_pp_kernel<false, F32OUT>), grid, block, 0, stream, qp, kp, vp, o, lse2, q16,
                         o_lo, B, S, H, Hkv, G, scale2, n_tiles, ord);
  } else if (variant == 2) {
    launch_fwd_t<8, 3, F32OUT>(qp, kp, vp, o, lse2, q16, o_lo, B, S, H, Hkv, causal, scale2, ord, stream);
  } else {
    launch_fwd_t<4, 2, F32OUT>(qp, kp, vp, o, lse2, q16, o_lo, B, S, H, Hkv, causal, scale2, ord, stream);
  }
}

// The forward over a state (mm1_attn_fwd_state_size): K and V are converted
// into it first; the kernels then read k16 / v16 and, with `save`, write q16
// and o_lo for the backward.  F32 (o is float*): fp32 O, same kernels.
// variant: 0 = attn_fwd_pp_kernel (8 waves, two groups half a tile apart),
//          1 = 4 waves x 2-stage ring (two workgroups per CU),
//          2 = 8 waves x 3-stage ring (one workgroup per CU).
hipError_t launch_fwd(const void* q, const void* k, const void* v, void* o, float* lse2, bool f32,
                      _Float16* q16, _Float16* k16, _Float16* v16, uint8_t* o_lo, float* vmax, bool save,
                      int B, int S, int H, int Hkv, bool causal, float sm_scale, int variant, hipStream_t stream) {
  const float scale2 = sm_scale * 1.4426950408889634f;
  hipError_t e = launch_cvt_kv(k, v, k16, v16, nullptr, vmax, (long)B * S * Hkv * HD, stream);
  if (e != hipSuccess) return e;
  auto qp = static_cast<const __bf16*>(q);
  if (f32)
    launch_fwd_v<true>(qp, k16, v16, o, lse2, save ? q16 : nullptr, save ? o_lo : nullptr, B, S, H, Hkv, causal,
                       scale2, variant, stream);
  else
    launch_fwd_v<false>(qp, k16, v16, o, lse2, save ? q16 : nullptr, save ? o_lo : nullptr, B, S, H, Hkv, causal,
                        scale2, variant, stream);
  return hipGetLastError();
}

}  // namespace mm1
