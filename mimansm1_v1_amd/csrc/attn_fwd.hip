// Causal / full GQA flash-attention forward for gfx950.
//
// Follows the algorithm of flash_fwd, CODE/mimans/model/attention_tilelang.py:110-190:
// online softmax in the exp2 domain with scale2 = log2(e)/sqrt(D) (:114, :164-176),
// O normalised by the running sum (:182-183) and lse2 = log2(l) + m*scale2 (:186-188).
//
// Work decomposition (MI355X-first, not the reference's):
//   * The G query heads that share one KV head are packed into one row space:
//     packed row r of KV head g is position r / G, query head g*G + r % G.
//     A workgroup owns BM = 4*QW consecutive packed rows, so each K/V tile it
//     stages in LDS serves all G heads at once.
//   * The product is computed transposed, S^T = K Q^T (keys on the MFMA M axis,
//     queries on N), so every lane owns one query column: the row max needs a
//     single cross-half exchange and P^T feeds the next product as a B operand
//     straight from the accumulator registers (pi order, see mm1_common.h).
//   * O^T = V^T P^T keeps the same one-query-per-lane layout for the rescale;
//     V^T is read transposed from the row-major V tile.
//   * K and V tiles arrive by LDS DMA into a two-stage ring, one barrier per
//     key tile; no staging registers.
//   * The running max is only moved (and O, l rescaled) when a row's max
//     grows by more than 2^8 (log2 units); otherwise P = exp2(s - m_old) <= 256
//     stays exact in fp32 and bf16, and the final normalisation uses the same
//     frame, so the result is unchanged.
#include "mm1_common.h"

namespace mm1 {

constexpr float kRescaleThreshold = 8.0f;   // log2 units

template <int QW, bool CAUSAL>
__global__ __launch_bounds__(256, (QW == 32 ? 2 : 1)) void attn_fwd_kernel(
    const __bf16* __restrict__ q, const __bf16* __restrict__ k, const __bf16* __restrict__ v,
    __bf16* __restrict__ o, float* __restrict__ lse2,
    int B, int S, int H, int Hkv, int G, float scale2, int n_tiles) {
  constexpr int NQB = QW / 32;    // 32-query blocks per wave
  constexpr int BM = 4 * QW;      // packed rows per workgroup
  constexpr int BN = TILE_ROWS;   // keys per iteration
  constexpr int BUF = 2 * TILE_BYTES;
  __shared__ __attribute__((aligned(1024))) char smem[2 * BUF];

  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index (uniform)
  const int nbg = B * Hkv;
  int tile = blockIdx.x / nbg;
  if (CAUSAL) tile = n_tiles - 1 - tile;   // longest rows first
  const int bg = blockIdx.x % nbg;
  const int b = bg / Hkv, g = bg % Hkv;
  const int R = G * S;
  const int r0 = tile * BM;
  const int rw0 = r0 + w * QW;
  const bool wave_active = rw0 < R;

  const long kvstride = (long)Hkv * HD;
  const __bf16* kbase = k + ((long)b * S * Hkv + g) * HD;
  const __bf16* vbase = v + ((long)b * S * Hkv + g) * HD;
  const uint32_t dma_off = tile_lane_off(kvstride, tid);
  tile_dma<4>(smem, kbase, kvstride, S, dma_off, tid);
  tile_dma<4>(smem + TILE_BYTES, vbase, kvstride, S, dma_off, tid);

  // Query operands (B of S^T = K Q^T), loaded once.
  bf16x8 qreg[NQB][8];
  int qpos[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int rr = rw0 + 32 * qb + l32;
    const int p = rr / G;
    const int hh = rr - p * G;
    qpos[qb] = p;
    if (rr < R) {
      const __bf16* src = q + ((long)(b * S + p) * H + g * G + hh) * HD + 8 * h;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qreg[qb][ks] = *reinterpret_cast<const bf16x8*>(src + 16 * ks);
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) pin(qreg[qb][ks]);
    } else {
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
        for (int t = 0; t < 8; ++t) qreg[qb][ks][t] = (__bf16)0.f;
      }
    }
  }

  const int last_row_wg = min(r0 + BM, R) - 1;
  const int n_kt = CAUSAL ? (min(S - 1, last_row_wg / G) / BN + 1) : (S + BN - 1) / BN;
  const int pw_lo = rw0 / G;
  const int pw_hi = wave_active ? min(S - 1, (min(rw0 + QW, R) - 1) / G) : -1;

  f32x16 oacc[4][NQB];
  float m_run[NQB], l_run[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[db][qb] = zero16();
  }
  wait_dma();
  __syncthreads();

  for (int kt = 0; kt < n_kt; ++kt) {
    const char* kl = smem + (kt & 1) * BUF;
    const char* vl = kl + TILE_BYTES;
    if (kt + 1 < n_kt) {
      char* nb = smem + ((kt + 1) & 1) * BUF;
      const int nk = (kt + 1) * BN;
      tile_dma<4>(nb, kbase + (long)nk * kvstride, kvstride, S - nk, dma_off, tid);
      tile_dma<4>(nb + TILE_BYTES, vbase + (long)nk * kvstride, kvstride, S - nk, dma_off, tid);
    }
    const int k0 = kt * BN;
    if (wave_active && (!CAUSAL || k0 <= pw_hi)) {
      f32x16 sacc[2][NQB];
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) sacc[jb][qb] = zero16();
      }
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
          const bf16x8 a = lds_a_rows(kl, jb, ks, lane);
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) sacc[jb][qb] = mfma32(a, qreg[qb][ks], sacc[jb][qb]);
        }
      }
      const bool need_mask = CAUSAL ? (k0 + BN - 1 > pw_lo) : (k0 + BN > S);
      if (need_mask) {
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + 32 * jb + 8 * (r >> 2) + 4 * h + (r & 3);
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) {
              const bool masked = CAUSAL ? (key > qpos[qb]) : (key >= S);
              if (masked) sacc[jb][qb][r] = -INFINITY;
            }
          }
        }
      }
      // Row max of this tile; move the running max only when it grows by
      // more than the threshold (any lane of the wave -> whole wave rescales).
      float mnew[NQB];
      bool grow = false;
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        float mx = -INFINITY;
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[jb][qb][r]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        mnew[qb] = fmaxf(m_run[qb], mx);
        grow |= !((mnew[qb] - m_run[qb]) * scale2 <= kRescaleThreshold);
      }
      if (__any(grow)) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          const float m_new = mnew[qb];
          const bool none = (m_new == -INFINITY);
          const float alpha = none ? 1.f : exp2_fast((m_run[qb] - m_new) * scale2);
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < 4; ++db) oacc[db][qb] *= alpha;
          m_run[qb] = m_new;
        }
      }
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        const float ms = (m_run[qb] == -INFINITY) ? 0.f : m_run[qb] * scale2;
        float sum = 0.f;
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float p = exp2_fast(fmaf(sacc[jb][qb][r], scale2, -ms));
            sacc[jb][qb][r] = p;
            sum += p;
          }
        }
        l_run[qb] += sum;
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf16x8 pb[NQB];
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) pb[qb] = pack8(sacc[ks >> 1][qb], 8 * (ks & 1));
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const bf16x8 a = lds_a_tr(vl, db, ks, lane);
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) oacc[db][qb] = mfma32(a, pb[qb], oacc[db][qb]);
        }
      }
    }
    wait_dma();
    __syncthreads();
  }

  if (!wave_active) return;
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const float l_tot = l_run[qb] + __shfl_xor(l_run[qb], 32);
    const float inv = 1.f / l_tot;
    const int rr = rw0 + 32 * qb + l32;
    if (rr < R) {
      const int p = qpos[qb];
      const int hh = rr - p * G;
      __bf16* dst = o + ((long)(b * S + p) * H + g * G + hh) * HD;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) {
          bf16x4 val;
#pragma unroll
          for (int c = 0; c < 4; ++c) val[c] = (__bf16)(oacc[db][qb][4 * a4 + c] * inv);
          *reinterpret_cast<bf16x4*>(dst + 32 * db + 8 * a4 + 4 * h) = val;
        }
      }
      if (h == 0) lse2[((long)b * H + g * G + hh) * S + p] = m_run[qb] * scale2 + log2f(l_tot);
    }
  }
}

hipError_t launch_fwd(const void* q, const void* k, const void* v, void* o, float* lse2,
                      int B, int S, int H, int Hkv, bool causal, float sm_scale, int qw,
                      hipStream_t stream) {
  const int G = H / Hkv;
  const float scale2 = sm_scale * 1.4426950408889634f;
  const int BM = 4 * qw;
  const int n_tiles = (G * S + BM - 1) / BM;
  dim3 grid(n_tiles * B * Hkv), block(256);
  auto qp = static_cast<const __bf16*>(q);
  auto kp = static_cast<const __bf16*>(k);
  auto vp = static_cast<const __bf16*>(v);
  auto op = static_cast<__bf16*>(o);
  if (qw == 64) {
    if (causal)
      hipLaunchKernelGGL((attn_fwd_kernel<64, true>), grid, block, 0, stream, qp, kp, vp, op, lse2, B, S, H, Hkv, G, scale2, n_tiles);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<64, false>), grid, block, 0, stream, qp, kp, vp, op, lse2, B, S, H, Hkv, G, scale2, n_tiles);
  } else {
    if (causal)
      hipLaunchKernelGGL((attn_fwd_kernel<32, true>), grid, block, 0, stream, qp, kp, vp, op, lse2, B, S, H, Hkv, G, scale2, n_tiles);
    else
      hipLaunchKernelGGL((attn_fwd_kernel<32, false>), grid, block, 0, stream, qp, kp, vp, op, lse2, B, S, H, Hkv, G, scale2, n_tiles);
  }
  return hipGetLastError();
}

}  // namespace mm1
