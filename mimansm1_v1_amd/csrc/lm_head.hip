// Fused cross-entropy head for gfx950: log-sum-exp over the vocabulary
// without materialising the [tokens, vocab] logits, and the logits gradient
// one vocabulary chunk at a time.
//
// Reference: CODE/mimans/model/lm_head_tilelang.py
//   logsumexp_kernel        :92-156   Lse[t] = log sum_v exp(H[t] . W[:, v]), online max/sum
//                                     over vocab tiles, fp32 accumulation of bf16 products
//   gather_target_logits    :186-190  the target's logit in fp32
//   FusedCrossEntropy       :193-243  loss = sum_valid (lse - target_logit) / count;
//                                     d_logits = (softmax - onehot) * mask * grad / count
// Layouts: hidden [T, d] bf16, weight [d, V] bf16 (the reference's
// [d_model, vocab] matrix), targets [T] int64 (ignore_index or 0 <= t < V).
//
// Decomposition.  The logits are tiles of the persistent GEMM of gemm_tn.h in
// its single-matrix layout (256 tokens x 256 vocabulary entries per
// workgroup, 64 entries per wave); the D tiles give a lane one token and 32
// of its wave's 64 entries, so per-token reductions are in-lane plus one
// exchange with lane ^ 32.
//   lm_lse_partial_kernel : per (token, 64-entry vocabulary block) the max m
//                           and sum_v exp(l_v - m), and the target's logit from
//                           the block that holds it;
//   lm_lse_combine_kernel : per token, the fixed-order combination of its
//                           partials into lse (natural log) and the token loss;
//   lm_dlogits_kernel     : bf16 d_logits of one vocabulary chunk,
//                           (exp(l - lse) - [v == target]) * mask * scale.
// Everything is deterministic (no atomics, fixed reduction orders).
#include <hip/hip_runtime.h>
#include <math.h>

#include "gemm_tn.h"

namespace mm1 {

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float shfl_xor32(float v) { return __shfl_xor(v, 32); }

}  // namespace

// Partials: part[t][blk] = (max, sum of exp(l - max)) over vocabulary block blk
// (64 entries, blk = 4 * column block + wave column), (-inf, 0) for a block
// beyond the vocabulary.  tlogit[t] = the logit of column targets[t], or of
// column 0 when the target is negative (ignore_index) or >= V, as the
// reference's gather over targets.clamp(min=0); written by the one lane that
// holds that column.
__global__ __launch_bounds__(512, 1) void lm_lse_partial_kernel(
    const __bf16* __restrict__ h, const __bf16* __restrict__ w, const long long* __restrict__ targets,
    float2* __restrict__ part, float* __restrict__ tlogit, int T, int d, int V, int n_mblk, int n_nblk) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv & 1, wn = wv >> 1, hh = lane >> 5;
  const gemm::Problem p{h, w, w, T, d, V, V, n_mblk, n_nblk};
  const int n_part = 4 * n_nblk;
  gemm::run<false>(p, smem, [](int, int) {}, [&](int mb, int nb, f32x16 (&acc)[2][4]) {
    const int v0 = nb * 256 + 64 * wn;             // this wave's 64 vocabulary entries
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = mb * gemm::BM + 128 * wm + 32 * i + (lane & 31);
      float m = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int v = v0 + 32 * b + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (v < V) m = fmaxf(m, acc[b][i][r]);
        }
      }
      m = fmaxf(m, shfl_xor32(m));
      float s = 0.f;
      if (m > -INFINITY) {
        const float ms = m * kLog2e;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int v = v0 + 32 * b + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (v < V) s += exp2_fast(acc[b][i][r] * kLog2e - ms);
          }
        }
      }
      s += shfl_xor32(s);
      if (tok < T) {
        if (hh == 0) part[(long)tok * n_part + 4 * nb + wn] = make_float2(m, s);
        if (targets != nullptr) {
          long long tv = targets[tok];
          if (tv < 0 || tv >= V) tv = 0;     // the reference gathers column clamp(t, min=0)
          if (tv >= v0 && tv < v0 + 64) {
            const int rel = (int)(tv - v0);
            const int b = rel >> 5, rr = rel & 31;       // block, row inside the D tile
            if (((rr >> 2) & 1) == hh) {
              const int reg = 4 * (rr >> 3) + (rr & 3);
              float val = 0.f;
#pragma unroll
              for (int bb = 0; bb < 2; ++bb) {
#pragma unroll
                for (int q = 0; q < 16; ++q)
                  if (bb == b && q == reg) val = acc[bb][i][q];
              }
              tlogit[tok] = val;
            }
          }
        }
      }
    }
  });
}

// One wave per token: lse = m* + ln(sum_j s_j exp(m_j - m*)) over the token's
// partials, in one pass: each lane folds partials lane, lane + 64, ... into a
// running (max, sum) in index order, then the lanes' pairs merge by a fixed
// shuffle tree (deterministic); the token loss is lse - target_logit (0 for
// ignored or out-of-range targets).
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;                    // both empty
  s = s * exp2_fast((m - mn) * kLog2e) + s2 * exp2_fast((m2 - mn) * kLog2e);
  m = mn;
}

__global__ __launch_bounds__(256) void lm_lse_combine_kernel(
    const float2* __restrict__ part, const float* __restrict__ tlogit, const long long* __restrict__ targets,
    float* __restrict__ lse, float* __restrict__ loss, int T, int V, int n_part, long long ignore_index) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= T) return;
  const float2* row = part + (long)tok * n_part;
  float m = -INFINITY, s = 0.f;
  int j = lane;
  for (; j + 192 < n_part; j += 256) {            // four loads in flight per lane
    float2 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = row[j + 64 * u];
#pragma unroll
    for (int u = 0; u < 4; ++u) lse_merge(m, s, v[u].x, v[u].y);
  }
  for (; j < n_part; j += 64) {
    const float2 v = row[j];
    lse_merge(m, s, v.x, v.y);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float m2 = __shfl_xor(m, o), s2 = __shfl_xor(s, o);
    lse_merge(m, s, m2, s2);
  }
  if (lane == 0) {
    const float l = m + log2f(s) * kLn2;
    lse[tok] = l;
    if (loss != nullptr) {
      const long long tv = targets[tok];
      loss[tok] = (tv != ignore_index && tv >= 0 && tv < V) ? l - tlogit[tok] : 0.f;
    }
  }
}

// d_logits of vocabulary entries [v0, v0 + vn): the GEMM runs over the
// columns of weight + v0; out[t][v] (row stride ld) = bf16((exp(l - lse[t]) -
// [v0 + v == target[t]]) * scale) for valid targets, 0 for ignored ones.
// `scale` is a device scalar (the loss gradient over the valid count).
__global__ __launch_bounds__(512, 1) void lm_dlogits_kernel(
    const __bf16* __restrict__ h, const __bf16* __restrict__ w, const long long* __restrict__ targets,
    const float* __restrict__ lse, const float* __restrict__ scale, __bf16* __restrict__ out, long ld,
    int T, int d, int V, int v0, int vn, long long ignore_index, int n_mblk, int n_nblk) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = wv & 1, wn = wv >> 1;
  const gemm::Problem p{h, w + v0, w + v0, T, d, V, vn, n_mblk, n_nblk};
  const float sc = *scale;
  // the rows go out through 4 KiB per wave above the GEMM's ring
  char* stage = smem + gemm::LDS_BYTES + gemm::STAGE_BYTES * wv;
  // Targets and lse of the tile's tokens, loaded at its first k step (the
  // loads land during the products, not in the epilogue).
  long long tv[4];
  float l2[4];
  auto pro = [&](int mb, int) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = min(mb * gemm::BM + 128 * wm + 32 * i + (lane & 31), T - 1);
      tv[i] = targets[tok];
      l2[i] = lse[tok] * kLog2e;
    }
  };
  gemm::run<false>(p, smem, pro, [&](int mb, int nb, f32x16 (&acc)[2][4]) {
    const int c0 = nb * 256 + 64 * wn;             // this wave's first column of the chunk
    const long tok0 = (long)mb * gemm::BM + 128 * wm;
    auto val = [&](int i, int b, int q) {
      const long long t = tv[i];
      const bool valid = t != ignore_index && t >= 0 && t < V;
      const float coef = valid ? sc : 0.f;
      const long long tcol = t - v0;               // the target's column in this chunk
      const int c = c0 + 32 * b + 8 * q + 4 * (lane >> 5);
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pr = exp2_fast(acc[b][i][4 * q + e] * kLog2e - l2[i]);
        if (c + e == tcol) pr -= 1.f;
        o[e] = (__bf16)(pr * coef);
      }
      return o;
    };
    gemm::store_rows128(
        stage, lane, val,
        [&](int r) -> __bf16* { return tok0 + r < T ? out + (tok0 + r) * ld + c0 : nullptr; },
        [&](int c) { return c0 + 8 * c < vn; });
  });
}

static hipError_t gemm_geometry(int T, int cols, int& n_mblk, int& n_nblk, int& grid) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  n_mblk = (T + gemm::BM - 1) / gemm::BM;
  n_nblk = (cols + 255) / 256;
  grid = gemm::persistent_grid(cus, n_mblk * n_nblk);
  return hipSuccess;
}

size_t lm_head_workspace_bytes(int T, int V) {
  const long n_part = 4L * ((V + 255) / 256);
  return (size_t)T * n_part * sizeof(float2) + (size_t)T * sizeof(float) + 256;
}

hipError_t launch_lm_lse(const void* hidden, const void* weight, const long long* targets, long long ignore_index,
                         float* lse, float* tlogit_out, float* loss, void* workspace, int T, int d, int V,
                         hipStream_t stream) {
  int n_mblk, n_nblk, grid;
  hipError_t e = gemm_geometry(T, V, n_mblk, n_nblk, grid);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(lm_lse_partial_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)gemm::LDS_BYTES);
  if (e != hipSuccess) return e;
  const int n_part = 4 * n_nblk;
  auto part = static_cast<float2*>(workspace);
  float* tl = tlogit_out != nullptr
                  ? tlogit_out
                  : reinterpret_cast<float*>(static_cast<char*>(workspace) + (size_t)T * n_part * sizeof(float2));
  hipLaunchKernelGGL(lm_lse_partial_kernel, dim3(grid), dim3(512), gemm::LDS_BYTES, stream,
                     static_cast<const __bf16*>(hidden), static_cast<const __bf16*>(weight), targets, part, tl,
                     T, d, V, n_mblk, n_nblk);
  hipLaunchKernelGGL(lm_lse_combine_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, part, tl, targets, lse,
                     targets != nullptr ? loss : nullptr, T, V, n_part, ignore_index);
  return hipGetLastError();
}

hipError_t launch_lm_dlogits(const void* hidden, const void* weight, const long long* targets,
                             long long ignore_index, const float* lse, const float* scale, void* dlogits, long ld,
                             int T, int d, int V, int v0, int vn, hipStream_t stream) {
  int n_mblk, n_nblk, grid;
  hipError_t e = gemm_geometry(T, vn, n_mblk, n_nblk, grid);
  if (e != hipSuccess) return e;
  const size_t lds = gemm::LDS_BYTES + 8 * gemm::STAGE_BYTES;   // ring + the epilogue's staging
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(lm_dlogits_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(lm_dlogits_kernel, dim3(grid), dim3(512), lds, stream,
                     static_cast<const __bf16*>(hidden), static_cast<const __bf16*>(weight), targets, lse, scale,
                     static_cast<__bf16*>(dlogits), ld, T, d, V, v0, vn, ignore_index, n_mblk, n_nblk);
  return hipGetLastError();
}

}  // namespace mm1
