// QK-RMSNorm + RoPE between the fused QKV projection and the attention kernel
// (the sublayer prologue of CODE/mimans/model/attention_tilelang.py:483-487),
// forward and backward, for gfx950.
//
// Input: the fused projection qkv [B, S, (H + 2*Hkv) * 128] bf16 (columns: H
// query heads, Hkv key heads, Hkv value heads).  Forward, per query / key head
// row of 128 (AT:423-428, :458-461):
//   y   = bf16( x * rsqrt(mean(x^2) + eps) * w )        fp32 math, w fp32 [128]
//   out = bf16( bf16(y * c) + bf16(rotate_half(y) * s) )
// with c = bf16(cos[pos]), s = bf16(sin[pos]) from fp32 tables [rot_len, 128]
// whose halves repeat (cat(angles, angles), AT:442-444), rotate_half(y) =
// cat(-y[64:], y[:64]).  The bf16 roundings are the reference's: the norm casts
// back to the input dtype and the rotation runs in bf16 tensor arithmetic.
// Value rows are copied into a contiguous V.  Without QK-norm (w == nullptr)
// y = x.
//
// Work decomposition: one wave per token; a row of 128 is one 16-lane group,
// 8 elements per lane (one 16-byte load), and the four groups of the wave
// take the token's rows in turn, so the tables and weights are loaded once per
// token.  The rotation partner of element d (d +- 64) sits in lane ^ 8 of the
// same group.  The backward accumulates the norm-weight gradients per lane,
// sums them over the workgroup's row groups in LDS and writes one partial per
// workgroup; qknorm_dw_reduce_kernel adds the partials in a fixed order, so
// the result is deterministic.
#include "mm1_common.h"

namespace mm1 {

__device__ __forceinline__ float bf16r(float x) { return (float)(__bf16)x; }

// sum over the 16 lanes of a row group
__device__ __forceinline__ float group16_sum(float v) {
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 1);
  return v;
}

struct QkvGeometry {
  int H, Hkv, S, rows_per_token;   // rows_per_token = H + 2 * Hkv
  long n_tokens;
};

// One wave per token: its four 16-lane groups take rows g, g+4, g+8, ... of
// the token, so a lane's cos / sin / weight values (8 columns at one
// position) are loaded once and serve every row.
__global__ __launch_bounds__(256) void qknorm_rope_fwd_kernel(
    const __bf16* __restrict__ qkv, const float* __restrict__ wq, const float* __restrict__ wk,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    __bf16* __restrict__ q, __bf16* __restrict__ k, __bf16* __restrict__ v,
    QkvGeometry geo, float eps) {
  const int l16 = threadIdx.x & 15, grp = (threadIdx.x >> 4) & 3;
  const long t = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= geo.n_tokens) return;   // whole waves leave together
  const int pos = (int)(t % geo.S);
  float c[8], sn[8], wqv[8], wkv[8];
  {
    const f32x4* cr = reinterpret_cast<const f32x4*>(cos_t + (long)pos * HD + 8 * l16);
    const f32x4* sr = reinterpret_cast<const f32x4*>(sin_t + (long)pos * HD + 8 * l16);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const f32x4 a = cr[h2], b = sr[h2];
#pragma unroll
      for (int j = 0; j < 4; ++j) { c[4 * h2 + j] = bf16r(a[j]); sn[4 * h2 + j] = bf16r(b[j]); }
    }
    if (wq) {
#pragma unroll
      for (int j = 0; j < 8; ++j) { wqv[j] = wq[8 * l16 + j]; wkv[j] = wk[8 * l16 + j]; }
    }
  }
  const __bf16* src = qkv + t * geo.rows_per_token * HD + 8 * l16;
  for (int r = grp; r < geo.rows_per_token; r += 4) {
    const bf16x8 xin = *reinterpret_cast<const bf16x8*>(src + r * HD);
    if (r >= geo.H + geo.Hkv) {   // value head: copy
      *reinterpret_cast<bf16x8*>(v + (t * geo.Hkv + (r - geo.H - geo.Hkv)) * HD + 8 * l16) = xin;
      continue;
    }
    const bool is_q = r < geo.H;
    float y[8];
    if (wq) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf((float)xin[j], (float)xin[j], ss);
      const float rs = rsqrtf(group16_sum(ss) * (1.f / HD) + eps);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = bf16r((float)xin[j] * rs * (is_q ? wqv[j] : wkv[j]));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (float)xin[j];
    }
    bf16x8 out;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float partner = __shfl_xor(y[j], 8);            // element d +- 64
      const float rot = l16 < 8 ? -partner : partner;       // rotate_half
      out[j] = (__bf16)(bf16r(y[j] * c[j]) + bf16r(rot * sn[j]));
    }
    __bf16* dst = is_q ? q + (t * geo.H + r) * HD : k + (t * geo.Hkv + (r - geo.H)) * HD;
    *reinterpret_cast<bf16x8*>(dst + 8 * l16) = out;
  }
}

// Backward.  Per query / key row, with xn = x * rs (fp32):
//   g1 = bf16(dout * c), g2 = bf16(dout * s)
//   dy = bf16(g1 + rotate_half^T(g2)),  rotate_half^T(g)[d] = g[d+64] (d < 64), -g[d-64]
//   dw += dy * xn;  dxn = dy * w
//   dx = rs * dxn - x * rs^3 * mean(dxn * x)                  (rounded to bf16)
// Value rows copy dV.  Waves stride over the tokens (one token per wave at a
// time, as in the forward); dw partials go to dw_part[blockIdx.x][2][128]
// (query weight, key weight).
__global__ __launch_bounds__(256) void qknorm_rope_bwd_kernel(
    const __bf16* __restrict__ qkv, const float* __restrict__ wq, const float* __restrict__ wk,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    const __bf16* __restrict__ dq, const __bf16* __restrict__ dk, const __bf16* __restrict__ dv,
    __bf16* __restrict__ dqkv, float* __restrict__ dw_part, QkvGeometry geo, float eps) {
  __shared__ float red[16][2][HD];
  const int l16 = threadIdx.x & 15, slot = threadIdx.x >> 4, grp = slot & 3;
  const bool norm = wq != nullptr;
  float dwq[8], dwk[8], wqv[8], wkv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    dwq[j] = 0.f;
    dwk[j] = 0.f;
    wqv[j] = norm ? wq[8 * l16 + j] : 0.f;
    wkv[j] = norm ? wk[8 * l16 + j] : 0.f;
  }

  for (long t = (long)blockIdx.x * 4 + (threadIdx.x >> 6); t < geo.n_tokens; t += (long)gridDim.x * 4) {
    const int pos = (int)(t % geo.S);
    float c[8], sn[8];
    {
      const f32x4* cr = reinterpret_cast<const f32x4*>(cos_t + (long)pos * HD + 8 * l16);
      const f32x4* sr = reinterpret_cast<const f32x4*>(sin_t + (long)pos * HD + 8 * l16);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const f32x4 a = cr[h2], b = sr[h2];
#pragma unroll
        for (int j = 0; j < 4; ++j) { c[4 * h2 + j] = bf16r(a[j]); sn[4 * h2 + j] = bf16r(b[j]); }
      }
    }
    const long row0 = t * geo.rows_per_token;
    for (int r = grp; r < geo.rows_per_token; r += 4) {
      const long row = row0 + r;
      if (r >= geo.H + geo.Hkv) {   // value head: gradient passes through
        const bf16x8 g = *reinterpret_cast<const bf16x8*>(dv + (t * geo.Hkv + (r - geo.H - geo.Hkv)) * HD + 8 * l16);
        *reinterpret_cast<bf16x8*>(dqkv + row * HD + 8 * l16) = g;
        continue;
      }
      const bool is_q = r < geo.H;
      const bf16x8 gin = *reinterpret_cast<const bf16x8*>(
          (is_q ? dq + (t * geo.H + r) * HD : dk + (t * geo.Hkv + (r - geo.H)) * HD) + 8 * l16);
      float dy[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float g1 = bf16r((float)gin[j] * c[j]);
        const float g2 = bf16r((float)gin[j] * sn[j]);
        const float partner = __shfl_xor(g2, 8);
        dy[j] = bf16r(g1 + (l16 < 8 ? partner : -partner));
      }
      bf16x8 out;
      if (norm) {
        const bf16x8 xin = *reinterpret_cast<const bf16x8*>(qkv + row * HD + 8 * l16);
        float x[8], ss = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) { x[j] = (float)xin[j]; ss = fmaf(x[j], x[j], ss); }
        const float rs = rsqrtf(group16_sum(ss) * (1.f / HD) + eps);
        float dxn[8], dot = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float xn = x[j] * rs;
          if (is_q) dwq[j] = fmaf(dy[j], xn, dwq[j]);
          else dwk[j] = fmaf(dy[j], xn, dwk[j]);
          dxn[j] = dy[j] * (is_q ? wqv[j] : wkv[j]);
          dot = fmaf(dxn[j], x[j], dot);
        }
        const float c3 = rs * rs * rs * group16_sum(dot) * (1.f / HD);
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (__bf16)(rs * dxn[j] - x[j] * c3);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) out[j] = (__bf16)dy[j];
      }
      *reinterpret_cast<bf16x8*>(dqkv + row * HD + 8 * l16) = out;
    }
  }
  if (!norm) return;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    red[slot][0][8 * l16 + j] = dwq[j];
    red[slot][1][8 * l16 + j] = dwk[j];
  }
  __syncthreads();
  const int which = threadIdx.x >> 7, d = threadIdx.x & 127;   // 256 threads = 2 x 128 sums
  float s = 0.f;
  for (int i = 0; i < 16; ++i) s += red[i][which][d];
  dw_part[((long)blockIdx.x * 2 + which) * HD + d] = s;
}

// dwq, dwk = sums of the per-workgroup partials: one workgroup per output
// value (2 x 128), each thread adds a fixed stride of partials, then a fixed
// LDS tree -- the summation order never changes, so the result is
// deterministic.
__global__ __launch_bounds__(256) void qknorm_dw_reduce_kernel(const float* __restrict__ dw_part, int n_part,
                                                               float* __restrict__ dwq, float* __restrict__ dwk) {
  __shared__ float acc[256];
  const int which = blockIdx.x >> 7, d = blockIdx.x & 127;
  float s = 0.f;
  for (int i = threadIdx.x; i < n_part; i += 256) s += dw_part[((long)i * 2 + which) * HD + d];
  acc[threadIdx.x] = s;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) acc[threadIdx.x] += acc[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) (which ? dwk : dwq)[d] = acc[0];
}

constexpr int kQkNormBwdBlocks = 1024;

size_t qknorm_bwd_workspace_bytes() { return (size_t)kQkNormBwdBlocks * 2 * HD * sizeof(float); }

hipError_t launch_qknorm_fwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                             const float* sin_t, void* q, void* k, void* v, int B, int S, int H, int Hkv,
                             float eps, hipStream_t stream) {
  QkvGeometry geo{H, Hkv, S, H + 2 * Hkv, (long)B * S};
  const long blocks = (geo.n_tokens + 3) / 4;
  hipLaunchKernelGGL(qknorm_rope_fwd_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const __bf16*>(qkv), wq, wk, cos_t, sin_t, static_cast<__bf16*>(q),
                     static_cast<__bf16*>(k), static_cast<__bf16*>(v), geo, eps);
  return hipGetLastError();
}

hipError_t launch_qknorm_bwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                             const float* sin_t, const void* dq, const void* dk, const void* dv,
                             void* dqkv, float* dwq, float* dwk, void* workspace, int B, int S, int H,
                             int Hkv, float eps, hipStream_t stream) {
  QkvGeometry geo{H, Hkv, S, H + 2 * Hkv, (long)B * S};
  const long need = (geo.n_tokens + 3) / 4;
  const int blocks = (int)(need < kQkNormBwdBlocks ? need : kQkNormBwdBlocks);
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(qknorm_rope_bwd_kernel, dim3(blocks), dim3(256), 0, stream,
                     static_cast<const __bf16*>(qkv), wq, wk, cos_t, sin_t, static_cast<const __bf16*>(dq),
                     static_cast<const __bf16*>(dk), static_cast<const __bf16*>(dv),
                     static_cast<__bf16*>(dqkv), part, geo, eps);
  if (wq) hipLaunchKernelGGL(qknorm_dw_reduce_kernel, dim3(2 * HD), dim3(256), 0, stream, part, blocks, dwq, dwk);
  return hipGetLastError();
}

}  // namespace mm1
