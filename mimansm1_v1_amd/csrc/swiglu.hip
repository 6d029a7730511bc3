// SwiGLU feed-forward kernels for gfx950: the gate/up projection with the
// SiLU * up epilogue fused into the GEMM, and the elementwise SwiGLU gradient.
//
// Reference: CODE/mimans/model/swiglu_tilelang.py
//   gate_up_swiglu  :119-156  Act  = bf16(silu(X Wg) * (X Wu)), fp32 accumulate and epilogue
//   gate_up_split   :158-200  Gate = bf16(X Wg), Up = bf16(X Wu)
//   FusedSwiGLU     :278-301  act  = F.silu(Gate) * Up in bf16 tensor ops (:284)
//   swiglu_grad     :202-240  dGate = bf16(dA u s (1 + g (1 - s))), dUp = bf16(dA g s),
//                             s = sigmoid(g), inputs bf16 read into fp32
// Layouts (row-major, contiguous rows): X [T, d] bf16, Wg / Wu [d, F] bf16
// (the reference's [d_model, ffn] parameters), outputs [T, F] bf16.
//
// GEMM: the persistent core of gemm_tn.h in its PAIRED layout (each LDS
// weight row holds 64 gate and the same 64 up columns), so a wave's
// accumulator blocks 0, 1 (gate) and 2, 3 (up) hold the gate and up values of
// the same (token, column) pairs and the epilogue is elementwise in registers.
// A workgroup tile is 256 tokens x 128 columns of both Gate and Up.
#include <hip/hip_runtime.h>

#include "gemm_tn.h"

namespace mm1 {

namespace {

__device__ __forceinline__ float bf16r(float x) { return (float)(__bf16)x; }

// sigmoid(g) = 1 / (1 + 2^(-g log2 e)) with the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32: about 1 ulp each in fp32, far below the bf16
// rounding that follows; an IEEE division would cost ten instructions per
// element in the epilogue).  For g -> -inf, 2^(...) -> inf and the
// reciprocal gives 0, so silu(g) -> -0, as the reference's g / (1 + exp(-g)).
__device__ __forceinline__ float sigmoidf_(float g) {
  return __builtin_amdgcn_rcpf(1.f + exp2_fast(-g * 1.4426950408889634f));
}

}  // namespace

// ACT: 0 = no activation output, 1 = act = bf16(silu(g) * u) on the fp32
// accumulators (gate_up_swiglu), 2 = act = bf16(bf16(silu(bf16(g))) * bf16(u)),
// the rounding of F.silu(Gate) * Up on bf16 tensors (FusedSwiGLU.forward).
// SPLIT: also store Gate and Up (rounded to bf16).
template <int ACT>
__device__ __forceinline__ bf16x4 act_quad(const f32x16& g, const f32x16& u, int q) {
  bf16x4 av;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float gf = g[4 * q + e], uf = u[4 * q + e];
    if (ACT == 1) {
      av[e] = (__bf16)(gf * sigmoidf_(gf) * uf);
    } else {
      const float gb = bf16r(gf);
      av[e] = (__bf16)(bf16r(gb * sigmoidf_(gb)) * bf16r(uf));
    }
  }
  return av;
}

__device__ __forceinline__ bf16x4 round_quad(const f32x16& a, int q) {
  bf16x4 v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (__bf16)a[4 * q + e];
  return v;
}

template <bool SPLIT, int ACT>
__global__ __launch_bounds__(512, 1) void swiglu_gate_up_kernel(
    const __bf16* __restrict__ x, const __bf16* __restrict__ wg, const __bf16* __restrict__ wu,
    __bf16* __restrict__ gate, __bf16* __restrict__ up, __bf16* __restrict__ act,
    int T, int d, int F, int n_mblk, int n_nblk) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w & 1, wn = w >> 1;
  const gemm::Problem p{x, wg, wu, T, d, F, F, n_mblk, n_nblk};
  // the outputs go out through 4 KiB per wave above the GEMM's ring
  char* stage = smem + gemm::LDS_BYTES + gemm::STAGE_BYTES * w;
  // Epilogue of a tile: acc[0][i] / acc[1][i] give lane the token
  // m0 + 128wm + 32i + (lane & 31) and, in registers 4q .. 4q+3, the columns
  // n0 + 32wn + 8q + 4(lane/32) + 0..3 of Gate / Up (n0 = 128 nb, wn = 0..3).
  gemm::run<true>(p, smem, [](int, int) {}, [&](int mb, int nb, f32x16 (&acc)[2][4]) {
    const long tok0 = (long)mb * gemm::BM + 128 * wm;
    const int col0 = nb * 128 + 32 * wn;
    auto rows = [&](__bf16* out) {
      return [=](int r) -> __bf16* { return tok0 + r < T ? out + (tok0 + r) * F + col0 : nullptr; };
    };
    if (SPLIT) {
      gemm::store_rows64(stage, lane, [&](int i, int q) { return round_quad(acc[0][i], q); }, rows(gate));
      gemm::store_rows64(stage, lane, [&](int i, int q) { return round_quad(acc[1][i], q); }, rows(up));
    }
    if (ACT != 0)
      gemm::store_rows64(stage, lane, [&](int i, int q) { return act_quad<ACT>(acc[0][i], acc[1][i], q); },
                         rows(act));
  });
}

// dGate, dUp from dAct, Gate, Up (all bf16 [T, F], rows of F elements; the
// outputs have row stride ld_out, so both can land in one [T, 2F] buffer).
// Eight columns per thread.
__global__ __launch_bounds__(256) void swiglu_grad_kernel(
    const __bf16* __restrict__ dact, const __bf16* __restrict__ gate, const __bf16* __restrict__ up,
    __bf16* __restrict__ dgate, __bf16* __restrict__ dup, long n8, int F8, long ld_out) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (long)gridDim.x * blockDim.x) {
    const long row = i / F8, c8 = i - row * F8;
    const long in = row * F8 * 8 + c8 * 8;
    const bf16x8 da = *reinterpret_cast<const bf16x8*>(dact + in);
    const bf16x8 gv = *reinterpret_cast<const bf16x8*>(gate + in);
    const bf16x8 uv = *reinterpret_cast<const bf16x8*>(up + in);
    bf16x8 og, ou;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = (float)da[j], g = (float)gv[j], u = (float)uv[j];
      const float s = sigmoidf_(g);
      og[j] = (__bf16)(a * u * s * (1.f + g * (1.f - s)));
      ou[j] = (__bf16)(a * g * s);
    }
    const long out = row * ld_out + c8 * 8;
    *reinterpret_cast<bf16x8*>(dgate + out) = og;
    *reinterpret_cast<bf16x8*>(dup + out) = ou;
  }
}

template <bool SPLIT, int ACT>
static hipError_t launch_gate_up_t(const __bf16* x, const __bf16* wg, const __bf16* wu, __bf16* gate,
                                   __bf16* up, __bf16* act, int T, int d, int F, hipStream_t stream) {
  auto kern = swiglu_gate_up_kernel<SPLIT, ACT>;
  const size_t lds = gemm::LDS_BYTES + 8 * gemm::STAGE_BYTES;   // ring + the epilogue's staging
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  int dev = 0, cus = 0;
  e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int n_mblk = (T + gemm::BM - 1) / gemm::BM, n_nblk = F / 128;
  hipLaunchKernelGGL(kern, dim3(gemm::persistent_grid(cus, n_mblk * n_nblk)), dim3(512), lds,
                     stream, x, wg, wu, gate, up, act, T, d, F, n_mblk, n_nblk);
  return hipGetLastError();
}

// mode: 0 = act only, fp32 epilogue (gate_up_swiglu); 1 = gate and up only
// (gate_up_split); 2 = gate, up and act with bf16 rounding steps (FusedSwiGLU).
hipError_t launch_swiglu_gate_up(const void* x, const void* wg, const void* wu, void* gate, void* up,
                                 void* act, int T, int d, int F, int mode, hipStream_t stream) {
  auto xp = static_cast<const __bf16*>(x);
  auto gp = static_cast<const __bf16*>(wg);
  auto up_w = static_cast<const __bf16*>(wu);
  auto go = static_cast<__bf16*>(gate);
  auto uo = static_cast<__bf16*>(up);
  auto ao = static_cast<__bf16*>(act);
  switch (mode) {
    case 0: return launch_gate_up_t<false, 1>(xp, gp, up_w, go, uo, ao, T, d, F, stream);
    case 1: return launch_gate_up_t<true, 0>(xp, gp, up_w, go, uo, ao, T, d, F, stream);
    default: return launch_gate_up_t<true, 2>(xp, gp, up_w, go, uo, ao, T, d, F, stream);
  }
}

hipError_t launch_swiglu_grad(const void* dact, const void* gate, const void* up, void* dgate, void* dup,
                              int T, int F, long ld_out, hipStream_t stream) {
  const long n8 = (long)T * (F / 8);
  const long want = (n8 + 255) / 256;
  const int blocks = (int)(want < 8192 ? want : 8192);
  hipLaunchKernelGGL(swiglu_grad_kernel, dim3(blocks), dim3(256), 0, stream,
                     static_cast<const __bf16*>(dact), static_cast<const __bf16*>(gate),
                     static_cast<const __bf16*>(up), static_cast<__bf16*>(dgate), static_cast<__bf16*>(dup),
                     n8, F / 8, ld_out);
  return hipGetLastError();
}

}  // namespace mm1
