// Issue-rate probe of gfx950's matrix core: how many FLOP/s of
// v_mfma_f32_32x32x16_f16 the chip sustains when each product comes with a
// given mix of other instructions and no memory traffic.  It is the
// practical ceiling the attention kernels are measured against (the chip
// lowers its clock under dense MFMA load, and VALU / LDS instructions share
// the SIMD's issue with the products).  Not part of the attention library:
// built as its own small library and driven by bench.py --mfma-ceiling.
//
// Each wave runs four independent accumulator chains; every product is
// followed by the mode's other instructions, placed by scheduling barriers:
//   0  products only (register operands)
//   1  + 4 v_fma_f32
//   2  + 4 v_fma_f32 + 1 v_exp_f32
//   3  A operand from LDS (1 ds_read_b128 per product, read one trip ahead)
//   4  A from LDS (ds_read_b128) and B from LDS (2 ds_read_b64_tr_b16)
//   5  the dK/dV kernel's mix per product: 2 LDS reads (A by ds_read_b128,
//      B by a ds_read_b64_tr_b16 pair on every other product), 3 v_fma_f32,
//      an exp every other product
//   6  no products: 4 ds_read_b128 per trip (LDS read bandwidth)
//   7  no products: 8 ds_read_b64_tr_b16 per trip (transposed reads)
//   8  products only, one dependent chain per wave (each product
//      accumulates onto the previous one's result)
//   9  products only, two dependent chains per wave
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mm1probe {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
#define PROBE_LDS __attribute__((address_space(3)))

template <int MODE>
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(float* __restrict__ out, int iters, float s) {
  __shared__ __attribute__((aligned(16))) char lds[16384];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < 16384 / 4; i += 256) reinterpret_cast<float*>(lds)[i] = 1e-3f * (float)(i & 255);
  __syncthreads();
  // every wave reads the same LDS bytes (as the kernels' waves share a
  // tile): A fragments from the first 8 KiB, B from the second;
  // consecutive 16 (8) bytes per lane: no bank conflicts
  const char* a_base = lds + 16 * lane;
  const char* b_base = lds + 8192 + 8 * lane;
  f16x8 a, b;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    a[t] = (_Float16)(0.001f * (lane + t + w));
    b[t] = (_Float16)(0.002f * (lane - t));
  }
  f32x16 acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = f32x16{};
  float x[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) x[i] = s * (float)(lane + i);

  auto read_a = [&](int j, int o = 0) -> f16x8 {
    return *reinterpret_cast<const PROBE_LDS f16x8*>((const PROBE_LDS char*)a_base + 1024 * j + o);
  };
  auto read_b = [&](int j, int o = 0) -> f16x8 {
    f16x8 r;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (PROBE_LDS s16x4*)((const PROBE_LDS char*)b_base + 1024 * j + 512 * h + o));
      const f16x4 f = __builtin_bit_cast(f16x4, v);
#pragma unroll
      for (int t = 0; t < 4; ++t) r[4 * h + t] = f[t];
    }
    return r;
  };

  constexpr bool A_LDS = MODE >= 3 && MODE <= 5;   // A operand read from LDS each trip
  f16x8 fa[4], fb[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    fa[j] = A_LDS || MODE == 6 ? read_a(j) : a;
    fb[j] = (MODE == 4 || MODE == 7 || (MODE == 5 && (j & 1) == 0)) ? read_b(j) : b;
  }
  f16x8 ld[4] = {a, a, a, b};
  for (int it = 0; it < iters; ++it) {
    // modes 6, 7: the trip's offset keeps the reads in the loop; each value
    // is summed one trip after its read, so the reads do not wait
    const int o = (it & 1) * 4096;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (MODE == 6 || MODE == 7) {
        fa[j] += ld[j];
        ld[j] = MODE == 6 ? *reinterpret_cast<const volatile PROBE_LDS f16x8*>(
                                (const PROBE_LDS char*)a_base + 1024 * j + o)
                          : read_b(j, o >> 1);
        continue;
      }
      // modes 8, 9: one / two accumulators for the trip's four products
      constexpr int NACC = MODE == 8 ? 1 : MODE == 9 ? 2 : 4;
      acc[j % NACC] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[j], fb[j], acc[j % NACC], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (A_LDS) {
        fa[j] = read_a(j);   // for the next trip
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      if (MODE == 4 || (MODE == 5 && (j & 1) == 0)) {
        fb[j] = read_b(j);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      constexpr int NF = MODE == 1 || MODE == 2 ? 4 : MODE == 5 ? 3 : 0;
#pragma unroll
      for (int v = 0; v < NF; ++v) x[(3 * j + v) % 12] = fmaf(x[(3 * j + v) % 12], s, 0.5f);
      if (NF) __builtin_amdgcn_sched_group_barrier(0x002, NF, 0);
      if (MODE == 2 || (MODE == 5 && (j & 1) == 1)) {
        x[(5 * j) % 12] = __builtin_amdgcn_exp2f(x[(5 * j) % 12]);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
      }
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sum += acc[j][r];
  }
#pragma unroll
  for (int i = 0; i < 12; ++i) sum += x[i];
#pragma unroll
  for (int j = 0; j < 4; ++j) sum += (float)fa[j][0] + (float)fb[j][7] + (float)ld[j][3];
  out[blockIdx.x * 256 + tid] = sum;
}

}  // namespace mm1probe

// Launch `blocks` workgroups of 4 waves running `iters` trips of 4 products
// each; out holds blocks * 256 floats.  Returns a hipError_t.
extern "C" int mm1_probe_mfma_ceiling(int mode, float* out, int blocks, int iters, hipStream_t stream) {
  using namespace mm1probe;
  const dim3 g(blocks), t(256);
  switch (mode) {
    case 0: hipLaunchKernelGGL(mfma_ceiling_kernel<0>, g, t, 0, stream, out, iters, 0.999f); break;
    case 1: hipLaunchKernelGGL(mfma_ceiling_kernel<1>, g, t, 0, stream, out, iters, 0.999f); break;
    case 2: hipLaunchKernelGGL(mfma_ceiling_kernel<2>, g, t, 0, stream, out, iters, 0.999f); break;
    case 3: hipLaunchKernelGGL(mfma_ceiling_kernel<3>, g, t, 0, stream, out, iters, 0.999f); break;
    case 4: hipLaunchKernelGGL(mfma_ceiling_kernel<4>, g, t, 0, stream, out, iters, 0.999f); break;
    case 5: hipLaunchKernelGGL(mfma_ceiling_kernel<5>, g, t, 0, stream, out, iters, 0.999f); break;
    case 6: hipLaunchKernelGGL(mfma_ceiling_kernel<6>, g, t, 0, stream, out, iters, 0.999f); break;
    case 7: hipLaunchKernelGGL(mfma_ceiling_kernel<7>, g, t, 0, stream, out, iters, 0.999f); break;
    case 8: hipLaunchKernelGGL(mfma_ceiling_kernel<8>, g, t, 0, stream, out, iters, 0.999f); break;
    case 9: hipLaunchKernelGGL(mfma_ceiling_kernel<9>, g, t, 0, stream, out, iters, 0.999f); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}
