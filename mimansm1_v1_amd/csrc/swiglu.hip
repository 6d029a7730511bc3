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
// GEMM decomposition.  The product is computed transposed, D = W^T X^T
// (rows = output columns n, columns = tokens), so that a lane of an MFMA
// result holds four consecutive columns of one token and the epilogue stores
// 8 bytes at a time.  A workgroup (4 waves, one per SIMD) owns 256 tokens x
// 128 columns of both Gate and Up, in k steps of 64 staged in a two-slot LDS
// ring by the LDS DMA:
//   * X: two 64 x 256 B tiles; row r of tile t holds tokens 128t + r (left
//     half) and 128t + 64 + r (right half), 64 k values each;
//   * W: two 64 x 256 B tiles; row k of tile t holds Wg[k][64t .. 64t+63] then
//     Wu[k][64t .. 64t+63].
// Wave (wm, wn) accumulates tokens 128wm .. +127 against tile wn's 64 gate and
// the same 64 up columns (16 accumulator tiles, in AGPRs), so every lane holds
// the gate and up values of the same (token, column) pairs and the epilogue is
// elementwise in registers.  W^T is read with the LDS transpose read in
// natural k order, X with row reads; both are conflict-free on the swizzled
// tile layout.  64 KiB of operands per 64 MFMAs per wave keeps the per-CU load
// rate at half of what the matrix cores would need with 128 x 128 tiles.
#include <hip/hip_runtime.h>

#include "mm1_common.h"

namespace mm1 {

namespace {

constexpr int SG_BM = 256;          // tokens per workgroup
constexpr int SG_BN = 128;          // gate (and up) columns per workgroup
constexpr int SG_BK = 64;           // k per ring slot
constexpr int SG_SLOT = 4 * TILE_BYTES;   // X tiles 0, 1; W tiles 0, 1
constexpr int SG_NSTAGE = 2;

// Per-lane byte offsets of the transposed (natural k order) reads of column
// block blk (32 columns) of a k-major weight tile, halves r = 0, 1 (k rows
// 16ks + 8h + 4r + j/4 for lane group h; adding 16ks leaves swz(row) unchanged).
struct TrNat {
  int off[2];
};

__device__ __forceinline__ TrNat make_tr_nat(int lane, int blk) {
  TrNat t;
  const int h = lane >> 5, g = (lane >> 4) & 1, j = lane & 15, jj = j >> 2;
  const int chunk = 4 * blk + 2 * g + ((j & 3) >> 1), half = j & 1;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int row = 8 * h + 4 * r + jj;
    t.off[r] = row * 256 + ((chunk ^ swz(row)) << 4) + 8 * half;
  }
  return t;
}

// B operand (16 k x 32 columns) from a k-major weight tile: the column block
// of `t`, k step kk (tile rows 16kk .. +15); lane holds k = 16kk + 8(lane/32) + 0..7.
__device__ __forceinline__ bf16x8 tr_nat(const char* tile, const TrNat& t, int kk) {
  bf16x8 out;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const bf16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (MM1_LDS bf16x4*)(tile + 4096 * kk + t.off[r]));
#pragma unroll
    for (int q = 0; q < 4; ++q) out[4 * r + q] = v[q];
  }
  return out;
}

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

// Tile order.  Tiles (128 tokens x 64 columns) are numbered in groups of
// SG_GROUP token blocks: consecutive tiles walk down SG_GROUP token blocks,
// then move one column block right.  The grid is persistent (one workgroup
// per CU); workgroups are dealt round-robin to the 8 XCDs, and XCD x works
// through the x-th eighth of the tile sequence with its workgroups taking
// consecutive tiles, so at any time an XCD's 32 CUs hold a block of about 8 x 4
// tiles whose X rows and weight columns are shared in that XCD's L2.
constexpr int SG_GROUP = 8;

__device__ __forceinline__ void tile_coords(int t, int n_mblk, int n_nblk, int& mb, int& nb) {
  const int per_group = SG_GROUP * n_nblk;
  const int group = t / per_group, first = group * SG_GROUP;
  const int gm = min(SG_GROUP, n_mblk - first);
  const int local = t - group * per_group;
  mb = first + local % gm;
  nb = local / gm;
}

// ACT: 0 = no activation output, 1 = act = bf16(silu(g) * u) on the fp32
// accumulators (gate_up_swiglu), 2 = act = bf16(bf16(silu(bf16(g))) * bf16(u)),
// the rounding of F.silu(Gate) * Up on bf16 tensors (FusedSwiGLU.forward).
// SPLIT: also store Gate and Up (rounded to bf16).
template <bool SPLIT, int ACT>
__device__ __forceinline__ void store_quad(const f32x16& g, const f32x16& u, int q, long o,
                                           __bf16* __restrict__ gate, __bf16* __restrict__ up,
                                           __bf16* __restrict__ act) {
  bf16x4 gv, uv, av;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float gf = g[4 * q + e], uf = u[4 * q + e];
    gv[e] = (__bf16)gf;
    uv[e] = (__bf16)uf;
    if (ACT == 1) {
      av[e] = (__bf16)(gf * sigmoidf_(gf) * uf);
    } else if (ACT == 2) {
      const float gb = (float)gv[e];
      av[e] = (__bf16)(bf16r(gb * sigmoidf_(gb)) * (float)uv[e]);
    }
  }
  if (SPLIT) {
    *reinterpret_cast<bf16x4*>(gate + o) = gv;
    *reinterpret_cast<bf16x4*>(up + o) = uv;
  }
  if (ACT != 0) *reinterpret_cast<bf16x4*>(act + o) = av;
}

template <bool SPLIT, int ACT>
__global__ __launch_bounds__(256, 1) void swiglu_gate_up_kernel(
    const __bf16* __restrict__ x, const __bf16* __restrict__ wg, const __bf16* __restrict__ wu,
    __bf16* __restrict__ gate, __bf16* __restrict__ up, __bf16* __restrict__ act,
    int T, int d, int F, int n_mblk, int n_nblk) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1;
  const int wu_ = __builtin_amdgcn_readfirstlane(w);

  // This workgroup's tiles: XCD x = blockIdx % 8 owns tiles [t0, t1) of the
  // sequence; its workgroups (index blockIdx / 8 among the XCD's n_wg) take
  // every n_wg-th tile of it.
  const int total = n_mblk * n_nblk;
  const int xcd = blockIdx.x & 7, n_wg = gridDim.x >> 3;
  const int t0 = (int)(((long)xcd * total) >> 3), t1 = (int)(((long)(xcd + 1) * total) >> 3);
  const int first = t0 + (int)(blockIdx.x >> 3);
  const int n_mine = first < t1 ? (t1 - first + n_wg - 1) / n_wg : 0;
  const int n_kt = d / SG_BK;
  const int n_steps = n_mine * n_kt;
  if (n_steps == 0) return;

  // DMA addressing.  Lane L of wave w fills slot (row 16q + 4w + L/16, chunk
  // L%16) of a tile (q = 0..3); the logical chunk c = (L%16) ^ swz(row) does
  // not depend on q.  X tile t, row r, chunk c: token 128t + r + 64(c/8),
  // k 8(c%8); W tile t, row k, chunk c: column 64t + 8(c%8) of Wg (c < 8) or
  // Wu.  Every copy is a wave-uniform base (scalar registers: the tensor plus
  // the k offset of the step) and a per-lane 32-bit byte offset computed once
  // per tile; the gate and up halves of a weight row quad are two copies with
  // complementary lane masks.
  const int lrow = 4 * w + (lane >> 4);
  const int chunk = (lane & 15) ^ (((lane >> 4) << 2) | (w & 3));
  const int x_tok = lrow + 64 * (chunk >> 3);
  const int c8 = 8 * (chunk & 7);
  const bool gate_half = chunk < 8;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  uint32_t xoff[2][4], woff[2][4];
  auto tile_offsets = [&](int tile) {
    int mb, nb;
    tile_coords(tile, n_mblk, n_nblk, mb, nb);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int tok = min(mb * SG_BM + 128 * t + 16 * q + x_tok, T - 1);
        xoff[t][q] = (uint32_t)(((long)tok * d + c8) * 2);
        woff[t][q] = (uint32_t)(((long)(16 * q + lrow) * F + nb * SG_BN + 64 * t + c8) * 2);
      }
    }
  };
  // Stage k block kt of the tile whose offsets are loaded into `slot`.
  auto issue = [&](int kt, int slot) {
    const uint32_t sl = lds0 + slot * SG_SLOT;
    const char* xb = reinterpret_cast<const char*>(x) + (long)kt * SG_BK * 2;
    const char* gb = reinterpret_cast<const char*>(wg) + (long)kt * SG_BK * F * 2;
    const char* ub = reinterpret_cast<const char*>(wu) + (long)kt * SG_BK * F * 2;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        dma16_sbase(xoff[t][q], xb, sl + t * TILE_BYTES + (4 * q + wu_) * 1024);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t dst = sl + (2 + t) * TILE_BYTES + (4 * q + wu_) * 1024;
        if (gate_half) dma16_sbase(woff[t][q], gb, dst);
        else dma16_sbase(woff[t][q], ub, dst);
      }
    }
  };

  const LdsBases lb = make_lds_bases(lane);
  const TrNat tn0 = make_tr_nat(lane, 0), tn1 = make_tr_nat(lane, 1), tn2 = make_tr_nat(lane, 2),
              tn3 = make_tr_nat(lane, 3);

  // Operands of k step kk of a slot: X^T columns (4 token blocks) and W^T
  // rows (gate blocks 0, 1, up blocks 0, 1).
  struct Frags {
    bf16x8 xb[4], w[4];
  };
  auto load_frags = [&](const char* xs, const char* ws, int kk, Frags& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      f.xb[i] = *reinterpret_cast<const bf16x8*>(xs + (i & 1) * 8192 + (lb.row ^ (128 * (i >> 1) + 32 * kk)));
    f.w[0] = tr_nat(ws, tn0, kk);
    f.w[1] = tr_nat(ws, tn1, kk);
    f.w[2] = tr_nat(ws, tn2, kk);
    f.w[3] = tr_nat(ws, tn3, kk);
  };

  tile_offsets(first);
  issue(0, 0);
  int s = 0;
  for (int ti = 0; ti < n_mine; ++ti) {
    f32x16 accg[2][4], accu[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        accg[j][i] = zero16();
        accu[j][i] = zero16();
      }
    }
    for (int kt = 0; kt < n_kt; ++kt, ++s) {
      const int slot = s & 1;
      wait_dma();          // this wave's copies of step s have landed (and its earlier stores)
      lds_barrier();       // ... and everyone's; everyone is also done with the other slot
      const char* xs = smem + slot * SG_SLOT + wm * TILE_BYTES;
      const char* ws = smem + slot * SG_SLOT + (2 + wn) * TILE_BYTES;
      Frags cur, nxt;
      load_frags(xs, ws, 0, cur);
      // prefetch the next step (the next tile's first k block after the last)
      if (s + 1 < n_steps) {
        if (kt + 1 == n_kt) tile_offsets(first + (ti + 1) * n_wg);
        issue(kt + 1 == n_kt ? 0 : kt + 1, slot ^ 1);
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk + 1 < 4) load_frags(xs, ws, kk + 1, nxt);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          accg[0][i] = mfma32(cur.w[0], cur.xb[i], accg[0][i]);
          accu[0][i] = mfma32(cur.w[2], cur.xb[i], accu[0][i]);
          accg[1][i] = mfma32(cur.w[1], cur.xb[i], accg[1][i]);
          accu[1][i] = mfma32(cur.w[3], cur.xb[i], accu[1][i]);
        }
        if (kk + 1 < 4) cur = nxt;
      }
    }

    // Epilogue of the tile: D tile (j, i) gives lane the token
    // m0 + 128wm + 32i + (lane & 31) and, in registers 4q .. 4q+3, the columns
    // n0 + 64wn + 32j + 8q + 4(lane/32) + 0..3.
    int mb, nb;
    tile_coords(first + ti * n_wg, n_mblk, n_nblk, mb, nb);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = mb * SG_BM + 128 * wm + 32 * i + (lane & 31);
      if (tok < T) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const long o0 = (long)tok * F + nb * SG_BN + 64 * wn + 32 * j + 4 * (lane >> 5);
#pragma unroll
          for (int q = 0; q < 4; ++q) store_quad<SPLIT, ACT>(accg[j][i], accu[j][i], q, o0 + 8 * q, gate, up, act);
        }
      }
    }
  }
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

constexpr size_t kSwigluLds = (size_t)SG_NSTAGE * SG_SLOT;

template <bool SPLIT, int ACT>
static hipError_t launch_gate_up_t(const __bf16* x, const __bf16* wg, const __bf16* wu, __bf16* gate,
                                   __bf16* up, __bf16* act, int T, int d, int F, hipStream_t stream) {
  auto kern = swiglu_gate_up_kernel<SPLIT, ACT>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)kSwigluLds);
  if (e != hipSuccess) return e;
  int dev = 0, cus = 0;
  e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int n_mblk = (T + SG_BM - 1) / SG_BM, n_nblk = F / SG_BN;
  const int total = n_mblk * n_nblk;
  // one workgroup per CU (the ring takes 128 KiB of LDS), a multiple of the 8 XCDs
  int grid = ((cus > 0 ? cus : 256) + 7) & ~7;
  if (grid > ((total + 7) & ~7)) grid = (total + 7) & ~7;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), kSwigluLds, stream, x, wg, wu, gate, up, act, T, d, F,
                     n_mblk, n_nblk);
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
