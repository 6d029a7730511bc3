// Shared device helpers for the gfx950 causal GQA flash-attention kernels.
//
// Tensor layouts (all contiguous, matching the reference's BSHD convention,
// CODE/mimans/model/attention_tilelang.py:119-124 and :253-261):
//   Q, O, dO, dQ : [B, S, H,   128] bf16
//   K, V, dK, dV : [B, S, Hkv, 128] bf16
//   lse2, delta  : [B, H, S]        fp32   (lse2 in log2 units, :186-188)
//
// Matrix-core convention (v_mfma_f32_32x32x16_bf16, wave64):
//   A operand (32 x 16): lane l holds row (l & 31), eight k values;
//   B operand (16 x 32): lane l holds column (l & 31), eight k values;
//   the k values a lane holds are the same set for A and B, so any fixed
//   permutation of k inside a 16-block cancels in the product.
//   C/D (32 x 32 fp32, 16 regs): lane l holds column (l & 31); register r
//   holds row 8*(r/4) + 4*(l/32) + (r%4).
// A D tile read as a B operand of the next product therefore pairs slot t of
// k-step s with row 16*s + 8*(t/4) + 4*(l/32) + (t%4): the "pi" order below.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mm1 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int HD = 128;            // head_dim supported by the kernels
constexpr int TILE_ROWS = 64;      // rows in one LDS tile
constexpr int TILE_BYTES = TILE_ROWS * HD * 2;   // 16 KiB

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Eight consecutive accumulator registers (base, base+1, ..., base+7) as a
// bf16 MFMA operand (round to nearest even).
__device__ __forceinline__ bf16x8 pack8(const f32x16& v, int base) {
  bf16x8 r;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t] = (__bf16)v[base + t];
  return r;
}

// ---------------------------------------------------------------------------
// LDS tile layouts (byte offsets inside one 16 KiB tile).
//
// Row tile: [64 rows][128 cols] bf16, 256 B per row; 16-byte chunk c of row
// r lives at chunk c ^ (r & 15) so that 16 consecutive rows read at one
// logical chunk hit 16 different bank groups.
__device__ __forceinline__ int row_off(int row, int chunk) {
  return row * 256 + ((chunk ^ (row & 15)) << 4);
}

// Transposed tile: [128 cols][64 rows] bf16, 128 B per column, rows inside
// each 16-block stored in pi order (bits 2 and 3 of the row swapped) so that
// one 16-byte read returns the eight rows a lane needs for one k-step.
// Chunks are XOR-swizzled by a function of the column that keeps both the
// 32-lane column reads and the tile writes spread over the banks.
__device__ __forceinline__ int pi_pos(int j) {
  return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
}
__device__ __forceinline__ int tr_off(int col, int jp) {
  const int swz = ((col >> 1) ^ (col >> 3)) & 7;
  return col * 128 + ((((jp >> 3) ^ swz)) << 4) + ((jp & 7) << 1);
}

// 256 threads stage a 64 x 128 bf16 tile through registers: thread t owns
// rows 4*(t>>4) .. +3 and columns 8*(t&15) .. +7.  Rows at or beyond
// `nvalid` read as zero.
struct TileRegs {
  u32x4 r[4];
};

__device__ __forceinline__ void tile_load(TileRegs& t, const __bf16* __restrict__ base,
                                          long stride, int nvalid, int tid) {
  const int rg = tid >> 4, c = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * rg + i;
    if (row < nvalid) {
      t.r[i] = *reinterpret_cast<const u32x4*>(base + (long)row * stride + 8 * c);
    } else {
      t.r[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

__device__ __forceinline__ void tile_store_rows(const TileRegs& t, char* lds, int tid) {
  const int rg = tid >> 4, c = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    *reinterpret_cast<u32x4*>(lds + row_off(4 * rg + i, c)) = t.r[i];
  }
}

__device__ __forceinline__ void tile_store_tr(const TileRegs& t, char* lds, int tid) {
  const int rg = tid >> 4, c = tid & 15;
  const int jp0 = pi_pos(4 * rg);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t w0 = t.r[0][m], w1 = t.r[1][m], w2 = t.r[2][m], w3 = t.r[3][m];
    const u32x2 lo = {(w0 & 0xffffu) | (w1 << 16), (w2 & 0xffffu) | (w3 << 16)};
    const u32x2 hi = {(w0 >> 16) | (w1 & 0xffff0000u), (w2 >> 16) | (w3 & 0xffff0000u)};
    const int col = 8 * c + 2 * m;
    *reinterpret_cast<u32x2*>(lds + tr_off(col, jp0)) = lo;
    *reinterpret_cast<u32x2*>(lds + tr_off(col + 1, jp0)) = hi;
  }
}

// A operand from a row tile: rows 32*blk + (lane&31), k-step ks (16 columns).
__device__ __forceinline__ bf16x8 lds_a_rows(const char* lds, int blk, int ks, int lane) {
  return *reinterpret_cast<const bf16x8*>(lds + row_off(32 * blk + (lane & 31), 2 * ks + (lane >> 5)));
}

// A operand from a transposed tile: columns 32*blk + (lane&31), rows of k-step
// ks (16 rows) in pi order.
__device__ __forceinline__ bf16x8 lds_a_tr(const char* lds, int blk, int ks, int lane) {
  return *reinterpret_cast<const bf16x8*>(lds + tr_off(32 * blk + (lane & 31), 16 * ks + 8 * (lane >> 5)));
}

}  // namespace mm1
