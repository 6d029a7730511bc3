// Persistent bf16 GEMM core for gfx950 shared by the SwiGLU and LM-head
// kernels: D = W^T X^T over token blocks of 256 and column blocks of 256,
// fp32 accumulation, with the epilogue supplied by the caller.
//
//   X [T, d] bf16 rows (tokens), W [d, ldw] bf16 rows (k), D[col][token].
//
// A workgroup (8 waves, two per SIMD, one workgroup per CU) owns 256 tokens
// x 256 columns and walks k in steps of 64 staged in a two-slot LDS ring (64
// KiB per slot) by the LDS DMA:
//   * X: two 64 x 256 B tiles; row r of tile t holds tokens 128t + r (left
//     half) and 128t + 64 + r (right half), 64 k values each;
//   * W: two 64 x 256 B tiles, row k of tile t holding the columns
//       PAIRED  : w0[k][64t .. 64t+63] then w1[k][64t .. 64t+63] (the SwiGLU
//                 gate and up weights, workgroup column step 128 of each);
//       !PAIRED : w0[k][128t .. 128t+127] (workgroup column step 256).
// Wave (wm, wn), wm = w & 1, wn = w >> 1 (0..3), accumulates tokens
// 128wm .. +127 against two 32-column blocks of W tile wn >> 1: PAIRED: w0
// block wn & 1 (acc[0]) and the same w1 block (acc[1]); !PAIRED: blocks
// 2(wn & 1) and 2(wn & 1) + 1.  acc[b][i] is the 32 x 32 product of block b
// and token block i (lane: token 32i + (lane & 31); register 4q + e: column
// 8q + 4(lane/32) + e of the block).  Two waves per SIMD let one wave's LDS
// reads run under the other's MFMAs (128 accumulators each).  W^T is read
// with the LDS transpose read in natural k order, X with row reads; both
// conflict-free on the swizzled tile layout.  Tiles are dealt to the 8 XCDs
// in contiguous runs of a grouped order (8 token blocks, then the next
// column block) so an XCD's concurrent tiles share X rows and W columns in
// its L2.  A ragged last round is split into half tiles (see run()).
#pragma once
#include "mm1_common.h"

namespace mm1 {
namespace gemm {

constexpr int BM = 256;                    // tokens per workgroup
constexpr int BK = 64;                     // k per ring slot
constexpr int SLOT = 4 * TILE_BYTES;       // X tiles 0, 1; W tiles 0, 1
constexpr int NSTAGE = 2;
constexpr size_t LDS_BYTES = (size_t)NSTAGE * SLOT;
constexpr int GROUP = 8;                   // token blocks per group of the tile order

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

// A operand (32 columns x 16 k) from a k-major weight tile: the column block
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

__device__ __forceinline__ void tile_coords(int t, int n_mblk, int n_nblk, int& mb, int& nb) {
  const int per_group = GROUP * n_nblk;
  const int group = t / per_group, first = group * GROUP;
  const int gm = min(GROUP, n_mblk - first);
  const int local = t - group * per_group;
  mb = first + local % gm;
  nb = local / gm;
}

struct Problem {
  const __bf16* x;
  const __bf16* w0;
  const __bf16* w1;   // PAIRED only
  int T, d;           // tokens, reduction length (multiple of 64)
  int ldw;            // row stride of w0 / w1 in elements
  int ncols;          // !PAIRED: columns of w0 that exist (multiple of 8); later ones are clamped
  int n_mblk, n_nblk;
};

// Stores one bf16 output of a wave's tile, 128 tokens x 32 columns, whose
// values the lane holds as val(i, q): the bf16x4 of columns 8q + 4(lane/32)
// .. +3 of token 32i + (lane & 31) (the accumulator layout above).  Stored
// directly, an instruction writes 32 separate 16-byte pieces; here they go
// through `lds` (4 KiB owned by the wave) in two rounds of 64 tokens, after
// which each lane holds 16 bytes of one token's 64-byte row and an
// instruction writes the rows of 16 tokens.  row(r) is the global address of
// the first column of token r (0..127) of the tile, or nullptr for a token
// outside the tensor.  The 16-byte chunks of LDS row r are permuted by
// chunk ^ ((r >> 2) & 3), which spreads the writes over the banks.
// wave_sync() orders the lanes' exchange, which the compiler's per-thread
// view of memory does not see.
constexpr int STAGE_BYTES = 4096;          // per wave

template <class Val, class Row>
__device__ __forceinline__ void store_rows64(char* lds, int lane, Val&& val, Row&& row) {
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int r = 32 * ii + l32;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x4 v = val(2 * half + ii, q);
        *reinterpret_cast<bf16x4*>(lds + r * 64 + ((q ^ ((r >> 2) & 3)) << 4) + 8 * h) = v;
      }
    }
    wave_sync();
    bf16x8 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 16 * k + (lane >> 2), c = lane & 3;
      x[k] = *reinterpret_cast<const bf16x8*>(lds + r * 64 + ((c ^ ((r >> 2) & 3)) << 4));
    }
    wave_sync();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 16 * k + (lane >> 2), c = lane & 3;
      __bf16* p = row(64 * half + r);
      if (p) *reinterpret_cast<bf16x8*>(p + 8 * c) = x[k];
    }
  }
}

// The same for a wave's 128 tokens x 64 columns of the single-matrix layout
// (two 32-column blocks): val(i, b, q) is the bf16x4 of columns
// 32b + 8q + 4(lane/32) .. +3 of token 32i + (lane & 31).  Four rounds of 32
// tokens through `lds` (4 KiB owned by the wave); each lane then holds 16
// bytes of one token's 128-byte row and an instruction writes the rows of 8
// tokens.  row(r) is the global address of the first column of token r or
// nullptr; chunk_ok(c) says whether the 8 columns 8c .. 8c+7 exist.  Chunks
// of LDS row r are permuted by chunk ^ ((r >> 1) & 7).
template <class Val, class Row, class ChunkOk>
__device__ __forceinline__ void store_rows128(char* lds, int lane, Val&& val, Row&& row, ChunkOk&& chunk_ok) {
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x4 v = val(i, b, q);
        const int chunk = (4 * b + q) ^ ((l32 >> 1) & 7);
        *reinterpret_cast<bf16x4*>(lds + l32 * 128 + (chunk << 4) + 8 * h) = v;
      }
    }
    wave_sync();
    bf16x8 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 8 * k + (lane >> 3), c = lane & 7;
      x[k] = *reinterpret_cast<const bf16x8*>(lds + r * 128 + ((c ^ ((r >> 1) & 7)) << 4));
    }
    wave_sync();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 8 * k + (lane >> 3), c = lane & 7;
      __bf16* p = row(32 * i + r);
      if (p && chunk_ok(c)) *reinterpret_cast<bf16x8*>(p + 8 * c) = x[k];
    }
  }
}

// Launch geometry: one workgroup per CU, a multiple of the 8 XCDs.
inline int persistent_grid(int cus, int total_tiles) {
  int grid = ((cus > 0 ? cus : 256) + 7) & ~7;
  const int cap = (total_tiles + 7) & ~7;
  return grid < cap ? grid : cap;
}

// The persistent loop of one workgroup (512 threads, all of which must call
// it); pro(mb, nb) runs at the start of each tile, epi(mb, nb, acc) at its
// end with acc[2][4] as described above.
template <bool PAIRED, class Pro, class Epi>
__device__ __forceinline__ void run(const Problem& p, char* smem, Pro&& pro, Epi&& epi) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w & 1, wn = w >> 1;
  const int wu_ = __builtin_amdgcn_readfirstlane(w);

  const int total = p.n_mblk * p.n_nblk;
  const int xcd = blockIdx.x & 7, n_wg = gridDim.x >> 3, j = (int)(blockIdx.x >> 3);
  const int t0 = (int)(((long)xcd * total) >> 3), t1 = (int)(((long)(xcd + 1) * total) >> 3);
  const int first = t0 + j;
  // Ragged last round: when at most half of this XCD's workgroups would get
  // one more tile, its rem leftover tiles are split by W tile into 2 rem half
  // tiles, one for each of the first 2 rem workgroups (the waves of the other
  // W tile skip the products and the epilogue), so no workgroup runs a whole
  // extra tile alone.
  const int n_full = (t1 - t0) / n_wg, rem = (t1 - t0) % n_wg;
  const bool split = rem > 0 && 2 * rem <= n_wg;
  const int n_mine = split ? n_full + (j < 2 * rem ? 1 : 0)
                           : (first < t1 ? (t1 - first + n_wg - 1) / n_wg : 0);
  auto tile_at = [&](int ti, int& half) {   // half: -1 whole tile, else the W tile kept
    if (split && ti == n_full) {
      half = j & 1;
      return t0 + n_full * n_wg + (j >> 1);
    }
    half = -1;
    return first + ti * n_wg;
  };
  const int n_kt = p.d / BK;
  const int n_steps = n_mine * n_kt;
  if (n_steps == 0) return;

  // DMA addressing: wave w fills row quads rq = 8q + w (q = 0, 1) of every
  // tile, rows 32q + 4w + L/16; rq & 3 == w & 3, so the logical chunk
  // c = (L%16) ^ swz(row) is the same for both quads.
  const int lrow = 4 * w + (lane >> 4);
  const int chunk = (lane & 15) ^ (((lane >> 4) << 2) | (w & 3));
  const int x_tok = lrow + 64 * (chunk >> 3);
  const int c8 = 8 * (chunk & 7);
  const bool first_half = chunk < 8;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  uint32_t xoff[2][2], woff[2][2];
  auto tile_offsets = [&](int tile) {
    int mb, nb;
    tile_coords(tile, p.n_mblk, p.n_nblk, mb, nb);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int col = PAIRED ? nb * 128 + 64 * t + c8 : min(nb * 256 + 128 * t + 8 * chunk, p.ncols - 8);
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int tok = min(mb * BM + 128 * t + 32 * q + x_tok, p.T - 1);
        xoff[t][q] = (uint32_t)(((long)tok * p.d + c8) * 2);
        woff[t][q] = (uint32_t)(((long)(32 * q + lrow) * p.ldw + col) * 2);
      }
    }
  };
  auto issue = [&](int kt, int slot) {
    const uint32_t sl = lds0 + slot * SLOT;
    const char* xb = reinterpret_cast<const char*>(p.x) + (long)kt * BK * 2;
    const char* b0 = reinterpret_cast<const char*>(p.w0) + (long)kt * BK * p.ldw * 2;
    const char* b1 = reinterpret_cast<const char*>(p.w1) + (long)kt * BK * p.ldw * 2;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int q = 0; q < 2; ++q)
        dma16_sbase(xoff[t][q], xb, sl + t * TILE_BYTES + (8 * q + wu_) * 1024);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t dst = sl + (2 + t) * TILE_BYTES + (8 * q + wu_) * 1024;
        if (PAIRED) {
          if (first_half) dma16_sbase(woff[t][q], b0, dst);
          else dma16_sbase(woff[t][q], b1, dst);
        } else {
          dma16_sbase(woff[t][q], b0, dst);
        }
      }
    }
  };

  const LdsBases lb = make_lds_bases(lane);
  const int blk0 = PAIRED ? (wn & 1) : 2 * (wn & 1);
  const TrNat ta = make_tr_nat(lane, blk0);
  const TrNat tb = make_tr_nat(lane, PAIRED ? 2 + (wn & 1) : blk0 + 1);

  struct Frags {
    bf16x8 xb[4], w[2];
  };
  auto load_frags = [&](const char* xs, const char* ws, int kk, Frags& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      f.xb[i] = *reinterpret_cast<const bf16x8*>(xs + (i & 1) * 8192 + (lb.row ^ (128 * (i >> 1) + 32 * kk)));
    f.w[0] = tr_nat(ws, ta, kk);
    f.w[1] = tr_nat(ws, tb, kk);
  };

  int iss_ti = 0, iss_kt = 0;
  auto issue_next = [&](int slot) {
    int h;
    if (iss_kt == 0) tile_offsets(tile_at(iss_ti, h));
    issue(iss_kt, slot);
    if (++iss_kt == n_kt) {
      iss_kt = 0;
      ++iss_ti;
    }
  };
  issue_next(0);

  int s = 0;
  for (int ti = 0; ti < n_mine; ++ti) {
    int mb, nb, half;
    tile_coords(tile_at(ti, half), p.n_mblk, p.n_nblk, mb, nb);
    const bool active = half < 0 || (wn >> 1) == half;   // wave-uniform
    f32x16 acc[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[b][i] = zero16();
    }
    for (int kt = 0; kt < n_kt; ++kt, ++s) {
      const int slot = s & 1;
      wait_dma();          // this wave's copies of step s (the only ones in flight) have landed
      lds_barrier();       // ... and everyone's; everyone is also done with the other slot
      if (kt == 0) pro(mb, nb);
      if (s + 1 < n_steps) issue_next(slot ^ 1);
      if (active) {
        const char* xs = smem + slot * SLOT + wm * TILE_BYTES;
        const char* ws = smem + slot * SLOT + (2 + (wn >> 1)) * TILE_BYTES;
        Frags cur, nxt;
        load_frags(xs, ws, 0, cur);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          if (kk + 1 < 4) load_frags(xs, ws, kk + 1, nxt);
          // keep the next k step's reads ahead of this one's products: the
          // scheduler would otherwise sink them and wait on each pair
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[0][i] = mfma32(cur.w[0], cur.xb[i], acc[0][i]);
            acc[1][i] = mfma32(cur.w[1], cur.xb[i], acc[1][i]);
          }
          __builtin_amdgcn_sched_barrier(0);
          if (kk + 1 < 4) cur = nxt;
        }
      }
    }
    if (active) epi(mb, nb, acc);
  }
}

}  // namespace gemm
}  // namespace mm1
