// Shared device helpers for the gfx950 causal GQA flash-attention kernels.
//
// Tensor layouts (all contiguous, matching the reference's BSHD convention,
// CODE/mimans/model/attention_tilelang.py:119-124 and :253-261):
//   Q, O, dO, dQ : [B, S, H,   128] bf16 at the interface
//   K, V, dK, dV : [B, S, Hkv, 128] bf16 at the interface
//   lse2, delta  : [B, H, S]        fp32   (lse2 in log2 units, :186-188)
//
// Operand precision.  The attention products run on fp16 operands
// (v_mfma_f32_32x32x16_f16, the same rate as the bf16 form on gfx950):
// Q, K, V and dO are converted once to fp16 copies (exact for bf16 values in
// [2^-17, 65504]; dO is first scaled by a power of two), and the rounded
// intermediates P (softmax weights) and dS are fp16, with 11 significant bits
// against bf16's 8.  The GEMMs of the SwiGLU / head kernels keep bf16
// operands (bf16x8, mfma32).
//
// Matrix-core convention (32x32x16 MFMA, wave64):
//   A operand (32 x 16): lane l holds row (l & 31), eight k values;
//   B operand (16 x 32): lane l holds column (l & 31), eight k values;
//   the k values a lane holds are the same set for A and B, so any fixed
//   permutation of k inside a 16-block cancels in the product.
//   C/D (32 x 32 fp32, 16 regs): lane l holds column (l & 31); register r
//   holds row 8*(r/4) + 4*(l/32) + (r%4).
// A D tile read as a B operand of the next product therefore pairs slot t of
// k-step s with row 16*s + 8*(t/4) + 4*(l/32) + (t%4): the "pi" order.  A
// operands that meet such a B operand are read in the same pi order.
//
// LDS tiles are 64 rows x 128 16-bit values (256 B per row, 16 KiB),
// row-major, with the sixteen 16-byte chunks of row r permuted by
// chunk ^ swz(r).  They are filled straight from global memory by the LDS DMA
// path (global_load_lds_dwordx4: lane L of a wave lands at base + 16*L), and
// read either row-wise (ds_read_b128: a row of 8 k values per lane) or
// transposed (two ds_read_b64_tr_b16: a column of 8 rows per lane).  swz() is
// chosen so that both read patterns touch each bank once per 16-lane phase:
//   * row reads: 16 consecutive rows at one logical chunk -> 16 chunks;
//   * transposed reads: 4 consecutive rows (aligned to 4) x 4 consecutive
//     8-byte columns -> 16 different chunk slots.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// k-steps by which rows_chain2's operand reads run ahead of their products
// (1 measured faster than 0; 2 no faster than 1).
#ifndef MM1_FWD_PREFETCH
#define MM1_FWD_PREFETCH 1
#endif

// Forces a lambda or helper inline (large kernel bodies otherwise get real calls).
#define MM1_INLINE __attribute__((always_inline))

namespace mm1 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// the operand type of the fp16 LDS transpose read builtin
typedef __fp16 fp16x4_tr __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

#define MM1_LDS __attribute__((address_space(3)))
#define MM1_GLOBAL __attribute__((address_space(1)))

constexpr int HD = 128;            // head_dim supported by the kernels
constexpr int TILE_ROWS = 64;      // rows in one LDS tile
constexpr int TILE_BYTES = TILE_ROWS * HD * 2;   // 16 KiB

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The attention products: fp16 operands, fp32 accumulation.
__device__ __forceinline__ f32x16 mfma32h(const f16x8& a, const f16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// x of this lane combined with x of the lane 32 apart (the other half of a
// 32x32 product column), as VALU work: v_permlane32_swap exchanges the two
// halves of a register without an LDS round trip.
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// N products in order: product i takes the A fragment load(i), read PF
// products ahead of it, and after product i comes between(i).  Scheduling
// barriers keep that order, so the VALU work handed to between() runs while
// the products in flight occupy the matrix core (the compiler would
// otherwise gather it after the last product) and every read stays PF
// products ahead of its use.
template <int N, int PF, class Load, class Mma, class Between>
__device__ __forceinline__ void mfma_chain(Load&& load, Mma&& mma, Between&& between) {
  decltype(load(0)) fa[PF + 1];
#pragma unroll
  for (int i = 0; i < PF; ++i) {
    fa[i] = load(i);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (i + PF < N) fa[(i + PF) % (PF + 1)] = load(i + PF);
    __builtin_amdgcn_sched_barrier(0);
    mma(i, fa[i % (PF + 1)]);
    __builtin_amdgcn_sched_barrier(0);
    between(i);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// mfma_chain whose first PF fragments the caller read earlier (before a
// barrier, say), so the first product waits for no read.
template <int N, int PF, class Frag, class Load, class Mma, class Between>
__device__ __forceinline__ void mfma_chain_from(const Frag (&first)[PF], Load&& load, Mma&& mma,
                                                Between&& between) {
  static_assert(PF >= 1 && PF < N, "prefetch depth");
  Frag fa[PF + 1];
#pragma unroll
  for (int i = 0; i < PF; ++i) fa[i] = first[i];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (i + PF < N) fa[(i + PF) % (PF + 1)] = load(i + PF);
    __builtin_amdgcn_sched_barrier(0);
    mma(i, fa[i % (PF + 1)]);
    __builtin_amdgcn_sched_barrier(0);
    between(i);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Issue priority of this wave among the waves of its SIMD (0-3, higher
// first; equal priorities go oldest first).  Scheduling barriers on both
// sides keep the products where the caller put them relative to it.
template <int P>
__device__ __forceinline__ void wave_prio() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(P);
  __builtin_amdgcn_sched_barrier(0);
}

// -x, elementwise (flips the sign bits: exact)
__device__ __forceinline__ f16x8 neg8(const f16x8& x) {
  return __builtin_bit_cast(f16x8, __builtin_bit_cast(u32x4, x) ^ 0x80008000u);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Eight consecutive accumulator registers (base .. base+7) as an fp16 MFMA
// operand (round to nearest even, v_cvt_pk_f16_f32).
__device__ __forceinline__ f16x8 pack8(const f32x16& v, int base) {
  f16x8 r;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t] = (_Float16)v[base + t];
  return r;
}

// Eight bf16 values as fp16 (exact for |x| in [2^-17, 65504]).
__device__ __forceinline__ f16x8 bf16_to_f16(const bf16x8& x) {
  f16x8 r;
#pragma unroll
  for (int t = 0; t < 8; ++t) r[t] = (_Float16)(float)x[t];
  return r;
}

// Wait until all of this wave's outstanding global loads, LDS DMA copies
// included, have landed.  Inline assembly on purpose: the compiler does not
// see the DMA copies, so it would treat a builtin s_waitcnt as redundant and
// drop it.
__device__ __forceinline__ void wait_dma() { __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Workgroup barrier that orders LDS traffic only: unlike __syncthreads() it
// does not wait for outstanding global loads (LDS DMA prefetches keep
// flying).  Copies a wave needs before the barrier are waited for explicitly.
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Materialise a loaded operand here: the compiler may not sink the load into
// a loop, where its wait would also drain the LDS DMA copies in flight.
__device__ __forceinline__ void pin(bf16x8& x) { __asm__ volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(f16x8& x) { __asm__ volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(float& x) { __asm__ volatile("" : "+v"(x)); }

__device__ __forceinline__ int swz(int row) { return ((row & 3) << 2) | ((row >> 2) & 3); }

// Byte offset of logical 16-byte chunk `chunk` (0..15) of `row`.
__device__ __forceinline__ int row_off(int row, int chunk) {
  return row * 256 + ((chunk ^ swz(row)) << 4);
}

// LDS DMA: every lane of the wave copies `bytes` (16 or 4) from its global
// address to lds_base + bytes * lane.  Issued as inline assembly so that the
// compiler does not track the copy: it would otherwise wait for all
// outstanding copies (vmcnt(0)) before any LDS read it cannot prove disjoint
// from the copy target, which serialises the prefetch ring.  The kernels wait
// for the copies themselves (wait_dma / explicit vmcnt) before the barrier
// that publishes a tile; compiler-generated vmcnt waits for other loads can
// only over-wait because of the extra copies in flight.  lds_base must be
// wave-uniform.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const MM1_LDS void*)p;
}

__device__ __forceinline__ void dma16(const void* src, uint32_t lds_base) {
  __asm__ volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                   :: "v"(src), "s"(lds_base) : "memory", "m0");
}

__device__ __forceinline__ void dma4(const void* src, uint32_t lds_base) {
  __asm__ volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                   :: "v"(src), "s"(lds_base) : "memory", "m0");
}

// Same copy with a wave-uniform global base (scalar register pair) and a
// per-lane byte offset.
__device__ __forceinline__ void dma16_sbase(uint32_t lane_off, const void* sbase, uint32_t lds_base) {
  __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                   :: "v"(lane_off), "s"(sbase), "s"(lds_base) : "memory", "m0");
}

// Copy a 64 x 128 tile of 16-bit values into LDS with the DMA path.  Row r of the tile is
// at base + r*stride elements; rows at or beyond nvalid re-read row nvalid-1
// (finite data the kernels mask out).  NW waves share the 16 row quads; wave
// w copies quads w, w + NW, ...
//
// Lane L of wave w fills LDS slot (row 4*rq + L/16, chunk L%16), i.e. logical
// chunk (L%16) ^ swz(row).  Since swz(row) = 4*(L/16) + (rq & 3) and
// rq & 3 == w & 3 for every quad of the wave (NW is a multiple of 4), a lane's
// byte offset inside its row quad is the same for every quad and every tile:
// tile_lane_off() computes it once, and a full tile is copied with a scalar
// base per quad and no per-lane address arithmetic.
__device__ __forceinline__ uint32_t tile_lane_off(long stride, int tid) {
  const int lane = tid & 63, w = tid >> 6;
  const int rr = lane >> 4;
  const int chunk = (lane & 15) ^ ((rr << 2) | (w & 3));
  return (uint32_t)((rr * stride + 8 * chunk) * 2);
}

template <int NW, class T>
__device__ __forceinline__ void tile_dma(char* lds, const T* base, long stride, int nvalid,
                                         uint32_t lane_off, int tid) {
  static_assert(NW % 4 == 0, "row-quad swizzle needs a multiple of 4 waves");
  static_assert(sizeof(T) == 2, "16-bit elements");
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t l0 = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  if (nvalid >= TILE_ROWS) {
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i) {
      const int rq = i * NW + w;
      const char* sbase = reinterpret_cast<const char*>(base) + (long)(4 * rq) * stride * 2;
      __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                       :: "v"(lane_off), "s"(sbase), "s"(l0 + rq * 1024) : "memory", "m0");
    }
  } else {
    const int L = tid & 63;
#pragma unroll
    for (int i = 0; i < 16 / NW; ++i) {
      const int rq = i * NW + w;                 // row quad: rows 4rq .. 4rq+3
      const int row = 4 * rq + (L >> 4);
      const int chunk = (L & 15) ^ swz(row);     // logical chunk this lane's slot holds
      const int grow = min(row, nvalid - 1);
      dma16(base + (long)grow * stride + 8 * chunk, l0 + rq * 1024);
    }
  }
}

// Copy a 32 x 128 tile of 16-bit values (the layout of the first 32 rows of
// a 64-row tile) with the LDS DMA path; issued by all 8 waves, wave w copies
// row quad w (so swz(row) = 4*(L/16) + (w & 3) and tile_lane_off() applies
// as above).
template <class T>
__device__ __forceinline__ void tile32_dma(char* lds, const T* base, long stride, int nvalid,
                                           uint32_t lane_off, int tid) {
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t l0 = __builtin_amdgcn_readfirstlane(lds_addr(lds)) + w * 1024;
  if (nvalid >= 32) {
    const char* sbase = reinterpret_cast<const char*>(base) + (long)(4 * w) * stride * 2;
    __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                     :: "v"(lane_off), "s"(sbase), "s"(l0) : "memory", "m0");
  } else {
    const int L = tid & 63;
    const int row = 4 * w + (L >> 4);
    const int chunk = (L & 15) ^ swz(row);
    dma16(base + (long)min(row, nvalid - 1) * stride + 8 * chunk, l0);
  }
}

// Copy 64 consecutive floats (elements >= nvalid re-read element nvalid-1)
// into LDS; issued by one whole wave.
__device__ __forceinline__ void vec64_dma(char* lds, const float* base, int nvalid, int lane) {
  dma4(base + min(lane, nvalid - 1), __builtin_amdgcn_readfirstlane(lds_addr(lds)));
}

// ---------------------------------------------------------------------------
// Precomputed per-lane LDS addressing.  Every operand read of a tile is one of
// a few per-lane byte offsets plus a compile-time constant, so loops need no
// address arithmetic and the constants fold into the ds_read offset field.
//
// Row reads (rows_a: the A operand from a tile whose rows are the MFMA M
//   axis, rows 32*blk + (lane&31), k-step ks = columns 16*ks .. +15):
//   offset = blk*8192 + (row_base ^ 32*ks), with
//   row_base = (lane&31)*256 + 16*((lane>>5) ^ swz(lane&31)).
// Transposed reads (tr_a: the A operand from a tile whose rows are the k
//   axis, M index = tile column 32*blk + (lane&31), k-step ks = tile rows
//   16*ks .. +15 in pi order): offset = 4096*ks + tr_base[blk][r], r = 0, 1.
//   Within each 16-lane group, ds_read_b64_tr_b16 gives lane i element
//   (i & 3) of the 8-byte chunks addressed by lanes 4t + (i >> 2), t = 0..3;
//   lane j of the group therefore addresses row 16ks + 8r + 4h + (j >> 2),
//   columns 4(j & 3) .. +3 of its 16-column strip.
struct LdsBases {
  int row;
  int tr[4][2];
};

__device__ __forceinline__ LdsBases make_lds_bases(int lane) {
  LdsBases b;
  const int l32 = lane & 31, h = lane >> 5;
  b.row = l32 * 256 + 16 * (h ^ swz(l32));
  const int g = (lane >> 4) & 1, j = lane & 15, jj = j >> 2;
  const int x = 2 * g + ((j & 3) >> 1), half = j & 1;
  const int p0 = (4 * h + jj) * 256 + 8 * half + 64 * jj + 16 * (x ^ h);
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
#pragma unroll
    for (int r = 0; r < 2; ++r) b.tr[blk][r] = (p0 ^ (64 * blk + 32 * r)) + 2048 * r;
  }
  return b;
}

__device__ __forceinline__ f16x8 rows_a(const char* tile, const LdsBases& lb, int blk, int ks) {
  return *reinterpret_cast<const f16x8*>(tile + blk * 8192 + (lb.row ^ (32 * ks)));
}

// acc[jb] += A B over the 8 k-steps for the two 32-row blocks jb = 0, 1 of a
// row-major LDS tile (A = rows_a, B in registers), the A fragments read one
// k-step ahead of their products.  The scheduling barriers keep them there:
// the compiler would otherwise sink each read to its product, so every
// product pair would wait for the full LDS latency.
__device__ __forceinline__ void rows_chain2(const char* tile, const LdsBases& lb, const f16x8 (&b)[8],
                                            f32x16 (&acc)[2]) {
  constexpr int PF = MM1_FWD_PREFETCH;
  f16x8 fa[PF + 1][2];
#pragma unroll
  for (int ks = 0; ks < PF; ++ks) {
    fa[ks][0] = rows_a(tile, lb, 0, ks);
    fa[ks][1] = rows_a(tile, lb, 1, ks);
  }
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    if (ks + PF < 8) {
      fa[(ks + PF) % (PF + 1)][0] = rows_a(tile, lb, 0, ks + PF);
      fa[(ks + PF) % (PF + 1)][1] = rows_a(tile, lb, 1, ks + PF);
    }
    __builtin_amdgcn_sched_barrier(0);
    acc[0] = mfma32h(fa[ks % (PF + 1)][0], b[ks], acc[0]);
    acc[1] = mfma32h(fa[ks % (PF + 1)][1], b[ks], acc[1]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Stores a wave's 32 x 128 fp32 product tile as bf16 rows, each value times
// `scale` (per lane), through `lds`: 8 KiB owned by the wave.  In registers
// lane l holds tile row l & 31 and, in acc[db][r], the values
// 32db + 8(r/4) + 4(l/32) + r%4 of it (the D layout of the products), so a
// direct store instruction writes 32 separate 16-byte pieces.  Written to LDS
// and read back, each lane holds 16 bytes of one row and a store instruction
// covers four whole 256-byte rows.  The 16-byte chunks of LDS row i are
// permuted by chunk ^ (i & 15), which spreads both the writes (32 rows at
// one chunk) and the reads (16 chunks of one row) over the banks.  dst(i) is
// the global address of tile row i, or nullptr for a row outside the tensor.
// The lanes exchange data through LDS, which the compiler's per-thread view
// of memory does not see: wave_sync() keeps the writes before the reads.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One pass of store_tile_bf16: value(db, r) of every register through LDS
// to the rows dst(i).
template <class Val, class Dst>
__device__ __forceinline__ void store_tile_pass(Val&& value, char* lds, int lane, Dst&& dst) {
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      bf16x4 val;
#pragma unroll
      for (int c = 0; c < 4; ++c) val[c] = value(db, 4 * a4 + c);
      const int chunk = (4 * db + a4) ^ (l32 & 15);
      *reinterpret_cast<bf16x4*>(lds + l32 * 256 + chunk * 16 + 8 * h) = val;
    }
  }
  wave_sync();
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int row = 4 * k + (lane >> 4), ch = lane & 15;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(lds + row * 256 + ((ch ^ (row & 15)) << 4));
    __bf16* p = dst(row);
    if (p) *reinterpret_cast<bf16x8*>(p + 8 * ch) = x;
  }
}

template <class Dst>
__device__ __forceinline__ void store_tile_bf16(const f32x16 (&acc)[4], float scale, char* lds, int lane,
                                                Dst&& dst) {
  store_tile_pass([&](int db, int r) MM1_INLINE { return (__bf16)(acc[db][r] * scale); }, lds, lane, dst);
}

// The 8 mantissa bits of an fp32 x that follow its truncation to bf16:
// bits 16..9 of x (bit 7 of the byte is the truncation's last bit).  With
// the round-to-nearest bf16 output o, o and this byte give 15 mantissa bits
// of x back (lo8_decode); the residual costs one byte per value.
__device__ __forceinline__ uint32_t lo8_bits(float x) { return (__float_as_uint(x) >> 9) & 0xffu; }

// x from o = bf16(x) (round to nearest even) and q = lo8_bits(x): o is the
// truncation T of x or T + 1 (as sign-magnitude integers); q's top bit is T's
// last bit, which tells the two apart.  The 9 bits below the byte are taken
// at the middle of their range: |result - x| <= 2^-15 |x|.
__device__ __forceinline__ float lo8_decode(uint32_t o_bits, uint32_t q) {
  const uint32_t t = o_bits - ((o_bits ^ (q >> 7)) & 1u);
  return __uint_as_float((t << 16) | ((q & 0x7fu) << 9) | 0x100u);
}

// store_tile_bf16, and then lo8_bits of every value x = acc * scale to the
// 128-byte rows dst_lo(i), also through the wave's 8 KiB (once its
// first-pass reads are done): a lane writes its 4-value groups as dwords at
// 16-byte chunk (c ^ (i & 7)) of row i, then reads back 16-byte pieces, so a
// store instruction covers eight whole rows.
template <class Dst, class DstLo>
__device__ __forceinline__ void store_tile_bf16_lo(const f32x16 (&acc)[4], float scale, char* lds, int lane,
                                                   Dst&& dst, DstLo&& dst_lo) {
  store_tile_pass([&](int db, int r) MM1_INLINE { return (__bf16)(acc[db][r] * scale); }, lds, lane, dst);
  wave_sync();
  const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      uint32_t w = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) w |= lo8_bits(acc[db][4 * a4 + c] * scale) << (8 * c);
      const int col = 32 * db + 8 * a4 + 4 * h;   // byte column of the 4 values
      const int chunk = (col >> 4) ^ (l32 & 7);
      *reinterpret_cast<uint32_t*>(lds + l32 * 128 + (chunk << 4) + (col & 15)) = w;
    }
  }
  wave_sync();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int row = 8 * k + (lane >> 3), ch = lane & 7;
    const u32x4 x = *reinterpret_cast<const u32x4*>(lds + row * 128 + ((ch ^ (row & 7)) << 4));
    uint8_t* p = dst_lo(row);
    if (p) *reinterpret_cast<u32x4*>(p + 16 * ch) = x;
  }
}

__device__ __forceinline__ f16x8 tr_a(const char* tile, const LdsBases& lb, int blk, int ks) {
  f16x8 out;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const f16x4 v = __builtin_bit_cast(
        f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((MM1_LDS fp16x4_tr*)(tile + 4096 * ks + lb.tr[blk][r])));
#pragma unroll
    for (int t = 0; t < 4; ++t) out[4 * r + t] = v[t];
  }
  return out;
}

}  // namespace mm1
