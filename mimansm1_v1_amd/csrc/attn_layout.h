// Host-side layouts of the buffers the caller owns: the forward state (the
// fp16 operand copies and the O residual the backward reads) and the
// backward workspace (fp16 dO, the scaled Delta, the scale, the dK/dV
// partial sums).  Every region starts on a 256-byte boundary.
#pragma once
#include <stddef.h>

namespace mm1 {

// Grid sizes of the conversion kernels: one partial maximum per workgroup.
constexpr int kCvtBlocks = 512;     // attn_cvt16_kernel (K, V, Q)
#ifndef MM1_DELTA_BLOCKS
#define MM1_DELTA_BLOCKS 1024
#endif
constexpr int kDeltaBlocks = MM1_DELTA_BLOCKS;  // attn_delta16_kernel (max|dO|)

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Forward state, per (B, S, H, Hkv), D = 128:
//   q16  [B,S,H,D]   fp16   Q converted (written by the forward / prep)
//   k16  [B,S,Hkv,D] fp16
//   v16  [B,S,Hkv,D] fp16
//   olo  [B,S,H,D]   u8     the 8 mantissa bits of the forward's fp32 O
//                           after its bf16 truncation (lo8_bits)
//   vmax [kCvtBlocks] fp32  partial maxima of |V|
struct FwdState {
  size_t q16, k16, v16, olo, vmax, bytes;
};

inline FwdState fwd_state(int B, int S, int H, int Hkv) {
  const size_t nq = (size_t)B * S * H * 128, nkv = (size_t)B * S * Hkv * 128;
  FwdState s;
  s.q16 = 0;
  s.k16 = s.q16 + align256(nq * 2);
  s.v16 = s.k16 + align256(nkv * 2);
  s.olo = s.v16 + align256(nkv * 2);
  s.vmax = s.olo + align256(nq);
  s.bytes = s.vmax + align256(kCvtBlocks * 4);
  return s;
}

// Backward workspace:
//   do16     [B,S,H,D] fp16   fp16(2^E dO)
//   delta    [B,H,S]   fp32   -2^E Delta
//   lse      [B,H,S]   fp32   lse2 - log2(sm_scale): exp2(s scale2 - lse) = P sm_scale
//   dmax     [kDeltaBlocks] fp32  partial maxima of |dO|
//   scale    [64] fp32        scale[0] = 2^-E, scale[1] = 2^E
//   partials                  the dK/dV partial sums (fp32), as large as the
//                             per-head tiling needs: 2 * G slots of
//                             [B,S,Hkv,D] (none when G == 1)
struct BwdWs {
  size_t do16, delta, lse, dmax, scale, partials, bytes;
};

inline BwdWs bwd_ws(int B, int S, int H, int Hkv) {
  const size_t nq = (size_t)B * S * H * 128, nkv = (size_t)B * S * Hkv * 128;
  const int G = H / Hkv;
  BwdWs w;
  w.do16 = 0;
  w.delta = w.do16 + align256(nq * 2);
  w.lse = w.delta + align256((size_t)B * H * S * 4);
  w.dmax = w.lse + align256((size_t)B * H * S * 4);
  w.scale = w.dmax + align256(kDeltaBlocks * 4);
  w.partials = w.scale + 256;
  w.bytes = w.partials + (G > 1 ? align256((size_t)2 * G * nkv * 4) : 0);
  return w;
}

}  // namespace mm1
