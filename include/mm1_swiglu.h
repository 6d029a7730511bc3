/* C ABI of the gfx950 SwiGLU feed-forward kernels (same library and
 * conventions as mm1_attn.h: bf16 tensors as `void*`, the HIP stream as
 * `void*`, caller-owned buffers, no allocation, no synchronisation, return
 * 0 / a negative MM1_E_* code / a positive hipError_t).
 *
 * Replaces the TileLang kernels of CODE/mimans/model/swiglu_tilelang.py.
 * Layouts (row-major, contiguous rows, 16-byte aligned):
 *   x            [T, d_model] bf16
 *   w_gate, w_up [d_model, ffn] bf16 (the reference's parameter layout)
 *   gate, up, act, d_act [T, ffn] bf16
 * Requirements: T >= 1, d_model and ffn positive multiples of 128 (the
 * reference's FFNConfig asserts the same, swiglu_tilelang.py:314-316).
 */
#ifndef MM1_SWIGLU_H
#define MM1_SWIGLU_H

#include <stddef.h>

#include "mm1_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Gate/up projection with the SwiGLU epilogue, one launch:
 *  mode MM1_SWIGLU_ACT   (0): act = bf16(silu(x w_gate) * (x w_up)) from the
 *                             fp32 accumulators; gate, up unused (may be NULL).
 *                             Replaces gate_up_swiglu (swiglu_tilelang.py:119-156).
 *  mode MM1_SWIGLU_SPLIT (1): gate = bf16(x w_gate), up = bf16(x w_up); act unused.
 *                             Replaces gate_up_split (:158-200).
 *  mode MM1_SWIGLU_TRAIN (2): gate and up as mode 1, and
 *                             act = bf16(bf16(silu(gate)) * up) on the bf16 values:
 *                             gate_up_split followed by FusedSwiGLU.forward's
 *                             `F.silu(gate) * up` (:283-284), fused.
 * fp32 accumulation over d_model; bf16 MFMA. */
#define MM1_SWIGLU_ACT 0
#define MM1_SWIGLU_SPLIT 1
#define MM1_SWIGLU_TRAIN 2
int mm1_swiglu_gate_up(const void* x, const void* w_gate, const void* w_up,
                       void* gate, void* up, void* act,
                       int T, int d_model, int ffn, int mode, void* stream);

/* SwiGLU gradient: with s = sigmoid(gate), in fp32 from the bf16 inputs,
 *   d_gate = bf16(d_act * up * s * (1 + gate * (1 - s))),  d_up = bf16(d_act * gate * s).
 * d_gate and d_up rows have stride ld_out elements (ld_out >= ffn, a multiple
 * of 8), so both can be written into one [T, 2*ffn] buffer.
 * Replaces swiglu_grad (swiglu_tilelang.py:202-240). */
int mm1_swiglu_grad(const void* d_act, const void* gate, const void* up,
                    void* d_gate, void* d_up, int T, int ffn, long ld_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MM1_SWIGLU_H */
