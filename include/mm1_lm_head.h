/* C ABI of the gfx950 fused cross-entropy head (same library and conventions
 * as mm1_attn.h: bf16 tensors as `void*`, the HIP stream as `void*`,
 * caller-owned buffers, no allocation, no synchronisation, return 0 / a
 * negative MM1_E_* code / a positive hipError_t).
 *
 * Replaces the TileLang log-sum-exp kernel and the logits work of
 * FusedCrossEntropy in CODE/mimans/model/lm_head_tilelang.py.
 * Layouts (row-major, contiguous rows, 16-byte aligned):
 *   hidden  [T, d_model] bf16 (already multiplied by the logit scale, as
 *           LMHead.forward does before the kernel, lm_head_tilelang.py:318-319)
 *   weight  [d_model, vocab] bf16
 *   targets [T] int64: a class in [0, vocab) or ignore_index; any other value
 *           is treated as ignored
 *   lse, target_logit, loss [T] fp32 (natural log)
 * Requirements: T >= 1; d_model and vocab positive multiples of 128.
 */
#ifndef MM1_LM_HEAD_H
#define MM1_LM_HEAD_H

#include <stddef.h>

#include "mm1_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of scratch mm1_lm_head_lse needs (per-token partial maxima and sums,
 * one per 64-entry column group of each 256-entry vocabulary block). */
size_t mm1_lm_head_workspace_size(int T, int vocab);

/* lse[t] = log sum_v exp(hidden[t] . weight[:, v]) with fp32 accumulation of
 * the bf16 products, the [T, vocab] logits never stored.  With targets:
 * target_logit[t] = hidden[t] . weight[:, c] (the same accumulation) with
 * c = targets[t], or c = 0 when targets[t] is negative (ignore_index) or
 * >= vocab, as the reference's gather over targets.clamp(min=0); and
 * loss[t] = lse[t] - target_logit[t], 0 for ignored or out-of-range targets
 * (either output may be NULL).  Replaces get_kernel((T, d_model, vocab))(hidden, weight) -> Lse
 * (logsumexp_kernel, lm_head_tilelang.py:92-156) and, in
 * FusedCrossEntropy.forward, gather_target_logits and the per-token loss
 * (:186-190, :201-209).  Deterministic. */
int mm1_lm_head_lse(const void* hidden, const void* weight, const long long* targets, long long ignore_index,
                    float* lse, float* target_logit, float* loss, void* workspace, size_t workspace_bytes,
                    int T, int d_model, int vocab, void* stream);

/* Logits gradient of vocabulary entries [v0, v0 + vn):
 *   d_logits[t][v - v0] = bf16((exp(logit[t][v] - lse[t]) - [v == targets[t]]) * scale[0])
 * for tokens with a valid target, 0 for ignored tokens; rows of d_logits have
 * stride ld (>= vn, a multiple of 8).  scale is a device fp32 scalar (the loss
 * gradient over the count of valid tokens).  v0 and vn are multiples of 128,
 * v0 + vn <= vocab.  Replaces the per-chunk `probs` of
 * FusedCrossEntropy.backward (lm_head_tilelang.py:226-238), which the caller
 * then multiplies into d_hidden and d_weight. */
int mm1_lm_head_dlogits(const void* hidden, const void* weight, const long long* targets, long long ignore_index,
                        const float* lse, const float* scale, void* d_logits, long ld,
                        int T, int d_model, int vocab, int v0, int vn, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MM1_LM_HEAD_H */
