/* C ABI of the MI355X (gfx950) causal GQA flash-attention library.
 *
 * Drop-in boundary for the attention kernels of Mimans M1
 * (CODE/mimans/model/attention_tilelang.py).  Plain C: bf16 tensors are passed
 * as `void*`, fp32 tensors as `float*`, the HIP stream as `void*`
 * (a hipStream_t; NULL = the default stream).  The caller owns every buffer;
 * the library allocates no device memory (apart from the static scratch of
 * mm1_attn_bwd_noalloc, below), never synchronises and is safe to call from
 * several host threads.  Its only host state is a cache of per-shape
 * workgroup dispatch tables (mm1_attn_dispatch_order) and, per backward
 * workspace address, the layout of the dK/dV partial sums the last
 * mm1_attn_bwd_dkdv_tiles call on it wrote (checked by the calls that sum
 * them).
 *
 * Layouts (all contiguous, last dimension stride 1):
 *   q, o, dO, dq : [B, S, H,   D] bf16
 *   k, v, dk, dv : [B, S, Hkv, D] bf16
 *   lse2, delta  : [B, H, S]      fp32
 * Requirements: B >= 1, S >= 1, H % Hkv == 0, D == 128, sm_scale > 0.
 *
 * Operand precision.  The products run on the matrix cores with fp16
 * operands and fp32 accumulation.  The library converts q, k, v (and dO,
 * after scaling it by a power of two chosen from max|dO| and max|V|) to fp16
 * copies, which is exact for bf16 values of magnitude in [2^-17, 65504];
 * q, k and v must lie within fp16's range (|x| <= 65504; smaller values lose
 * at most 2^-25 absolutely).  The softmax weights P and the score gradients
 * dS are rounded to fp16 (11 significant bits) before their products; the
 * reference rounds them to bf16 (8 bits, attention_tilelang.py:178-180,
 * :306-314).
 *
 * The forward state.  The forward leaves in a caller-owned buffer
 * (mm1_attn_fwd_state_size bytes) what the backward reads: the fp16 copies
 * of q, k, v, one residual byte per value of its fp32 output O (the 8
 * mantissa bits below bf16's, so the backward's Delta = rowsum(O dO) sees
 * 15 significant bits of O: the bf16 o and this byte) and partial maxima of
 * |V|.  A caller keeps it with (o, lse2) until the backward, as the
 * reference's FlashAttention.forward saves (q, k, v, out, lse)
 * (attention_tilelang.py:365).
 *
 * Return value: 0 on success, a negative MM1_E_* code for an argument error,
 * or a positive hipError_t from the launch.  mm1_attn_strerror() names both.
 */
#ifndef MM1_ATTN_H
#define MM1_ATTN_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MM1_ATTN_VERSION 4

#define MM1_OK 0
#define MM1_E_NULL (-1)        /* a required pointer is NULL */
#define MM1_E_SHAPE (-2)       /* B, S, H or Hkv out of range, or H % Hkv != 0 */
#define MM1_E_HEAD_DIM (-3)    /* head_dim other than 128 */
#define MM1_E_WORKSPACE (-4)   /* state or workspace smaller than its *_size() */
#define MM1_E_SCALE (-5)       /* sm_scale not a positive finite number */
#define MM1_E_ALIGN (-6)       /* a tensor pointer is not 16-byte aligned */
#define MM1_E_TILES (-7)       /* tiling index out of range (see mm1_attn_tile_count) */
#define MM1_E_LAYOUT (-8)      /* the workspace holds no dK/dV partial sums of this shape and
                                  dK/dV tiling (see mm1_attn_bwd_dkdv_reduce_tiles) */
#define MM1_E_SCRATCH (-9)     /* shape too large for mm1_attn_bwd_noalloc's static scratch */

/* Bytes of device memory mm1_attn_bwd_noalloc holds per device (see there). */
#define MM1_NOALLOC_SCRATCH_BYTES ((size_t)256 << 20)

/* Kernel kinds for the tiling queries below. */
#define MM1_TILES_FWD 0
#define MM1_TILES_DKDV 1
#define MM1_TILES_DQ 2

/* Library version (MM1_ATTN_VERSION of the build). */
int mm1_attn_version(void);

/* Bytes of the forward state of a shape (0 for a bad shape).  No
 * counterpart in the reference, whose backward reads the bf16 q, k, v and
 * out it saved (attention_tilelang.py:365, :370). */
size_t mm1_attn_fwd_state_size(int B, int S, int H, int Hkv, int D);

/* Forward: o = softmax(q k^T * sm_scale [+ causal mask]) v, per query head h
 * reading KV head h / (H / Hkv); lse2[b,h,i] = log2(e) * logsumexp_j(s_ij).
 * Also writes the forward state (state_bytes >= mm1_attn_fwd_state_size).
 * Replaces get_kernel("fwd", B, H, S, D, causal, groups)(q, k, v) -> (O, lse),
 * the TileLang kernel flash_fwd (attention_tilelang.py:110-190, called :364). */
int mm1_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse2,
                 void* state, size_t state_bytes,
                 int B, int S, int H, int Hkv, int D, int causal, float sm_scale, void* stream);

/* The forward with fp32 o [B, S, H, D]: the values mm1_attn_fwd rounds to
 * bf16, from the same kernel of tiling `tiles` (-1 = the default); the
 * state as mm1_attn_fwd's.  No counterpart in the reference, whose forward
 * writes bf16 O (attention_tilelang.py:182-185): for callers that check O
 * where one bf16 half-ulp of |O| is already more than their tolerance. */
int mm1_attn_fwd_f32(const void* q, const void* k, const void* v, float* o, float* lse2,
                     void* state, size_t state_bytes,
                     int B, int S, int H, int Hkv, int D, int causal, float sm_scale, int tiles,
                     void* stream);

/* A forward state without the forward: the fp16 copies of q, k, v and
 * max|V| (the O residual is not written; the backward then needs the
 * caller's delta, mm1_attn_bwd_prep_delta).  For a caller of the reference's
 * bwd kernel handle, which takes (q, k, v, dO, lse, Delta) directly
 * (attention_tilelang.py:386-388). */
int mm1_attn_prep(const void* q, const void* k, const void* v, void* state, size_t state_bytes,
                  int B, int S, int H, int Hkv, int D, void* stream);

/* Backward preprocess of the reference: delta[b,h,i] = sum_d o[b,i,h,d] *
 * dO[b,i,h,d] (fp32) from the bf16 o.  Replaces flash_delta(B, H, S, D)(O,
 * dO) -> Delta (attention_tilelang.py:192-217, called :380).  The backward
 * below computes its own Delta from the forward state (o plus its residual);
 * this call is the reference's operator for callers that want it. */
int mm1_attn_delta(const void* o, const void* dO, float* delta,
                   int B, int S, int H, int D, void* stream);

/* Bytes of the backward workspace of a shape (0 for a bad shape): fp16 dO,
 * the scaled Delta, lse2 - log2(sm_scale), the dO scale and the dK/dV
 * partial sums (2 * G fp32 slots of [B, S, Hkv, D] when G = H / Hkv > 1).  No counterpart in the
 * reference, whose backward takes caller-zeroed fp32 dQ/dK/dV accumulators
 * instead (attention_tilelang.py:381-383). */
size_t mm1_attn_bwd_workspace_size(int B, int S, int H, int Hkv, int D);

/* Backward: bf16 dq, dk, dv from (o, dO, lse2) and the forward state:
 * Delta from o and the state's residual, dO to fp16, dK/dV, then dQ with the
 * dK/dV group sum in the same launch.  Replaces flash_delta + get_kernel(
 * "bwd", ...)(q, k, v, dO, lse, Delta, dQ, dK, dV) + flash_unswizzle + the
 * dk/dv casts (attention_tilelang.py:380-389, :242-323).  Deterministic: no
 * atomics; bitwise identical across repeated calls. */
int mm1_attn_bwd(const void* o, const void* dO, const float* lse2,
                 const void* state, size_t state_bytes,
                 void* dq, void* dk, void* dv,
                 void* workspace, size_t workspace_bytes,
                 int B, int S, int H, int Hkv, int D, int causal, float sm_scale, void* stream);

/* mm1_attn_bwd without a workspace argument, for callers that cannot
 * allocate device memory around the call: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  No counterpart in the
 * reference.  It calls no allocating routine: the backward workspace of the
 * default tilings goes to a static device array of
 * MM1_NOALLOC_SCRATCH_BYTES (256 MiB), a device-side static of the library's
 * code object (not a hipMalloc).  A device maps it when the first
 * mm1_attn_bwd_noalloc call runs there (the HIP runtime then loads the code
 * object that holds it) and holds it until the process ends; loading the
 * library and calling its other entry points do not map it (they map the
 * kernels' code objects, about 2 MiB; tests/test_gpu_memory.py measures
 * both).
 * mm1_attn_bwd_noalloc_scratch_size() gives the bytes a shape needs (about
 * 150 MiB at the training shapes of 16,384 tokens); a shape needing more
 * returns MM1_E_SCRATCH.  Every call on one device shares that device's
 * array: calls that overlap on one device (several streams or host threads)
 * race and must be serialised by the caller.  Outputs equal mm1_attn_bwd's
 * (default tilings) bitwise. */
int mm1_attn_bwd_noalloc(const void* o, const void* dO, const float* lse2,
                         const void* state, size_t state_bytes, void* dq, void* dk, void* dv,
                         int B, int S, int H, int Hkv, int D, int causal, float sm_scale, void* stream);
size_t mm1_attn_bwd_noalloc_scratch_size(int B, int S, int H, int Hkv, int D, int causal);

/* The stages of the backward, for callers that schedule or time them
 * separately (same checks as mm1_attn_bwd).  mm1_attn_bwd runs
 * mm1_attn_bwd_prep, mm1_attn_bwd_dkdv_tiles, mm1_attn_bwd_dq_reduce_tiles;
 * mm1_attn_bwd_dq_tiles and mm1_attn_bwd_dkdv_reduce_tiles split the last
 * one into two launches (same results).
 *  - mm1_attn_bwd_prep: Delta from o and the state, fp16 dO and its scale,
 *    and lse2 - log2(sm_scale), into `workspace`.  mm1_attn_bwd_prep_delta
 *    takes the caller's delta instead of o (a state from mm1_attn_prep has
 *    no O residual).  The calls below read what a prep call wrote into the
 *    same workspace (lse2 included); the library cannot check that one did.
 *  - mm1_attn_bwd_dkdv_tiles: dK/dV.  With H == Hkv it writes bf16 dk, dv
 *    directly.  Otherwise, with the per-head tiling (1) it writes the
 *    per-query-head fp32 partial sums into `workspace` and leaves dk/dv
 *    untouched; with the grouped tiling (0) it writes bf16 dk, dv directly
 *    for the key tiles one workgroup covers and fp32 partials (one slot per
 *    chunk, see mm1_attn_dkdv_plan) for the others.
 *  - mm1_attn_bwd_dkdv_reduce_tiles: sums the partials of each KV head and
 *    writes bf16 dk, dv (no-op when H == Hkv).  It must name the dK/dV
 *    tiling of the mm1_attn_bwd_dkdv_tiles call that filled the workspace,
 *    with the same shape and `causal`: the library records, per workspace
 *    address, the layout that call wrote, and the summing calls return
 *    MM1_E_LAYOUT (launching nothing) when the record is missing or
 *    differs.  The record is keyed by address only: a workspace freed and
 *    reallocated at the same address (as a caching allocator does) with no
 *    dK/dV call since passes the check, and the sum then reads whatever the
 *    memory holds.  The same holds for mm1_attn_bwd_dq_reduce_tiles.
 *  - mm1_attn_bwd_dq_tiles: bf16 dq.
 *  - mm1_attn_bwd_dq_reduce_tiles: bf16 dq, and the group sum of
 *    mm1_attn_bwd_dkdv_reduce_tiles done by the tail of the same launch (must
 *    run after mm1_attn_bwd_dkdv_tiles on the same stream).
 * Tiling arguments index mm1_attn_tile_desc (-1 = the default).  Together
 * they replace flash_delta + flash_bwd + flash_unswizzle + casts
 * (attention_tilelang.py:192-323, :380-389); no counterpart as separate
 * calls. */
int mm1_attn_bwd_prep(const void* o, const void* dO, const float* lse2, const void* state, size_t state_bytes,
                      void* workspace, size_t workspace_bytes,
                      int B, int S, int H, int Hkv, int D, float sm_scale, void* stream);
int mm1_attn_bwd_prep_delta(const void* dO, const float* delta, const float* lse2, const void* state,
                            size_t state_bytes, void* workspace, size_t workspace_bytes,
                            int B, int S, int H, int Hkv, int D, float sm_scale, void* stream);
int mm1_attn_bwd_dkdv_tiles(const void* state, size_t state_bytes, void* dk, void* dv,
                            void* workspace, size_t workspace_bytes,
                            int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                            int dkdv_tiles, void* stream);
int mm1_attn_bwd_dkdv_reduce_tiles(void* workspace, size_t workspace_bytes, void* dk, void* dv,
                                   int B, int S, int H, int Hkv, int D, int causal, int dkdv_tiles,
                                   void* stream);
int mm1_attn_bwd_dq_tiles(const void* state, size_t state_bytes, void* dq,
                          void* workspace, size_t workspace_bytes,
                          int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                          int dq_tiles, void* stream);
int mm1_attn_bwd_dq_reduce_tiles(const void* state, size_t state_bytes,
                                 void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                                 int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                                 int dkdv_tiles, int dq_tiles, void* stream);

/* mm1_attn_bwd with an explicit tiling: what a tuned kernel handle
 * launches (-1 = the default of mm1_attn_bwd; MM1_E_TILES for an index out
 * of range). */
int mm1_attn_bwd_tiles(const void* o, const void* dO, const float* lse2,
                       const void* state, size_t state_bytes,
                       void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                       int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                       int dkdv_tiles, int dq_tiles, void* stream);

/* The backward with fp32 gradients: dq, dk, dv as fp32 [B,S,H,D] /
 * [B,S,Hkv,D], the values mm1_attn_bwd_tiles with the same tilings rounds to
 * bf16 (same kernels, same summation order).  Replaces the fp32 dQ / dK / dV
 * buffers that get_kernel("bwd", ...) fills (attention_tilelang.py:258-260,
 * :381-387) before flash_unswizzle and the casts: a caller that wants the
 * unrounded gradients (a parity check, an fp32 master-gradient path) uses
 * it. */
int mm1_attn_bwd_f32_tiles(const void* o, const void* dO, const float* lse2,
                           const void* state, size_t state_bytes,
                           float* dq, float* dk, float* dv, void* workspace, size_t workspace_bytes,
                           int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                           int dkdv_tiles, int dq_tiles, void* stream);

/* Tilings compiled into the library.  The reference autotunes each TileLang
 * kernel over a space of (block_M, block_N, threads, num_stages)
 * (attention_tilelang.py:61-98) and remembers the winner per (device, kernel,
 * shape) (get_kernel, :329-346; CODE/mimans/model/tuned.py:59-74); here the
 * space is the fixed set of gfx950 tilings built into this library, all with
 * the same results up to fp32 summation order.
 *  - mm1_attn_tile_count(kind): number of tilings of MM1_TILES_FWD,
 *    MM1_TILES_DKDV or MM1_TILES_DQ (0 for another kind);
 *  - mm1_attn_tile_desc(kind, i): static "key=value ..." description of
 *    tiling i (block_M, block_N, waves, stages, schedule), NULL if out of range.
 * Index 0 is each kind's default, which the calls without a tiling argument
 * use. */
int mm1_attn_tile_count(int kind);
const char* mm1_attn_tile_desc(int kind, int index);

/* mm1_attn_fwd with an explicit tiling (-1 = the default; MM1_E_TILES for an
 * index out of range): what a tuned kernel handle launches. */
int mm1_attn_fwd_tiles(const void* q, const void* k, const void* v, void* o, float* lse2,
                       void* state, size_t state_bytes,
                       int B, int S, int H, int Hkv, int D, int causal, float sm_scale,
                       int tiles, void* stream);

/* Workgroup dispatch order of a causal grid (diagnostic; no counterpart in
 * the reference, whose TileLang grids run in launch order).  The causal
 * forward and dQ launches with one workgroup per CU do not run their row
 * blocks in the default longest-first order: gfx950 deals launch slot b to
 * XCD b % 8 and, inside an XCD, its k-th workgroup to shader engine k % 4,
 * waiting in order for a free CU there; the library deals each XCD's row
 * blocks to the 4 SE lanes, packs each lane into its CUs in bins of equal
 * modelled work and lists the blocks in the order the CUs ask for them.
 * This call returns the table a launch of grid `kind` (MM1_TILES_FWD,
 * MM1_TILES_DQ, or MM1_TILES_DKDV with the grouped tiling 0) with tiling
 * `tiles` builds for a device with `cus` compute units: entry b is the work
 * item of launch slot b in the default numbering (0xFFFF for a slot without
 * one).  Writes min(n, cap) entries and returns n, the launch's grid size; 0
 * when the launch uses the default order (the per-head dK/dV tiling,
 * causal == 0 for the forward / dQ, a tiling with two workgroups per CU,
 * more items than the table holds, no modelled gain, or MM1_DISPATCH_ORDER=0
 * in the environment, read per call); a negative MM1_E_* code for bad
 * arguments.  Runs on the host only. */
int mm1_attn_dispatch_order(int kind, int tiles, int B, int S, int H, int Hkv, int causal, int cus,
                            unsigned short* out, int cap);

/* Work plan of the grouped dK/dV tiling (MM1_TILES_DKDV tiling 0; diagnostic,
 * no counterpart in the reference).  A workgroup of that launch owns one
 * 128-key tile of one (batch, KV head) and walks the 32-query tiles of all
 * G = H / Hkv query heads of the group, so K and V are read once per group
 * and the sum over the group's heads stays in registers.  Key tile kt meets
 * len = G * ceil((S - q0) / 32) query tiles (q0 = 128 * kt when causal, else
 * 0), split into nc = min(C, max(1, ceil(len / L))) chunks; chunk c walks
 * tiles c, c + nc, c + 2 * nc, ... < len of the position-major walk
 * (position tiles from the sequence end down, the G heads of each in turn).  L is the candidate chunk length whose workgroup order
 * the library's dispatch model rates fastest for `cus` compute units.
 * Writes out[0..4] = L, C, split_keys (keys [0, split_keys) of each batch lie
 * in key tiles with more than one chunk), the number of items in the default
 * numbering (n_kt * C * B * Hkv, item j = (kt * C + c) * B * Hkv + b * Hkv + g)
 * and the launch's table size (0: default order).  Runs on the host only. */
int mm1_attn_dkdv_plan(int B, int S, int H, int Hkv, int causal, int cus, int* out);

/* QK-RMSNorm + RoPE between the fused QKV projection and the attention
 * kernel.  Replaces, in Attention.forward (attention_tilelang.py:483-487), the
 * views of wq/wk/wv outputs, q_norm/k_norm (RMSNorm.forward, :423-428) and
 * apply_rope (:458-461) on Q and K, plus the .contiguous() copies (:492-493).
 *  - qkv: [B, S, (H + 2*Hkv) * D] bf16, columns = wq | wk | wv outputs;
 *  - wq, wk: the norm weights [D] fp32, or both NULL for qk_norm = False;
 *  - cos_t, sin_t: the Rotary tables [rot_len, D] fp32 (rot_len >= S);
 *  - q [B,S,H,D], k, v [B,S,Hkv,D] bf16 out (v is the copied value slice).
 * Numerics: the norm in fp32 rounded to bf16, the rotation in bf16 steps, as
 * the reference under bf16. */
int mm1_qknorm_rope_fwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                        const float* sin_t, void* q, void* k, void* v,
                        int B, int S, int H, int Hkv, int D, int rot_len, float eps, void* stream);

/* Backward of mm1_qknorm_rope_fwd: given dq, dk, dv (bf16, the attention
 * backward's outputs) writes dqkv [B, S, (H + 2*Hkv) * D] bf16 and, with the
 * norm, the weight gradients dwq, dwk [D] fp32 (deterministic two-stage sum;
 * needs a workspace of mm1_qknorm_rope_bwd_workspace_size() bytes).  Replaces
 * autograd through :423-428 and :458-461; no counterpart as a separate call. */
size_t mm1_qknorm_rope_bwd_workspace_size(void);
int mm1_qknorm_rope_bwd(const void* qkv, const float* wq, const float* wk, const float* cos_t,
                        const float* sin_t, const void* dq, const void* dk, const void* dv,
                        void* dqkv, float* dwq, float* dwk, void* workspace, size_t workspace_bytes,
                        int B, int S, int H, int Hkv, int D, int rot_len, float eps, void* stream);

/* Static description of a return code. */
const char* mm1_attn_strerror(int code);

#ifdef __cplusplus
}
#endif

#endif /* MM1_ATTN_H */
