/*
 * fattn.h -- the C ABI of the MI355X (gfx950) fused fp32 scaled-dot-product attention,
 * forward and deterministic backward, head_dim 32, 64 or 128.
 *
 * This is the drop-in boundary for the reference crate's hot path
 * (mi-for-the-rust-of-us/candle-fused-attn v0.4.0), whose kernels take head_dim 64 (32 and 128
 * are on its roadmap, ROADMAP.md:76-79). Each entry point names the reference interface it
 * replaces (path:line in that crate). Two levels are exported:
 *
 *   - kernel level (replaces the launcher src/cuda.rs and the three kernels of
 *     kernels/fused_attn.cu): operands are [b, h, s, d] views given by a base pointer (the
 *     view's first element) and (batch, head, seq) strides in floats, head_dim contiguous. The
 *     `fattn_*_f32` entries take any supported d; the `fattn_*_f32_d64` entries, named after the
 *     reference's kernels, are the same with the reference's check (d must be 64);
 *   - op level (replaces the candle custom ops' device bodies in src/lib.rs): operands are given
 *     as a storage pointer, an element offset, a shape and strides, exactly what a candle
 *     `Layout` holds, and the geometry, shape and alignment checks of src/lib.rs run here.
 *
 * Conventions (all entry points):
 *   - no torch, candle or HIP types in the signatures: `stream` is a hipStream_t passed as
 *     `void*` (NULL = the null stream);
 *   - every launch is asynchronous on `stream`; nothing here synchronises the stream, except
 *     fattn_bwd_status, which says so;
 *   - outputs are fully written, so they may be uninitialised; nothing is allocated: the
 *     caller owns O, L, dqkv and the backward workspace;
 *   - return 0 on success, a negative FATTN_E* code for a rejected argument (nothing is
 *     launched), or a positive hipError_t for a runtime failure; fattn_last_error() then holds
 *     a message of this thread prefixed like the reference's (`fused_attention:` or
 *     `fused_attention_qkv:`);
 *   - empty inputs (batch, heads or seq 0) are a successful no-op (empty outputs);
 *   - all arithmetic is fp32; backward results are bit-identical from run to run.
 */
#ifndef FATTN_H
#define FATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The reference's head dimension (src/lib.rs:91, CUDA_HEAD_DIM); the kernels here are also
 * built for FATTN_HEAD_DIM_MIN (32) and FATTN_HEAD_DIM_MAX (128). */
#define FATTN_HEAD_DIM 64
#define FATTN_HEAD_DIM_MIN 32
#define FATTN_HEAD_DIM_MAX 128

/* Validation failures (negative return codes). */
#define FATTN_EINVAL (-1)     /* null pointer, bad rank/shape, non-contiguous last dim, ... */
#define FATTN_EHEADDIM (-2)   /* head_dim not built (src/cuda.rs:85-93: the reference's is 64) */
#define FATTN_EALIGN (-3)     /* a row is not 16-byte aligned (src/lib.rs:431-435, :533-538) */
#define FATTN_ERANGE (-4)     /* a size exceeds the kernels' index or grid range */
#define FATTN_EWORKSPACE (-5) /* workspace missing, too small or misaligned */

/* ------------------------------------------------------------------------------------------
 * Kernel level. Replaces src/cuda.rs (forward :139-185, backward :187-260) and the kernels
 * fattn_fwd_f32_d64 (kernels/fused_attn.cu:469-598), fattn_bwd_dot_f32_d64 (:45-63) and
 * fattn_bwd_f32_d64 (:213-426). Strides are {batch, head, seq} in floats.
 * ------------------------------------------------------------------------------------------ */

/* Forward: O [b, s, h, d] contiguous (the merge-heads layout) and L [b, h, s], the row
 * log-sum-exp the backward needs. Replaces cuda::forward (src/cuda.rs:139-185). */
int fattn_fwd_f32(const float* q, const float* k, const float* v, float* o, float* lse,
                  int64_t b, int64_t h, int64_t s, int64_t d, float scale, int causal,
                  const int64_t q_strides[3], const int64_t k_strides[3],
                  const int64_t v_strides[3], void* stream);

/* Backward workspace (256-byte aligned). Replaces the temporaries cuda::backward allocates
 * (dsum and turn, src/cuda.rs:200-209). Its size picks how dQ is summed over key blocks:
 *   >= fattn_bwd_workspace_split_bytes: "split" -- every key block writes its dQ partials to the
 *      workspace (about s * s * b * h * d / 16 bytes); they are summed in key-block order by the
 *      last workgroups of step 2 (which wait, boundedly, only for key blocks dispatched before
 *      them) or by a third kernel; no key block waits on another (the faster way);
 *   below that, d <= 64, in fattn_bwd_f32 and the op-level backwards: "split by chunks" when the
 *      workspace holds the split state of enough (b, h) pairs for a chunk to fill the chip (a
 *      chunk of c pairs needs fattn_bwd_workspace_split_bytes(1, c, s, d)) -- steps 2 and 3 run
 *      per chunk of pairs, with the same results as the whole split, bit for bit;
 *   >= fattn_bwd_workspace_min_bytes, otherwise: "turns" -- key blocks add into dQ in place,
 *      in key-block order, under per-query-tile turn counters; D, counters and ticket only.
 * All are deterministic. fattn_bwd_workspace_bytes is the split size when that is at most
 * FATTN_SPLIT_MAX_BYTES, else the split of the largest worthwhile chunk within it (d <= 64),
 * else the minimum. All three return 0 for a negative size or an unsupported d. */
#define FATTN_SPLIT_MAX_BYTES ((size_t)4 << 30)
size_t fattn_bwd_workspace_bytes(int64_t b, int64_t h, int64_t s, int64_t d);
size_t fattn_bwd_workspace_min_bytes(int64_t b, int64_t h, int64_t s, int64_t d);
size_t fattn_bwd_workspace_split_bytes(int64_t b, int64_t h, int64_t s, int64_t d);

/* Backward step 1: D[b, h, i] = sum_c dO[b, i, h, c] * O[b, i, h, c] (fixed order) and the
 * counters of step 2 cleared. O is [b, s, h, d] contiguous; dO is read through do_strides. With
 * a split-size workspace at d <= 64, and at d 128 with s <= 256, there is nothing to do (step 2
 * computes D itself, and tags the state of its own dQ sums with a value unique to its launch;
 * returns 0 after the checks).
 * Replaces the fattn_bwd_dot_f32_d64 launch (src/cuda.rs:215-231). */
int fattn_bwd_prep_f32(const float* o, const float* d_o, const int64_t do_strides[3],
                       void* workspace, size_t workspace_bytes, int64_t b, int64_t h, int64_t s,
                       int64_t d, void* stream);

/* Backward step 2: dK and dV into ONE [b, s, 3, h, d] buffer (the fused qkv projection's
 * gradient layout); dQ summed over key blocks in a fixed order, so every rerun is bit-identical:
 * with a split-size workspace its partials go to the workspace (this step sums some query
 * tiles, step 3 the rest) and, for d <= 64, D is computed here from O (the forward's
 * [b, s, h, d] output); else dQ is complete after this step. Where D is not computed here it
 * comes from step 1, which must run first on the same workspace (running step 1 first is always
 * correct). Replaces the fattn_bwd_f32_d64 launch (src/cuda.rs:233-258), which takes no O. */
int fattn_bwd_main_f32(const float* q, const float* k, const float* v, const float* o,
                       const float* d_o, const float* lse, float* dqkv, void* workspace,
                       size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                       float scale, int causal, const int64_t q_strides[3],
                       const int64_t k_strides[3], const int64_t v_strides[3],
                       const int64_t do_strides[3], void* stream);

/* Backward step 3: with a split-size workspace, dQ = scale * (sum of step 2's partials in
 * key-block order) into part 0 of dqkv, for every query tile the last step 2 launch on this
 * workspace did not sum itself (its last workgroups sum the tiles the schedule gives them; the
 * same operations in the same order, so the result does not depend on which kernel summed a
 * tile), then it clears the sums' flags; with a smaller workspace nothing to do (returns 0). Has
 * no counterpart launch in the reference (its dQ is summed in place, as the turn mode here). */
int fattn_bwd_dq_f32(float* dqkv, void* workspace, size_t workspace_bytes, int64_t b, int64_t h,
                     int64_t s, int64_t d, float scale, int causal, void* stream);

/* All backward steps. Replaces cuda::backward (src/cuda.rs:187-260). Step 3 is launched only
 * where step 2 has no dQ sums, or while `stream` is capturing a HIP graph. */
int fattn_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                  const float* d_o, const float* lse, float* dqkv, void* workspace,
                  size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                  float scale, int causal, const int64_t q_strides[3],
                  const int64_t k_strides[3], const int64_t v_strides[3],
                  const int64_t do_strides[3], void* stream);

/* fattn_bwd_f32 without the workspace argument, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It has no
 * counterpart in the reference. It calls no allocating routine: the workspace is the library's
 * static scratch, FATTN_STATIC_SCRATCH_BYTES of device memory per GPU, held until the process
 * ends. dQ is summed as fattn_bwd_f32 sums it with a workspace of that size (the same kernels
 * and results): the split way when its workspace fits in the scratch, else at d <= 64 split by
 * chunks of (b, h) pairs where such chunks fit and fill the chip, else by turns; a shape whose minimum
 * workspace exceeds the scratch is refused with FATTN_EWORKSPACE before any launch. Every call on
 * one GPU shares that GPU's scratch: calls that overlap on one GPU (two streams, two threads)
 * race and must be ordered by the caller. */
#define FATTN_STATIC_SCRATCH_BYTES ((size_t)64 << 20)
int fattn_bwd_f32_noalloc(const float* q, const float* k, const float* v, const float* o,
                          const float* d_o, const float* lse, float* dqkv, int64_t b, int64_t h,
                          int64_t s, int64_t d, float scale, int causal,
                          const int64_t q_strides[3], const int64_t k_strides[3],
                          const int64_t v_strides[3], const int64_t do_strides[3], void* stream);

/* The same five under the reference's kernel names, with its head_dim check (d must be 64,
 * else FATTN_EHEADDIM with the reference's message, src/cuda.rs:85-93). */
int fattn_fwd_f32_d64(const float* q, const float* k, const float* v, float* o, float* lse,
                      int64_t b, int64_t h, int64_t s, int64_t d, float scale, int causal,
                      const int64_t q_strides[3], const int64_t k_strides[3],
                      const int64_t v_strides[3], void* stream);
int fattn_bwd_prep_f32_d64(const float* o, const float* d_o, const int64_t do_strides[3],
                           void* workspace, size_t workspace_bytes, int64_t b, int64_t h,
                           int64_t s, int64_t d, void* stream);
int fattn_bwd_main_f32_d64(const float* q, const float* k, const float* v, const float* o,
                           const float* d_o, const float* lse, float* dqkv, void* workspace,
                           size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                           float scale, int causal, const int64_t q_strides[3],
                           const int64_t k_strides[3], const int64_t v_strides[3],
                           const int64_t do_strides[3], void* stream);
int fattn_bwd_dq_f32_d64(float* dqkv, void* workspace, size_t workspace_bytes, int64_t b,
                         int64_t h, int64_t s, int64_t d, float scale, int causal, void* stream);
int fattn_bwd_f32_d64(const float* q, const float* k, const float* v, const float* o,
                      const float* d_o, const float* lse, float* dqkv, void* workspace,
                      size_t workspace_bytes, int64_t b, int64_t h, int64_t s, int64_t d,
                      float scale, int causal, const int64_t q_strides[3],
                      const int64_t k_strides[3], const int64_t v_strides[3],
                      const int64_t do_strides[3], void* stream);

/* ------------------------------------------------------------------------------------------
 * Op level: the candle custom ops' device bodies. A tensor is (storage, offset, shape,
 * strides), offset and strides in elements, as in a candle Layout.
 * ------------------------------------------------------------------------------------------ */

/* softmax(q k^T scale [+ causal mask]) v from a fused [b, s, 3 h d] projection laid out
 * [q | k | v] along the last dim. out: [b, s, h d] contiguous; lse: [b, h, s] contiguous.
 * Replaces FusedAttentionQkv::cuda_fwd (src/lib.rs:526-550) with qkv_geometry
 * (src/lib.rs:191-206). */
int fattn_qkv_forward(const float* qkv, int64_t offset, const int64_t shape[3],
                      const int64_t strides[3], int64_t heads, float scale, int causal,
                      float* out, float* lse, void* stream);

/* The gradient of the projection: dqkv [b, s, 3 h d] contiguous, from the forward's out and
 * lse and the output gradient grad [b, s, h d] (grad_strides, last one 1). Replaces
 * FusedAttentionQkv::bwd (src/lib.rs:554-579) and cuda_backward (src/lib.rs:329-366). */
int fattn_qkv_backward(const float* qkv, int64_t offset, const int64_t shape[3],
                       const int64_t strides[3], int64_t heads, float scale, int causal,
                       const float* out, const float* lse, const float* grad,
                       int64_t grad_offset, const int64_t grad_shape[3],
                       const int64_t grad_strides[3], float* dqkv, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Attention over [b, h, s, d] q, k, v with any strides (d contiguous, rows 16-byte aligned).
 * out: [b, s, h, d] contiguous (the caller's [b, h, s, d] result is its transposed view);
 * lse: [b, h, s]. Replaces FusedAttention::cuda_fwd (src/lib.rs:420-447) with check_shapes
 * and bhs_strides (src/lib.rs:181-220). */
int fattn_forward(const float* q, int64_t q_offset, const int64_t q_shape[4],
                  const int64_t q_strides[4], const float* k, int64_t k_offset,
                  const int64_t k_shape[4], const int64_t k_strides[4], const float* v,
                  int64_t v_offset, const int64_t v_shape[4], const int64_t v_strides[4],
                  float scale, int causal, float* out, float* lse, void* stream);

/* dQ, dK, dV into one [b, s, 3, h, d] buffer (the caller narrows and transposes it to three
 * [b, h, s, d] views), from the gradient of the [b, s, h, d] output (grad_shape/grad_strides
 * in that order). Replaces FusedAttention::bwd (src/lib.rs:449-490). */
int fattn_backward(const float* q, int64_t q_offset, const int64_t q_shape[4],
                   const int64_t q_strides[4], const float* k, int64_t k_offset,
                   const int64_t k_shape[4], const int64_t k_strides[4], const float* v,
                   int64_t v_offset, const int64_t v_shape[4], const int64_t v_strides[4],
                   float scale, int causal, const float* out, const float* lse,
                   const float* grad, int64_t grad_offset, const int64_t grad_shape[4],
                   const int64_t grad_strides[4], float* dqkv, void* workspace,
                   size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Diagnostics (no counterpart in the reference).
 * ------------------------------------------------------------------------------------------ */

/* The message of this thread's last failed call ("" if none). */
const char* fattn_last_error(void);

/* Library version string. */
const char* fattn_version(void);

/* Synchronises `stream`, then reads the backward's guard word from `workspace` into *status:
 * 0 = every dQ wait ended normally; nonzero = results are invalid: 1, a turn wait of the turn
 * hand-over hit its spin bound; 2, a ticket out of range (step 1 did not run on this
 * workspace); 3, a dQ sum of step 2 with no step 3 after it gave up waiting (the dQ rows
 * concerned hold NaN). For tests and debugging; any head_dim. */
int fattn_bwd_status(const void* workspace, size_t workspace_bytes, int64_t b, int64_t h,
                     int64_t s, void* stream, int* status);

#ifdef __cplusplus
}
#endif

#endif /* FATTN_H */
