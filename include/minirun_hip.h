/*
 * minirun_hip.h -- C-ABI of the MI355X (gfx950) MLA attention path.
 *
 * A drop-in for the MLX calls that Minirun's attention hot path makes.  Each
 * entry point names the reference interface it replaces (paths relative to
 * the nanguoyu/minirun-app tree).  The Swift side binds this header through a
 * module map (a HIPBridge module shaped like MLXBridge); INTEGRATION.md shows
 * that binding.
 *
 * Conventions
 *  - Every tensor is caller-owned device memory, passed as a plain pointer
 *    plus sizes and element strides.  bf16/f16 tensors are 16-bit patterns.
 *  - `stream` is a hipStream_t (NULL = the default stream).  Work is enqueued
 *    with no implicit synchronisation, except where an entry point says it
 *    synchronises (index validation).
 *  - Functions return mr_status and never abort.  mr_get_last_error() gives a
 *    message for the last non-OK status on the calling thread.
 *  - No entry point allocates device memory: scratch comes in as a
 *    caller-provided workspace whose size a *_workspace_size function states.
 */
#ifndef MINIRUN_HIP_H
#define MINIRUN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mr_status {
    MR_OK = 0,
    MR_INVALID_SHAPE = 1,       /* AffineBridgeError.shapeMismatch/.wrongRank, DeepSeekV4Error geometry */
    MR_INVALID_DTYPE = 2,       /* AffineBridgeError.wrongPackedDType/.wrongScaleDType/.scaleBiasDTypeMismatch */
    MR_INDEX_OUT_OF_RANGE = 3,  /* "token t names KV row i, outside the cache" */
    MR_DUPLICATE_INDEX = 4,     /* "token t names KV row i more than once" */
    MR_NONFINITE = 5,           /* NaN score / non-finite rotary angle */
    MR_HIP_ERROR = 6,           /* a HIP runtime call failed */
    MR_INVALID_ARGUMENT = 7,    /* null pointer, misalignment, bad stride */
    MR_WORKSPACE_TOO_SMALL = 8
} mr_status;

typedef enum mr_dtype {
    MR_BF16 = 0,
    MR_F16 = 1,
    MR_F32 = 2,
    MR_U32 = 3,
    MR_I32 = 4
} mr_dtype;

/* Library version string, e.g. "minirun-hip 0.1.0 gfx950". */
const char *mr_version(void);

/* Message of the last non-OK status returned on this thread ("" if none). */
const char *mr_get_last_error(void);

/* ------------------------------------------------------------------------
 * Absorbed-latent MLA decode and index-driven sparse decode.
 *
 * Replaces the attention core of K3MLA.forwardWithoutTrace, absorbed branch
 * (Sources/ModelAdapters/Operators/MLA.swift:174-197: scores, fp32 softmax,
 * probs . latents), and DeepSeekV4SparseAttention.forward
 * (Sources/ModelAdapters/Operators/DeepSeekV4Attention.swift:747-770,
 * batched form :861-920) when `indices` is given.
 *
 *   s_n = (q_lat[b,h] . latent[n] + q_rope[b,h] . rope_key[n]) * scale
 *   out[b,h] = sum_n softmax(s (+ sink_h))_n * latent[n]        (width kv_rank)
 *
 * Rows: n ranges over [0, n_ctx) of batch element b, or over the valid
 * entries of indices[b, 0:n_idx] (-1 = skip, DeepSeekV4Attention.swift:884-895).
 * An index list with no valid entry gives zeros (:896-899).  The sink, when
 * given, enters the max and the denominator only (:908-913).
 *
 * Layout: the cache is one bf16 row per position; the latent part and the
 * shared rope key are given as two (pointer, row stride) pairs so that both
 * the packed [P, 576] row and the reference's two arrays [P,512] + [P,64]
 * (MLA.swift:28-36) are expressible.  kv_rank must be 512; rope_dim 64 or 0
 * (0 = the V4 form, K = V = row).  Strides are in elements, multiples of 8;
 * base pointers 16-byte aligned.
 * ------------------------------------------------------------------------ */
typedef struct mr_mla_decode_args {
    int32_t batch, heads, n_ctx, kv_rank, rope_dim;
    float scale; /* e.g. 1/sqrt(qk_nope + qk_rope), MLA.swift:170 */
    const void *q_lat; /* bf16 [batch, heads, kv_rank] */
    int64_t q_lat_batch_stride, q_lat_head_stride;
    const void *q_rope; /* bf16 [batch, heads, rope_dim]; NULL iff rope_dim == 0 */
    int64_t q_rope_batch_stride, q_rope_head_stride;
    const void *latent; /* bf16 rows, kv_rank wide */
    int64_t latent_row_stride, latent_batch_stride;
    const void *rope_keys; /* bf16 rows, rope_dim wide; NULL iff rope_dim == 0 */
    int64_t rope_row_stride, rope_batch_stride;
    const int32_t *indices; /* optional int32 [batch, n_idx] */
    int32_t n_idx;
    const float *sinks; /* optional f32 [heads] */
    void *out;          /* [batch, heads, kv_rank] */
    mr_dtype out_dtype; /* MR_BF16 or MR_F32 */
    int64_t out_batch_stride, out_head_stride;
    void *workspace; /* device scratch, >= mr_mla_decode_workspace_size() bytes */
    size_t workspace_bytes;
    int32_t num_splits; /* 0 = choose; otherwise context splits per batch element */
    uint32_t flags;     /* MR_DECODE_* */
    /* Optional phase-accounting hook (the reference brackets this op as
     * sparseAttentionSeconds, DeepSeekV4Attention.swift:757-760): NULL, or
     * three hipEvent_t recorded on `stream` before the split kernel, between
     * it and the combine kernel, and after the combine kernel. */
    void *const *phase_events;
} mr_mla_decode_args;

#define MR_DECODE_VALIDATE_INDICES 1u  /* run mr_validate_indices first (synchronises) */
#define MR_DECODE_NO_TRANSPOSE_READ 2u /* debug: PV operand by scalar LDS reads */

size_t mr_mla_decode_workspace_size(const mr_mla_decode_args *args);
mr_status mr_mla_decode(const mr_mla_decode_args *args, void *stream);

/* Index validation with the reference's rules and error order
 * (DeepSeekV4Attention.swift:884-895): per token b in order, per entry in
 * order, -1 skips, an entry outside [0, n_rows) is INDEX_OUT_OF_RANGE, a
 * repeat of an earlier entry is DUPLICATE_INDEX.  Synchronises `stream`.
 * bad_token / bad_position (optional host pointers) receive the location.
 * Needs n_idx <= 4096 and a workspace of mr_validate_indices_workspace_size. */
size_t mr_validate_indices_workspace_size(int32_t batch, int32_t n_idx);
mr_status mr_validate_indices(const int32_t *indices, int32_t batch, int32_t n_idx,
                              int32_t n_rows, void *workspace, size_t workspace_bytes,
                              int32_t *bad_token, int32_t *bad_position, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MINIRUN_HIP_H */
