/*
 * minirun_hip.h -- C-ABI of the MI355X (gfx950) MLA attention path.
 *
 * A drop-in for the MLX calls that Minirun's attention hot path makes.  Each
 * entry point names the reference interface it replaces (paths relative to
 * the nanguoyu/minirun-app tree).  The Swift side binds this header through a
 * module map (a HIPBridge module shaped like MLXBridge); every declaration
 * is plain C11.
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
 *    caller-provided workspace whose size a *_workspace_size function states
 *    (0 for arguments whose widths or counts the entry point rejects, and
 *    for layouts of 2^56 bytes or more, which the entry point refuses with
 *    MR_INVALID_SHAPE).
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
 * Index checks (the reference throws on an entry outside [0, n_ctx) other
 * than -1, and on a repeated entry, :884-895), chosen by the caller:
 *  - index_status != NULL: checked on the device in the same launch, no
 *    host synchronisation.  index_status[3*b .. 3*b+2] receives (MR_OK, -1,
 *    -1) for a valid list of token b, else (MR_INDEX_OUT_OF_RANGE or
 *    MR_DUPLICATE_INDEX, position, value) of the first bad entry in the
 *    reference's order.  `out` of a token whose list is bad is unspecified.
 *  - index_status == NULL (the default): the same check runs first and the
 *    call returns its error (synchronises `stream`), as the reference's
 *    throwing call does.  MR_DECODE_VALIDATE_INDICES asks for this form even
 *    when index_status is given.
 *  - MR_DECODE_UNCHECKED: no check; a bad entry is skipped like -1 and a
 *    repeated one counts once per occurrence.
 * Any list the call takes can be checked (n_idx is at most 524288): a list
 * of up to 10176 entries is checked in LDS, a longer one in a hash table in
 * the workspace (mr_mla_decode_workspace_size includes it).
 *
 * Layout: the cache is one bf16 row per position; the latent part and the
 * shared rope key are given as two (pointer, row stride) pairs so that both
 * the packed [P, 576] row and the reference's two arrays [P,512] + [P,64]
 * (MLA.swift:28-36) are expressible.  kv_rank 512 with rope_dim 64 or 0 (0 =
 * the V4 form, K = V = row) runs the split kernel: strides in elements,
 * multiples of 8; base pointers 16-byte aligned.  Other widths (kv_rank 1 ..
 * 2048, rope_dim 0 .. 512, e.g. the reference's synthetic K3 artifact,
 * kv_lora 16 / rope 4) run an any-width kernel in fp32 (no bf16 rounding of
 * P), one workgroup per (batch, head), elements read one by one: pointers
 * element-aligned, strides covering the rows; its workspace only holds the
 * index checks' words and tables.
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
    int32_t *index_status; /* optional device int32 [batch][3]: see the index checks above */
} mr_mla_decode_args;

#define MR_DECODE_VALIDATE_INDICES 1u /* check the indices first and return the error (synchronises) */
/* Profiling aid, no reference counterpart: launch only the split kernel
 * (the split partials land in the workspace; `out` is not written), so a
 * caller can time that kernel over many launches between two events. */
#define MR_DECODE_SPLIT_ONLY 4u
#define MR_DECODE_UNCHECKED 8u /* no index checks (trusted producers) */

size_t mr_mla_decode_workspace_size(const mr_mla_decode_args *args);
mr_status mr_mla_decode(const mr_mla_decode_args *args, void *stream);

/* mr_mla_decode with no workspace argument and no allocation.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The caller passes inputs and outputs;
 * args->workspace / workspace_bytes are ignored.  Scratch is a
 * library-owned device array of MR_DECODE_NOALLOC_SCRATCH_BYTES per GPU
 * (held until the process ends); a call needing more
 * (mr_mla_decode_workspace_size) returns MR_WORKSPACE_TOO_SMALL.  Index
 * lists need index_status or MR_DECODE_UNCHECKED (no synchronous check).
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (concurrent streams or threads) race and must be serialised by the
 * caller. */
#define MR_DECODE_NOALLOC_SCRATCH_BYTES (48u * 1024u * 1024u)
mr_status mr_mla_decode_noalloc(const mr_mla_decode_args *args, void *stream);

/* Index validation with the reference's rules and error order
 * (DeepSeekV4Attention.swift:884-895): per token b in order, per entry in
 * order, -1 skips, an entry outside [0, n_rows) is INDEX_OUT_OF_RANGE, a
 * repeat of an earlier entry is DUPLICATE_INDEX.  Synchronises `stream`.
 * bad_token / bad_position (optional host pointers) receive the location.
 * Needs n_idx <= 4194304 and a workspace of mr_validate_indices_workspace_size
 * (lists of more than 10176 entries keep their hash tables there). */
size_t mr_validate_indices_workspace_size(int32_t batch, int32_t n_idx);
mr_status mr_validate_indices(const int32_t *indices, int32_t batch, int32_t n_idx,
                              int32_t n_rows, void *workspace, size_t workspace_bytes,
                              int32_t *bad_token, int32_t *bad_position, void *stream);


/* ------------------------------------------------------------------------
 * MLX affine quantized weights (Sources/MLXBridge/AffineWeights.swift).
 *
 * packed: uint32 [experts?, out_features, in_features * bits / 32], element j
 * of a word at bit offset bits*j (element 0 in the low bits: the word's
 * little-endian byte image is the checkpoint stream, MXFP4Weights.swift:42-48);
 * scales, biases: [experts?, out_features, in_features / group] in one of
 * bf16 / f16 / f32; w = scale * q + bias.
 * ------------------------------------------------------------------------ */
typedef struct mr_affine_weight {
    const uint32_t *packed;
    const void *scales;
    const void *biases;
    mr_dtype scale_dtype;
    int64_t out_features, in_features;
    int32_t group, bits;
} mr_affine_weight;

/* AffineWeights.init validation (AffineWeights.swift:84-157), in the
 * reference's order and with its messages: packed dtype, scale dtype,
 * scale/bias dtype agreement, scale/bias shape agreement, rank 2 or 3,
 * bits dividing 32, positive group, expert count, row count, in_features a
 * multiple of the group, group count.  Shapes are given as rank + dims.
 * On success fills the geometry (experts = 0 for a single matrix). */
mr_status mr_affine_validate(mr_dtype packed_dtype, int32_t packed_rank, const int64_t *packed_shape,
                             mr_dtype scales_dtype, int32_t scales_rank, const int64_t *scales_shape,
                             mr_dtype biases_dtype, int32_t biases_rank, const int64_t *biases_shape,
                             int32_t group, int32_t bits, int64_t *experts, int64_t *out_features,
                             int64_t *in_features);

/* AffineWeights.adopting (AffineWeights.swift:159-198): ownership of three
 * caller buffers (packed uint32, scales, biases: device memory, or pinned
 * host memory the device reads, such as the sub-regions of one StorageCore
 * slot) passes to an adopted weight, each buffer with its own finalizer.
 * Shapes follow the reference: packed [experts?, out, in * bits / 32],
 * scales and biases [experts?, out, in / group] (experts 0: no expert axis),
 * checked as mr_affine_validate checks them.
 * As in the reference, the finalizers own the buffers from the call on:
 * each runs exactly once, when the last reference to the weight is dropped
 * and the GPU work that reads it has completed.  A failing call drops the
 * weight at once, so all three have run when it returns its error.  They run
 * on a HIP runtime thread or on the releasing thread and must not call HIP
 * (the reference's release a buffer-pool lease, BufferPool.swift:45-90). */
typedef void (*mr_finalizer)(void *context);
typedef struct mr_adopted_affine mr_adopted_affine; /* opaque */
mr_status mr_affine_adopt(void *packed, void *scales, void *biases, mr_dtype scale_dtype, int64_t experts,
                          int64_t out_features, int64_t in_features, int32_t group, int32_t bits,
                          mr_finalizer packed_finalizer, void *packed_context, mr_finalizer scales_finalizer,
                          void *scales_context, mr_finalizer biases_finalizer, void *biases_context,
                          mr_adopted_affine **out);
/* The adopted weight as a descriptor for mr_affine_matmul and the others (a
 * view: valid while a reference is held). */
mr_status mr_adopted_affine_weight(const mr_adopted_affine *a, mr_affine_weight *out);
/* One more reference (another holder of the AffineWeights value), from any thread. */
mr_status mr_adopted_affine_retain(mr_adopted_affine *a);
/* Drops one reference, from any thread.  Dropping the last one enqueues the
 * finalizers on `stream` (NULL: the default stream, as in every other entry
 * point) behind the work already there, which must include every read of
 * the weight (order reads on other streams before it with an event).  The
 * handle is invalid after its last release: later calls with it return
 * MR_INVALID_ARGUMENT (unless a later adoption happens to reuse its address). */
mr_status mr_adopted_affine_release(mr_adopted_affine *a, void *stream);
/* Drops one reference; the last one runs the finalizers before the call
 * returns, on the calling thread.  For a weight no GPU work reads any more
 * (no counterpart in the reference, where the last holder's deinit decides;
 * here the caller states that no stream still reads the buffers). */
mr_status mr_adopted_affine_release_now(mr_adopted_affine *a);

/* affineDequantize (AffineWeights.swift:328-342): dense [out, in] in f32
 * (default, bit-exact: the bf16/f16-scale product is exact in fp32) or
 * bf16 (round-to-nearest-even of the f32 value). */
mr_status mr_affine_dequantize(const mr_affine_weight *w, void *out, mr_dtype out_dtype, void *stream);

/* affineMM (AffineWeights.swift:239-254): y[t, :] = x[t, :] . dequant(W)^T,
 * transpose fixed (W is [out, in]).  x: [tokens, in] bf16 or f32 with row
 * stride x_stride; y: [tokens, out] bf16 or f32 with row stride y_stride;
 * fp32 accumulation.  4-bit / group-64 / bf16 x / one token runs the fused
 * dequant-GEMV; 64 or more bf16 tokens of a 4-bit weight whose group is a
 * multiple of 32 (in_features a multiple of 32, out_features of 8, 16-byte
 * aligned x and y rows) run on MFMA: each k-tile dequantized into LDS and
 * split into two bf16 operands (hi = bf16(w), lo = bf16(w - hi)), so each
 * product misses x * w by at most 2^-18 |w|; other shapes run a generic
 * kernel. */
mr_status mr_affine_matmul(const void *x, mr_dtype x_dtype, int32_t tokens, int64_t x_stride,
                           const mr_affine_weight *w, void *y, mr_dtype y_dtype, int64_t y_stride,
                           void *stream);

/* Fixed-buffer hand-off of a StorageCore affine tile (QuantizedTileContainer
 * .swift:219-343; layout rules :496-640): one slot holds [packed | scales |
 * biases] for `rows` output rows of `cols` inputs, each sub-region a whole
 * number of 16 KiB units, so each can be adopted as its own operand without
 * a copy.  mr_affine_tile_view fills an mr_affine_weight over the slot's
 * bytes (pinned host memory the device reads, or device memory) and the
 * slot size; the geometry errors are the container's.  mr_tile_upload
 * copies a slot from pinned host memory to device memory on the stream
 * (asynchronous; the host slot must stay alive until the stream reaches it). */
mr_status mr_affine_tile_view(const void *tile, int64_t rows, int64_t cols, int32_t group, int32_t bits,
                              mr_dtype scale_dtype, mr_affine_weight *out, int64_t *tile_bytes);
mr_status mr_tile_upload(void *device_dst, const void *pinned_src, int64_t bytes, void *stream);

/* affineGatherMM (AffineWeights.swift:255-318): routed experts,
 * y[t, j, :] = x[t, :] . dequant(W[rhs[t, j]])^T.  w describes one expert
 * (out_features x in_features) of a stack of `experts` laid out back to back
 * (packed [experts][out][in*bits/32], scales/biases [experts][out][in/group]);
 * rhs_indices: device int32 [tokens][experts_per_token], need not be sorted,
 * may repeat; y: [tokens][experts_per_token][out] bf16 or f32, dense.  The
 * reference's preconditions (a stacked weight, indices matching the token
 * count) return MR_INVALID_ARGUMENT with its message.  An expert id outside
 * [0, experts) yields a zero row (MLX leaves it undefined).  4-bit /
 * group-64 / bf16 x runs the fused dequant-GEMV per (token, slot). */
mr_status mr_affine_gather_matmul(const void *x, mr_dtype x_dtype, int32_t tokens, int64_t x_stride,
                                  const mr_affine_weight *w, int64_t experts, const int32_t *rhs_indices,
                                  int32_t experts_per_token, void *y, mr_dtype y_dtype, void *stream);

/* ------------------------------------------------------------------------
 * Dense projections: k3Linear (Sources/ModelAdapters/Operators/Linear.swift:
 * 47-57), y = x . W^T with W stored output-major [out_features, in_features]
 * (the checkpoint's orientation; no transpose flag).  W is bf16 or f32 with
 * a row stride in elements (a multiple of 8, 16-byte aligned rows).
 * ------------------------------------------------------------------------ */
typedef struct mr_dense_weight {
    const void *weight;
    mr_dtype dtype; /* MR_BF16 or MR_F32 */
    int64_t out_features, in_features, row_stride;
} mr_dense_weight;

/* y[t, :] = x[t, :] . W^T for `tokens` rows of x (bf16 or f32, row stride
 * x_stride) into y (bf16 or f32, row stride y_stride), fp32 accumulation.
 * 64 or more bf16 tokens with a bf16 weight (in_features a multiple of 64,
 * out_features of 8, 16-byte aligned rows) run as an MFMA GEMM in tiles of
 * 256 (or 128) tokens x 256 outputs; otherwise every weight byte is read
 * once per tile of up to 8 tokens. */
mr_status mr_linear(const void *x, mr_dtype x_dtype, int32_t tokens, int64_t x_stride, const mr_dense_weight *w,
                    void *y, mr_dtype y_dtype, int64_t y_stride, void *stream);

/* One projection in either storage, as K3Projection holds a dense or a
 * quantized weight (Linear.swift:20-49; here the quantized form is the MLX
 * affine one).  MR_PROJ_NONE marks an absent optional projection. */
typedef enum mr_proj_kind { MR_PROJ_NONE = 0, MR_PROJ_AFFINE = 1, MR_PROJ_DENSE = 2 } mr_proj_kind;
typedef struct mr_projection {
    mr_proj_kind kind;
    mr_affine_weight affine; /* MR_PROJ_AFFINE */
    mr_dense_weight dense;   /* MR_PROJ_DENSE */
} mr_projection;

/* K3Norm.rms (Sources/ModelAdapters/Operators/Normalization.swift:15-19):
 * out = weight * (x * rsqrt(mean(x^2) + eps)) per row, fp32 arithmetic. */
mr_status mr_rmsnorm(const void *x, mr_dtype x_dtype, int64_t rows, int32_t dim, int64_t x_stride,
                     const void *weight, mr_dtype w_dtype, float eps, void *out, mr_dtype out_dtype,
                     int64_t out_stride, void *stream);

/* DeepSeekV4RotaryParameters (DeepSeekV4Attention.swift:28-99), host side:
 * pair frequencies base^(-2i/dim) with the YaRN ramp when original_len > 0.
 * freqs_out has dim/2 doubles. */
mr_status mr_rope_frequencies(int32_t dim, int32_t original_len, double base, double factor,
                              double beta_fast, double beta_slow, double *freqs_out);
/* Host cos/sin tables [n_pos, half] (DeepSeekV4Attention.swift:126-149):
 * angle = (inverse ? -1 : 1) * position * freq in double, rounded to float. */
mr_status mr_rope_table(const int64_t *positions, int64_t n_pos, const double *freqs, int32_t half,
                        int32_t inverse, float *cos_out, float *sin_out);
/* DeepSeekV4Rotary.apply (DeepSeekV4Attention.swift:108-165), device, in
 * place: x [n_pos, inner, row_stride] (bf16 or f32), columns
 * [col0, col0 + dim) rotated as adjacent pairs with the device tables
 * cos_t / sin_t [n_pos, dim/2]. */
mr_status mr_rope_apply(void *x, mr_dtype dtype, int64_t n_pos, int64_t inner, int64_t row_stride,
                        int64_t col0, int32_t dim, const float *cos_t, const float *sin_t, void *stream);

/* Latent-cache append (K3MLA.forward, MLA.swift:142-157): for each of
 * `tokens` kv_a rows [kv_rank ++ rope_dim] (bf16 or f32), write
 * RMSNorm(latent) * norm_w as bf16 to latent[start_row + t] and the rope
 * key, rotated with cos_t/sin_t [tokens, rope_dim/2], to rope[start_row + t].
 * cos_t = sin_t = NULL stores the key unrotated (K3's NoPE, MLA.swift:5-13). */
mr_status mr_mla_cache_append(const void *kv, mr_dtype kv_dtype, int64_t kv_stride, int64_t tokens,
                              const void *norm_w, mr_dtype w_dtype, float eps, int32_t kv_rank,
                              int32_t rope_dim, const float *cos_t, const float *sin_t, void *latent,
                              int64_t latent_row_stride, void *rope, int64_t rope_row_stride,
                              int64_t start_row, void *stream);

/* Query absorption (MLA.swift:180-188): q_lat[h] = q_nope[h] . W_UK[h] with
 * W_UK the rows h*(nope+v) .. +nope of kv_b_proj [heads*(nope+v), kv_rank]
 * (kv_rank 512), affine 4-bit group 64 or dense.  q: bf16 heads of
 * q_head_stride elements, nope part first; q_lat: bf16 [heads, kv_rank]. */
mr_status mr_mla_absorb_query(const void *q, int64_t q_head_stride, int32_t heads, int32_t nope_dim,
                              int32_t v_dim, const mr_projection *kv_b, void *q_lat,
                              int64_t q_lat_head_stride, void *stream);

/* Value un-absorption (MLA.swift:196-197): out[h] = ctx[h] . W_UV[h]^T with
 * W_UV the rows h*(nope+v)+nope .. +v of kv_b (affine or dense); ctx bf16
 * [heads, kv_rank], out [heads, v_dim] bf16 or f32 (contiguous). */
mr_status mr_mla_unabsorb_values(const void *ctx, int64_t ctx_head_stride, int32_t heads, int32_t nope_dim,
                                 int32_t v_dim, const mr_projection *kv_b, void *out, mr_dtype out_dtype,
                                 void *stream);

/* ------------------------------------------------------------------------
 * One decode token through the whole MLA block, absorbed branch of
 * K3MLA.forwardWithoutTrace (MLA.swift:91-98 -> :124-229):
 *   h = RMSNorm(x) (input norm; skipped when input_norm_w is NULL: K3 applies
 *       input_layernorm before the block)
 *   q = q_b(RMSNorm(q_a(h)))  [heads, nope + rope]
 *   kv = kv_a(h) -> cache row `position` (mr_mla_cache_append)
 *   q_lat = absorb(q_nope, kv_b)
 *   ctx = mr_mla_decode over rows [0, position]   (append, then attend)
 *   merged = unabsorb(ctx, kv_b)                   [heads * v]
 *   out = o_proj(merged * sigmoid(g_proj(h)))      (gate when g_proj is given,
 *                                                   MLA.swift:209-211)
 * Rotary: with rope_cos/rope_sin (device [qk_rope_dim/2], the angle table at
 * `position`) the query's rope slice and the cached key are rotated
 * (DeepSeek-style MLA); with both NULL nothing is rotated (K3 is NoPE,
 * MLA.swift:5-13: the slice is carried through unrotated).
 * Each projection is affine (MLX 4-bit) or dense (k3Linear); K3's attention
 * weights are dense bf16.  All activations between the projections are bf16.
 * Every stage is enqueued on `stream`, in order (dense projections of the
 * input run as one launch; the cache append rides in the absorption launch).
 * ------------------------------------------------------------------------ */
typedef struct mr_mla_block_args {
    int32_t hidden, q_lora_rank, heads, qk_nope_dim, qk_rope_dim, v_head_dim, kv_rank;
    float eps, scale;
    const void *x; /* bf16 [hidden], one token */
    const void *input_norm_w, *q_a_norm_w, *kv_a_norm_w;
    mr_dtype norm_w_dtype; /* bf16 or f32, all three */
    mr_projection q_a, q_b, kv_a, kv_b, o_proj;
    mr_projection g_proj; /* MR_PROJ_NONE: no output gate */
    void *cache_latent; /* bf16 rows, kv_rank wide */
    int64_t latent_row_stride;
    void *cache_rope; /* bf16 rows, qk_rope_dim wide */
    int64_t rope_row_stride;
    int32_t position, capacity; /* rows cached before this token; rows available */
    const float *rope_cos, *rope_sin; /* device [qk_rope_dim/2] at `position`, or both NULL (NoPE) */
    void *out; /* bf16 [hidden] */
    void *workspace;
    size_t workspace_bytes;
} mr_mla_block_args;

size_t mr_mla_decode_block_workspace_size(const mr_mla_block_args *args);
mr_status mr_mla_decode_block(const mr_mla_block_args *args, void *stream);

/* ------------------------------------------------------------------------
 * Causal MLA prefill, eager (expanded) form (K3MLA.forward,
 * Sources/ModelAdapters/Operators/MLA.swift:159-168,198-206; expand :231-245;
 * causalMask :257-275).  For each head h the keys are
 *   K[p] = [latent[p] . W_UK[h]^T  ++  rope_keys[p]]   (rope key shared)
 * and the values V[p] = latent[p] . W_UV[h]^T, with W_UK / W_UV the rows
 * h*(nope+v) + d and h*(nope+v) + nope + d of kv_b_proj [H*(nope+v),
 * kv_rank] (output-major, the layout k3Linear consumes, MLA.swift:180-186).
 * Query i of `tokens` sits at cache position n_ctx - tokens + i and sees
 * keys 0 .. n_ctx - tokens + i (the reference adds -FLT_MAX to the rest);
 * fp32 softmax.  out[i][h] = softmax(q . K^T * scale) . V.
 * Widths qk_nope 128, qk_rope 64, v_head 128, kv_rank 512 run on MFMA
 * (workspace: the up-projected keys/values in bf16, n_ctx * heads * 512
 * bytes; 16-byte aligned pointers, strides multiples of 8).  Other widths
 * (kv_rank and v_head 1 .. 2048, qk_nope 0 .. 1024, qk_rope 0 .. 512) run
 * any-width kernels in fp32 (workspace n_ctx * heads * (nope + v) * 4 bytes;
 * element-aligned pointers, strides covering the rows).
 * phase_events: NULL or 3 hipEvents recorded before the up-projection,
 * between the two kernels and after the attention.
 * ------------------------------------------------------------------------ */
typedef struct mr_mla_prefill_args {
    int32_t tokens; /* T >= 1 */
    int32_t n_ctx;  /* P >= T cached rows, the last T of which are the queries' */
    int32_t heads;
    int32_t qk_nope_dim, qk_rope_dim, v_head_dim, kv_rank;
    float scale; /* (qk_nope + qk_rope)^-1/2, MLA.swift:170 */
    const void *q; /* bf16 [T][H][nope + rope] */
    int64_t q_token_stride, q_head_stride;
    const void *latent; /* bf16 [P][kv_rank] (normed latent) */
    int64_t latent_row_stride;
    const void *rope_keys; /* bf16 [P][qk_rope] (rotated) */
    int64_t rope_row_stride;
    const void *kv_b; /* bf16 [H*(nope+v)][kv_rank] */
    int64_t kv_b_row_stride;
    void *out; /* [T][H][v_head] */
    mr_dtype out_dtype; /* MR_BF16 or MR_F32 */
    int64_t out_token_stride, out_head_stride;
    void *workspace;
    size_t workspace_bytes;
    void *const *phase_events;
} mr_mla_prefill_args;

size_t mr_mla_prefill_workspace_size(const mr_mla_prefill_args *args);
mr_status mr_mla_prefill(const mr_mla_prefill_args *args, void *stream);

/* ------------------------------------------------------------------------
 * A whole prompt through the MLA block in one call: K3MLA.forward
 * (MLA.swift:124-229; state == nil is position 0, a cached prefix of
 * `position` rows is the state's latents and shared keys):
 *   h = RMSNorm(x) per token (skipped when input_norm_w is NULL)
 *   q = q_b(RMSNorm(q_a(h)))            [T][heads][nope + rope]   (:131-139)
 *   kv = kv_a(h) -> cache rows position .. position+T-1, latent RMSNormed,
 *        shared key rotated at its position or carried (NoPE)   (:141-157)
 *   attn = causal attention of the T queries over rows 0 .. position+T-1,
 *          keys/values up-projected through kv_b (mr_mla_prefill)  (:159-206)
 *   out = o_proj(attn * sigmoid(g_proj(h)))  (gate when g_proj is given,
 *                                             :207-211)
 * Projections run over all T tokens (MFMA tiles from 64 tokens).  kv_b is
 * dense bf16 (K3's) or affine, dequantized to bf16 in the workspace.  Widths
 * as mr_mla_prefill takes them; qk_rope_dim even.  rope_cos / rope_sin:
 * device [T][qk_rope_dim/2], the angles at positions position .. position+T-1
 * (the query's rope slice and the cached keys rotate), or both NULL (NoPE).
 * All activations between stages are bf16; every stage is enqueued on
 * `stream`, in order.  Checks that can fail run before any cache write.
 * ------------------------------------------------------------------------ */
typedef struct mr_mla_prefill_block_args {
    int32_t tokens; /* T >= 1 prompt tokens */
    int32_t hidden, q_lora_rank, heads, qk_nope_dim, qk_rope_dim, v_head_dim, kv_rank;
    float eps, scale;
    const void *x; /* bf16 [T][hidden] */
    int64_t x_token_stride;
    const void *input_norm_w, *q_a_norm_w, *kv_a_norm_w;
    mr_dtype norm_w_dtype; /* bf16 or f32, all three */
    mr_projection q_a, q_b, kv_a, kv_b, o_proj;
    mr_projection g_proj; /* MR_PROJ_NONE: no output gate */
    void *cache_latent; /* bf16 rows, kv_rank wide */
    int64_t latent_row_stride;
    void *cache_rope; /* bf16 rows, qk_rope_dim wide (unused when 0) */
    int64_t rope_row_stride;
    int32_t position, capacity; /* rows cached before the first token; rows available */
    const float *rope_cos, *rope_sin; /* device [T][qk_rope_dim/2], or both NULL (NoPE) */
    void *out; /* bf16 [T][hidden] */
    int64_t out_token_stride;
    void *workspace;
    size_t workspace_bytes;
} mr_mla_prefill_block_args;

size_t mr_mla_prefill_block_workspace_size(const mr_mla_prefill_block_args *args);
mr_status mr_mla_prefill_block(const mr_mla_prefill_block_args *args, void *stream);

/* ------------------------------------------------------------------------
 * Index tables of DeepSeek V4 attention (DeepSeekV4Attention.swift:169-237),
 * host side, -1 = invalid entry.  `out` must hold rows*cols entries:
 * window: seq_len*min(seq_len, window) (or window when start_pos > 0);
 * compressed: seq_len*(seq_len/ratio) (or (start_pos+1)/ratio).
 * ------------------------------------------------------------------------ */
mr_status mr_attention_indices_window(int32_t window, int32_t seq_len, int32_t start_pos, int32_t *out,
                                      int32_t *rows, int32_t *cols);
mr_status mr_attention_indices_compressed(int32_t ratio, int32_t seq_len, int32_t start_pos, int32_t offset,
                                          int32_t *out, int32_t *rows, int32_t *cols);

/* ------------------------------------------------------------------------
 * Lightning-index scores (DeepSeekV4LightningIndexer.scores,
 * DeepSeekV4Attention.swift:530-549): scores[s][t] = sum_h w[s][h] *
 * max(q[s][h] . k[t], 0) in fp32 (NaN propagates), the producer of the
 * score matrix mr_topk_select ranks.  queries [seq][heads][dim] bf16 or f32
 * (strides in elements), keys [n_keys][key_dim] bf16 or f32 (row stride),
 * weights [w_rows][w_cols] f32 or bf16 (row stride), scores
 * [seq][out_row_stride] f32.  The geometry check is the reference's
 * (:533-541: seq, heads, dim > 0, key_dim == dim, weights [seq, heads]);
 * n_keys == 0 writes nothing (the reference returns [seq, 0]).  bf16 inputs
 * with dim 128 and heads a multiple of 16 up to 64 run on MFMA; other
 * shapes run a generic kernel.  Scores match the reference to fp32
 * rounding (its reduction order is MLX's), not bit for bit.
 * ------------------------------------------------------------------------ */
mr_status mr_indexer_scores(const void *queries, mr_dtype q_dtype, int32_t seq, int32_t heads, int32_t dim,
                            int64_t q_seq_stride, int64_t q_head_stride, const void *keys, mr_dtype k_dtype,
                            int32_t n_keys, int32_t key_dim, int64_t k_row_stride, const void *weights,
                            mr_dtype w_dtype, int32_t w_rows, int32_t w_cols, int64_t w_row_stride, float *scores,
                            int64_t out_row_stride, void *stream);

/* ------------------------------------------------------------------------
 * Lightning-indexer top-k selection (DeepSeekV4LightningIndexer.selecting,
 * DeepSeekV4Attention.swift:582-645), on the device, bit-exact.
 * scores [rows][cols] f32.  available = (start_pos + rows) / ratio keys are
 * ranked per row by descending score, ties by ascending key id; in row r
 * keys >= visible (visible = (r + 1) / ratio when start_pos == 0, else
 * available) compare as -infinity.  The first selected = min(top_k,
 * available) keys are written as offset + key, or -1 for a key >= visible.
 * Geometry errors are the reference's (:590-612), checked on the host; a
 * NaN score (anywhere in the matrix, :622-624) is reported through `status`
 * (device int32: 0 or MR_NONFINITE), with no host synchronisation; without
 * a status buffer (or with MR_TOPK_CHECK) the call reads the flags back and
 * returns MR_NONFINITE, as the reference throws; MR_TOPK_UNCHECKED skips
 * that read.  Any top_k; offset + available - 1 <= INT32_MAX.  Rows of
 * more than 32768 keys are ranked in slices of 32768 on as many workgroups
 * and merged; more than 4096 selected keys are ranked in slices of 4096
 * (each sorted whole) and merged.  Workspace: mr_topk_workspace_size(rows,
 * cols, top_k) bytes (per-row NaN flags; for sliced rows also the slices'
 * sorted lists, two buffers of rows x slices x min(top_k, slice) 8-byte
 * composites at the first merge round).
 * ------------------------------------------------------------------------ */
enum { MR_TOPK_CHECK = 1, MR_TOPK_UNCHECKED = 2 };

typedef struct mr_topk_args {
    const float *scores;
    int64_t score_row_stride;
    int32_t rows, cols;
    int32_t top_k, ratio, start_pos, offset;
    int32_t *out; /* device [rows][out_row_stride], selected entries per row */
    int64_t out_row_stride;
    int32_t *status; /* NULL or device int32 */
    int32_t flags;
    void *workspace;
    size_t workspace_bytes;
} mr_topk_args;

/* Host-only geometry check: the reference's errors, and the number of keys
 * each row receives. */
mr_status mr_topk_geometry(int32_t rows, int32_t cols, int32_t top_k, int32_t ratio, int32_t start_pos,
                           int32_t offset, int32_t *selected);
size_t mr_topk_workspace_size(int32_t rows, int32_t cols, int32_t top_k);
mr_status mr_topk_select(const mr_topk_args *args, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* MINIRUN_HIP_H */
