/*
 * mr_oracle.h -- CPU restatement of the Minirun MLA attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product library never links or calls it.
 *
 * Every function restates one piece of the reference (Swift over mlx-swift
 * 0.31.4, which cannot be built or imported here) and cites the file:line it
 * follows.  Where a function is pinned by a check other than its own formula,
 * the pinning test is named next to it; see the "pinned by" notes.
 *
 * Numeric conventions
 *  - bf16 values travel as uint16_t bit patterns; they are widened to float
 *    exactly (the high half of a float32, SafetensorsFile.swift:186-209).
 *  - "acc" arguments choose the accumulation type: 0 = float32 (what MLX
 *    computes), 1 = float64 (the tolerance anchor).
 *  - The file is compiled with -ffp-contract=off so that a*b+c is two
 *    roundings, as written.
 */
#ifndef MR_ORACLE_H
#define MR_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (mirror include/minirun_hip.h) ---- */
#define MRO_OK 0
#define MRO_INVALID_SHAPE 1
#define MRO_INVALID_DTYPE 2
#define MRO_INDEX_OUT_OF_RANGE 3
#define MRO_DUPLICATE_INDEX 4
#define MRO_NONFINITE 5

/* ---- dtypes for affine scales ---- */
#define MRO_BF16 0
#define MRO_F16 1
#define MRO_F32 2

/* ---- SplitMix64 (StorageCore/Generator/SplitMix64.swift:13-50) ---- */
uint64_t mro_splitmix_mix(uint64_t z);
uint64_t mro_splitmix_value(uint64_t seed, uint64_t index);
uint64_t mro_splitmix_derive(uint64_t seed, uint64_t label);
uint64_t mro_label(const char *name); /* FNV-1a 64 of a tensor label */

/* ---- bf16 / f16 helpers ---- */
uint16_t mro_f32_to_bf16(float x); /* round to nearest even */
float mro_bf16_to_f32(uint16_t h);
float mro_f16_to_f32(uint16_t h);

/* ---- seeded synthetic inputs ---- */
/* out[i] = bf16(mean + std * N(0,1)_i), Box-Muller over uniform pairs. */
void mro_fill_normal_bf16(uint64_t stream, int64_t n, double mean, double std_dev,
                          uint16_t *out, int threads);
/* out[i] = bf16(|std * N(0,1)_i|) */
void mro_fill_abs_normal_bf16(uint64_t stream, int64_t n, double std_dev, uint16_t *out,
                              int threads);
/* out[i] = top 32 bits of value(stream, i): uniform nibbles, uniform words. */
void mro_fill_u32(uint64_t stream, int64_t n, uint32_t *out, int threads);
/* Top-k sparse index set: the last `window` positions of [0, n_ctx) plus
 * (k - window) positions drawn without replacement from [0, n_ctx - window)
 * by a partial Fisher-Yates shuffle, sorted ascending. */
int mro_sparse_topk_indices(uint64_t stream, int32_t n_ctx, int32_t k, int32_t window,
                            int32_t *out);

/* ---- RoPE (DeepSeekV4Attention.swift:65-165) ---- */
int mro_rope_frequencies(int32_t dim, int32_t original_len, double base, double factor,
                         double beta_fast, double beta_slow, double *freqs_out);
/* cos/sin tables [n_pos, dim/2] in float, angle computed in double. */
int mro_rope_table(const int64_t *positions, int64_t n_pos, const double *freqs,
                   int32_t half, int inverse, float *cos_out, float *sin_out);
/* x: [n_pos, inner, dim] bf16 (row stride `row_stride` elements between
 * consecutive `inner` rows, rope slice starting at column `col0`); rotates
 * in place with adjacent pairs, fp32 arithmetic, result rounded to bf16. */
void mro_rope_apply_bf16(uint16_t *x, int64_t n_pos, int64_t inner, int64_t row_stride,
                         int64_t col0, int32_t dim, const float *cos_t, const float *sin_t);

/* ---- Dense projection, k3Linear (Linear.swift:55-57) ----
 * y[m, o] = sum_i x[m, i] * W[o, i], W output-major [out, in] with row
 * stride w_rs, bf16 bits (w_f32 = 0) or float (w_f32 = 1).  Pinned by
 * tests/test_oracle_math.py (identity and one-hot weights, linearity, an
 * fp64 product in numpy). */
void mro_linear(const float *x, int64_t M, const void *w, int w_f32, int64_t out_features,
                int64_t in_features, int64_t w_rs, int acc, float *y, int threads);

/* ---- K3MLA output gate (MLA.swift:209-211): out = merged * sigmoid(g),
 * sigmoid(g) = 1 / (1 + exp(-g)) in fp32.  Pinned by closed forms (g = 0
 * halves, large |g| passes or zeroes, sigmoid(-g) = 1 - sigmoid(g)) in
 * tests/test_oracle_math.py. */
void mro_sigmoid_gate(const float *merged, const float *g, int64_t n, float *out);

/* ---- RMSNorm (Normalization.swift:15-19) ---- */
void mro_rmsnorm(const float *x, int64_t rows, int64_t dim, const float *weight, float eps,
                 int acc, float *out);

/* ---- MLA absorbed decode (MLA.swift:174-197) ----
 * q_lat [B,H,R] bf16, q_rope [B,H,dr] bf16 (dr may be 0),
 * cache rows [B, n_ctx, row_stride] bf16 with latent at cols [0,R) and the
 * shared rope key at cols [R, R+dr).  Output ctx [B,H,R] float (pre-rounding). */
void mro_mla_decode(const uint16_t *q_lat, const uint16_t *q_rope, const uint16_t *cache,
                    int64_t row_stride, int64_t batch_stride, int32_t batch, int32_t heads,
                    int32_t n_ctx, int32_t kv_rank, int32_t rope_dim, float scale, int acc,
                    float *out, int threads);

/* ---- Sparse attention with sinks (DeepSeekV4Attention.swift:861-920) ----
 * q [B,H,Dk] (split as q_lat [B,H,R] + q_rope [B,H,dr]); rows: cache as above;
 * indices [B, n_idx] int32 with -1 = skip; sinks [H] float or NULL (no sink).
 * Output [B,H,R] float.  Returns MRO_OK / MRO_INDEX_OUT_OF_RANGE /
 * MRO_DUPLICATE_INDEX (validated before any arithmetic, :884-895). */
int mro_sparse_attention(const uint16_t *q_lat, const uint16_t *q_rope, const uint16_t *cache,
                         int64_t row_stride, int64_t batch_stride, int32_t batch,
                         int32_t heads, int32_t n_ctx, int32_t kv_rank, int32_t rope_dim,
                         const int32_t *indices, int32_t n_idx, const float *sinks,
                         float scale, int acc, float *out, int threads);
int mro_validate_indices(const int32_t *indices, int32_t n_idx, int32_t n_rows,
                         int32_t *bad_position);

/* ---- Eager causal MLA prefill (MLA.swift:159-168,198-206,231-275) ----
 * q [T,H,dn+dr] bf16, cache rows [P, row_stride] bf16 (latent R ++ rope dr),
 * w_uk, w_uv [R, H*dn] / [R, H*dv] bf16 (input-major: kv_b_proj[h*(dn+dv)+d, r]
 * = w_uk[r, h*dn+d]).  Query i attends keys <= P - T + i.  Only the
 * (t, h) pairs listed in sel_t/sel_h (n_sel of them) are computed; out is
 * [n_sel, dv] float.  Keys/values are formed in float (one bf16 rounding of
 * the up-projection when round_kv is set, as the HIP path stores them). */
void mro_mla_prefill_rows(const uint16_t *q, const uint16_t *cache, int64_t row_stride,
                          const uint16_t *w_uk, const uint16_t *w_uv, int32_t T, int32_t P,
                          int32_t heads, int32_t kv_rank, int32_t rope_dim, int32_t nope_dim,
                          int32_t v_dim, float scale, int round_kv, const int32_t *sel_t,
                          const int32_t *sel_h, int32_t n_sel, float *out, int threads);

/* ---- MLX affine quantization (MLXBridge/AffineWeights.swift:65-157,232-342) ---- */
int mro_affine_validate(int64_t out_features, int64_t packed_cols, int64_t scale_cols,
                        int32_t group, int32_t bits, int64_t *in_features_out);
int mro_affine_dequantize(const uint32_t *packed, const uint16_t *scales_or_f32,
                          const uint16_t *biases_or_f32, int32_t scale_dtype,
                          int64_t out_features, int64_t in_features, int32_t group,
                          int32_t bits, float *out, int threads);
/* y[m, o] = sum_i x[m, i] * W[o, i], W = dequant.  x float [M, in]. */
int mro_affine_matmul(const float *x, int64_t M, const uint32_t *packed,
                      const uint16_t *scales_or_f32, const uint16_t *biases_or_f32,
                      int32_t scale_dtype, int64_t out_features, int64_t in_features,
                      int32_t group, int32_t bits, int acc, float *y, int threads);

/* ---- Lightning-indexer selection and index tables
 *      (DeepSeekV4Attention.swift:169-237, 582-645) ---- */
int mro_topk_select(const float *scores, int32_t rows, int32_t cols, int32_t top_k,
                    int32_t ratio, int32_t start_pos, int32_t offset, int32_t *out,
                    int32_t *out_count);
/* DeepSeekV4LightningIndexer.scores (DeepSeekV4Attention.swift:530-549):
 * out[s][t] = sum_h w[s][h] * max(q[s][h] . k[t], 0) in fp32; the dot is
 * summed over d in order, the heads in order; NaN propagates through the
 * max.  q [S][H][D], k [T][D], w [S][H], out [S][T], all dense fp32. */
int mro_indexer_scores(const float *q, int32_t S, int32_t H, int32_t D, const float *k, int32_t T,
                       const float *w, float *out);
int mro_window_indices(int32_t window, int32_t seq_len, int32_t start_pos, int32_t *out,
                       int32_t *out_rows, int32_t *out_cols);
int mro_compressed_indices(int32_t ratio, int32_t seq_len, int32_t start_pos, int32_t offset,
                           int32_t *out, int32_t *out_rows, int32_t *out_cols);

#ifdef __cplusplus
}
#endif
#endif
