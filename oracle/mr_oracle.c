/*
 * mr_oracle.c -- CPU restatement of the Minirun MLA attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the tests check the library against it; it is
 * never part of the product): see mr_oracle.h.
 * Build: oracle/Makefile (gcc -O2 -fopenmp -ffp-contract=off).
 *
 * Pinning status, by function (the tests that pin each one are named in
 * tests/test_oracle_*.py):
 *   splitmix / derive        published SplitMix64 test vectors + the
 *                            reference's own stream==value identity
 *   bf16 rounding            hand KATs (ties-to-even, NaN, overflow)
 *   normal/abs-normal fill   moments + Python re-implementation
 *   sparse_topk_indices      structural invariants (sorted, unique, window)
 *   rope_*                   pos 0 identity, inverse∘forward, norm, relative
 *                            position property, fp64 KATs, YaRN closed form
 *   rmsnorm                  constant vector, scale invariance, numpy
 *   mla_decode               brute-force numpy fp64, absorbed == expanded,
 *                            N=1, equal scores, one-hot, permutation
 *   sparse_attention         all-indices == dense, single index, sink->-inf,
 *                            -1 skip, duplicates/out-of-range errors
 *   mla_prefill_rows         numpy fp64 expanded attention, T=1 == decode,
 *                            prefix consistency
 *   affine_*                 nibble KATs, pack/unpack round trip, closed
 *                            form bitwise, validation error order
 *   topk_select              brute force with the stated comparator, ties,
 *                            NaN, masking
 *   indexer_scores           numpy fp64 brute force, w = 0, negative dots,
 *                            linearity in w, positive key scaling, NaN
 *   window/compressed        hand-written tables from the reference's rules
 *   MLX reduction order      parity unpinned (needs MLX; tolerance instead)
 */
#include "mr_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define MRO_GAMMA 0x9E3779B97F4A7C15ULL

/* SplitMix64.swift:29-35 */
uint64_t mro_splitmix_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* SplitMix64.swift:40-43: the index-th output of a stream, closed form. */
uint64_t mro_splitmix_value(uint64_t seed, uint64_t index) {
    return mro_splitmix_mix(seed + (index + 1) * MRO_GAMMA);
}

/* SplitMix64.swift:48-50 */
uint64_t mro_splitmix_derive(uint64_t seed, uint64_t label) {
    return mro_splitmix_mix(seed ^ mro_splitmix_mix(label + 0xD1B54A32D192ED03ULL));
}

uint64_t mro_label(const char *name) {
    uint64_t h = 0xcbf29ce484222325ULL;
    for (const unsigned char *p = (const unsigned char *)name; *p; ++p) {
        h ^= *p;
        h *= 0x100000001b3ULL;
    }
    return h;
}

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t mro_f32_to_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* SafetensorsFile.swift:186-209: BF16 is the high half of a float32. */
float mro_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

float mro_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        float v = (float)man * (1.0f / 16777216.0f); /* man * 2^-24 */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

static inline double uniform53(uint64_t stream, uint64_t i) {
    return (double)(mro_splitmix_value(stream, i) >> 11) * (1.0 / 9007199254740992.0);
}

/* Box-Muller on the uniform pair (2j, 2j+1); element 2j takes the cosine
 * branch and 2j+1 the sine branch.  1-u keeps the logarithm finite. */
static inline double normal_at(uint64_t stream, int64_t i) {
    int64_t j = i >> 1;
    double u1 = uniform53(stream, (uint64_t)(2 * j));
    double u2 = uniform53(stream, (uint64_t)(2 * j + 1));
    double r = sqrt(-2.0 * log(1.0 - u1));
    double a = 6.283185307179586476925286766559 * u2;
    return (i & 1) ? r * sin(a) : r * cos(a);
}

static int pick_threads(int threads) {
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#else
    threads = 1;
#endif
    return threads;
}

void mro_fill_normal_bf16(uint64_t stream, int64_t n, double mean, double std_dev,
                          uint16_t *out, int threads) {
    threads = pick_threads(threads);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t i = 0; i < n; ++i)
        out[i] = mro_f32_to_bf16((float)(mean + std_dev * normal_at(stream, i)));
}

void mro_fill_abs_normal_bf16(uint64_t stream, int64_t n, double std_dev, uint16_t *out,
                              int threads) {
    threads = pick_threads(threads);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t i = 0; i < n; ++i)
        out[i] = mro_f32_to_bf16((float)fabs(std_dev * normal_at(stream, i)));
}

void mro_fill_u32(uint64_t stream, int64_t n, uint32_t *out, int threads) {
    threads = pick_threads(threads);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = (uint32_t)(mro_splitmix_value(stream, (uint64_t)i) >> 32);
}

static int cmp_i32(const void *a, const void *b) {
    int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
    return (x > y) - (x < y);
}

int mro_sparse_topk_indices(uint64_t stream, int32_t n_ctx, int32_t k, int32_t window,
                            int32_t *out) {
    if (n_ctx <= 0 || k <= 0 || window < 0 || window > k || k > n_ctx) return MRO_INVALID_SHAPE;
    int32_t m = n_ctx - window;
    int32_t draw = k - window;
    int32_t *pool = (int32_t *)malloc(sizeof(int32_t) * (size_t)(m > 0 ? m : 1));
    if (!pool) return MRO_INVALID_SHAPE;
    for (int32_t i = 0; i < m; ++i) pool[i] = i;
    for (int32_t i = 0; i < draw; ++i) {
        uint64_t span = (uint64_t)(m - i);
        int32_t j = i + (int32_t)(mro_splitmix_value(stream, (uint64_t)i) % span);
        int32_t t = pool[i];
        pool[i] = pool[j];
        pool[j] = t;
    }
    for (int32_t i = 0; i < draw; ++i) out[i] = pool[i];
    for (int32_t i = 0; i < window; ++i) out[draw + i] = m + i;
    free(pool);
    qsort(out, (size_t)k, sizeof(int32_t), cmp_i32);
    return MRO_OK;
}

/* DeepSeekV4Attention.swift:28-99: validation and the YaRN-ramped table. */
int mro_rope_frequencies(int32_t dim, int32_t original_len, double base, double factor,
                         double beta_fast, double beta_slow, double *freqs) {
    if (dim <= 0 || (dim % 2) != 0) return MRO_INVALID_SHAPE;
    if (original_len < 0) return MRO_INVALID_SHAPE;
    if (!(isfinite(base) && base > 1 && isfinite(factor) && factor > 0 && isfinite(beta_fast) &&
          beta_fast > 0 && isfinite(beta_slow) && beta_slow > 0))
        return MRO_INVALID_SHAPE;
    int32_t half = dim / 2;
    for (int32_t p = 0; p < half; ++p) freqs[p] = 1.0 / pow(base, (double)(p * 2) / (double)dim);
    if (original_len > 0) {
        double two_pi = 2.0 * 3.14159265358979323846;
        double cd_fast = (double)dim * log((double)original_len / (beta_fast * two_pi)) /
                         (2.0 * log(base));
        double cd_slow = (double)dim * log((double)original_len / (beta_slow * two_pi)) /
                         (2.0 * log(base));
        int64_t low = (int64_t)floor(cd_fast);
        if (low < 0) low = 0;
        int64_t high = (int64_t)ceil(cd_slow);
        if (high > dim - 1) high = dim - 1;
        double denom = (low == high) ? 0.001 : (double)(high - low);
        for (int32_t p = 0; p < half; ++p) {
            double ramp = ((double)p - (double)low) / denom;
            if (ramp < 0) ramp = 0;
            if (ramp > 1) ramp = 1;
            double smooth = 1.0 - ramp;
            freqs[p] = freqs[p] / factor * (1.0 - smooth) + freqs[p] * smooth;
        }
    }
    for (int32_t p = 0; p < half; ++p)
        if (!(isfinite(freqs[p]) && freqs[p] > 0)) return MRO_NONFINITE;
    return MRO_OK;
}

/* DeepSeekV4Attention.swift:126-149: angle in double, cos/sin rounded to float. */
int mro_rope_table(const int64_t *positions, int64_t n_pos, const double *freqs, int32_t half,
                   int inverse, float *cos_out, float *sin_out) {
    double direction = inverse ? -1.0 : 1.0;
    for (int64_t i = 0; i < n_pos; ++i)
        if (positions[i] < 0) return MRO_INVALID_SHAPE;
    for (int64_t i = 0; i < n_pos; ++i) {
        for (int32_t p = 0; p < half; ++p) {
            double angle = direction * (double)positions[i] * freqs[p];
            if (!isfinite(angle)) return MRO_NONFINITE;
            cos_out[i * half + p] = (float)cos(angle);
            sin_out[i * half + p] = (float)sin(angle);
        }
    }
    return MRO_OK;
}

/* DeepSeekV4Attention.swift:151-163: adjacent pairs in float, cast back. */
void mro_rope_apply_bf16(uint16_t *x, int64_t n_pos, int64_t inner, int64_t row_stride,
                         int64_t col0, int32_t dim, const float *cos_t, const float *sin_t) {
    int32_t half = dim / 2;
    for (int64_t s = 0; s < n_pos; ++s) {
        for (int64_t r = 0; r < inner; ++r) {
            uint16_t *v = x + (s * inner + r) * row_stride + col0;
            for (int32_t p = 0; p < half; ++p) {
                float e = mro_bf16_to_f32(v[2 * p]);
                float o = mro_bf16_to_f32(v[2 * p + 1]);
                float c = cos_t[s * half + p], sn = sin_t[s * half + p];
                float ec = e * c, os = o * sn, es = e * sn, oc = o * c;
                float re = ec - os;
                float im = es + oc;
                v[2 * p] = mro_f32_to_bf16(re);
                v[2 * p + 1] = mro_f32_to_bf16(im);
            }
        }
    }
}

/* Normalization.swift:15-19: w * (x * rsqrt(mean(x^2) + eps)). */
void mro_rmsnorm(const float *x, int64_t rows, int64_t dim, const float *weight, float eps,
                 int acc, float *out) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * dim;
        float *o = out + r * dim;
        if (acc) {
            double ss = 0;
            for (int64_t i = 0; i < dim; ++i) ss += (double)xr[i] * (double)xr[i];
            double inv = 1.0 / sqrt(ss / (double)dim + (double)eps);
            for (int64_t i = 0; i < dim; ++i) o[i] = (float)((double)weight[i] * ((double)xr[i] * inv));
        } else {
            float ss = 0;
            for (int64_t i = 0; i < dim; ++i) ss += xr[i] * xr[i];
            float mean = ss / (float)dim;
            float inv = 1.0f / sqrtf(mean + eps);
            for (int64_t i = 0; i < dim; ++i) o[i] = weight[i] * (xr[i] * inv);
        }
    }
}

/* One absorbed-MLA head: MLA.swift:188-196.
 *   scores = (q_lat . c^T + q_rot . k_rot^T) * scale; probs = softmax_fp32;
 *   out = probs . c   (the latent context; W_UV is applied by the caller). */
static void decode_head_f64(const uint16_t *ql, const uint16_t *qr, const uint16_t *rows,
                            int64_t row_stride, const int32_t *sel, int32_t n_sel,
                            int32_t kv_rank, int32_t rope_dim, const float *sink, float scale,
                            float *out) {
    double *s = (double *)malloc(sizeof(double) * (size_t)(n_sel > 0 ? n_sel : 1));
    double qlat[1024], qrot[256], acc[1024];
    for (int32_t r = 0; r < kv_rank; ++r) qlat[r] = mro_bf16_to_f32(ql[r]);
    for (int32_t j = 0; j < rope_dim; ++j) qrot[j] = mro_bf16_to_f32(qr[j]);
    double m = -INFINITY;
    for (int32_t i = 0; i < n_sel; ++i) {
        const uint16_t *c = rows + (int64_t)sel[i] * row_stride;
        double a = 0, b = 0;
        for (int32_t r = 0; r < kv_rank; ++r) a += qlat[r] * (double)mro_bf16_to_f32(c[r]);
        for (int32_t j = 0; j < rope_dim; ++j)
            b += qrot[j] * (double)mro_bf16_to_f32(c[kv_rank + j]);
        s[i] = (a + b) * (double)scale;
        if (s[i] > m) m = s[i];
    }
    if (sink && (double)*sink > m) m = (double)*sink;
    double l = 0;
    for (int32_t r = 0; r < kv_rank; ++r) acc[r] = 0;
    for (int32_t i = 0; i < n_sel; ++i) {
        double p = exp(s[i] - m);
        l += p;
        const uint16_t *c = rows + (int64_t)sel[i] * row_stride;
        for (int32_t r = 0; r < kv_rank; ++r) acc[r] += p * (double)mro_bf16_to_f32(c[r]);
    }
    if (sink) l += exp((double)*sink - m);
    for (int32_t r = 0; r < kv_rank; ++r) out[r] = n_sel > 0 ? (float)(acc[r] / l) : 0.0f;
    free(s);
}

static void decode_head_f32(const uint16_t *ql, const uint16_t *qr, const uint16_t *rows,
                            int64_t row_stride, const int32_t *sel, int32_t n_sel,
                            int32_t kv_rank, int32_t rope_dim, const float *sink, float scale,
                            float *out) {
    float *s = (float *)malloc(sizeof(float) * (size_t)(n_sel > 0 ? n_sel : 1));
    float qlat[1024], qrot[256], acc[1024];
    for (int32_t r = 0; r < kv_rank; ++r) qlat[r] = mro_bf16_to_f32(ql[r]);
    for (int32_t j = 0; j < rope_dim; ++j) qrot[j] = mro_bf16_to_f32(qr[j]);
    float m = -INFINITY;
    for (int32_t i = 0; i < n_sel; ++i) {
        const uint16_t *c = rows + (int64_t)sel[i] * row_stride;
        float a = 0, b = 0;
        for (int32_t r = 0; r < kv_rank; ++r) a += qlat[r] * mro_bf16_to_f32(c[r]);
        for (int32_t j = 0; j < rope_dim; ++j) b += qrot[j] * mro_bf16_to_f32(c[kv_rank + j]);
        s[i] = (a + b) * scale;
        if (s[i] > m) m = s[i];
    }
    if (sink && *sink > m) m = *sink;
    float l = 0;
    for (int32_t i = 0; i < n_sel; ++i) {
        s[i] = expf(s[i] - m);
        l += s[i];
    }
    if (sink) l += expf(*sink - m);
    for (int32_t r = 0; r < kv_rank; ++r) acc[r] = 0;
    for (int32_t i = 0; i < n_sel; ++i) {
        float p = s[i] / l; /* softmax first, then probs . latents */
        const uint16_t *c = rows + (int64_t)sel[i] * row_stride;
        for (int32_t r = 0; r < kv_rank; ++r) acc[r] += p * mro_bf16_to_f32(c[r]);
    }
    for (int32_t r = 0; r < kv_rank; ++r) out[r] = n_sel > 0 ? acc[r] : 0.0f;
    free(s);
}

void mro_mla_decode(const uint16_t *q_lat, const uint16_t *q_rope, const uint16_t *cache,
                    int64_t row_stride, int64_t batch_stride, int32_t batch, int32_t heads,
                    int32_t n_ctx, int32_t kv_rank, int32_t rope_dim, float scale, int acc,
                    float *out, int threads) {
    threads = pick_threads(threads);
    int32_t *sel = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_ctx > 0 ? n_ctx : 1));
    for (int32_t i = 0; i < n_ctx; ++i) sel[i] = i;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t bh = 0; bh < (int64_t)batch * heads; ++bh) {
        int64_t b = bh / heads;
        const uint16_t *ql = q_lat + bh * kv_rank;
        const uint16_t *qr = q_rope ? q_rope + bh * rope_dim : NULL;
        const uint16_t *rows = cache + b * batch_stride;
        if (acc)
            decode_head_f64(ql, qr, rows, row_stride, sel, n_ctx, kv_rank, rope_dim, NULL, scale,
                            out + bh * kv_rank);
        else
            decode_head_f32(ql, qr, rows, row_stride, sel, n_ctx, kv_rank, rope_dim, NULL, scale,
                            out + bh * kv_rank);
    }
    free(sel);
}

/* DeepSeekV4Attention.swift:884-895: one in-order scan; -1 skips, an entry
 * outside [0, n_rows) stops the scan with a range error, an entry equal to
 * an earlier (in-range) entry stops it with a duplicate error.  bad_position
 * receives the column where the scan stopped. */
static int cmp_i64(const void *a, const void *b) {
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return (x > y) - (x < y);
}

int mro_validate_indices(const int32_t *indices, int32_t n_idx, int32_t n_rows,
                         int32_t *bad_position) {
    /* (value, position) keys of the in-range entries, sorted: the first key
     * of a value holds the position where that value is first seen */
    int64_t *keys = (int64_t *)malloc(sizeof(int64_t) * (size_t)(n_idx > 0 ? n_idx : 1));
    int32_t n = 0;
    for (int32_t i = 0; i < n_idx; ++i) {
        int32_t v = indices[i];
        if (v >= 0 && v < n_rows) keys[n++] = ((int64_t)v << 32) | (int64_t)i;
    }
    qsort(keys, (size_t)n, sizeof(int64_t), cmp_i64);
    int status = MRO_OK;
    for (int32_t i = 0; i < n_idx && status == MRO_OK; ++i) {
        int32_t v = indices[i];
        if (v == -1) continue;
        if (v < 0 || v >= n_rows) {
            status = MRO_INDEX_OUT_OF_RANGE;
        } else {
            int32_t lo = 0, hi = n; /* first key with value v */
            while (lo < hi) {
                int32_t mid = (lo + hi) / 2;
                if ((keys[mid] >> 32) < v) lo = mid + 1; else hi = mid;
            }
            if ((int32_t)(keys[lo] & 0xffffffff) < i) status = MRO_DUPLICATE_INDEX;
        }
        if (status != MRO_OK && bad_position) *bad_position = i;
    }
    free(keys);
    return status;
}

int mro_sparse_attention(const uint16_t *q_lat, const uint16_t *q_rope, const uint16_t *cache,
                         int64_t row_stride, int64_t batch_stride, int32_t batch,
                         int32_t heads, int32_t n_ctx, int32_t kv_rank, int32_t rope_dim,
                         const int32_t *indices, int32_t n_idx, const float *sinks,
                         float scale, int acc, float *out, int threads) {
    if (!(scale > 0) || !isfinite(scale)) return MRO_INVALID_SHAPE;
    for (int32_t b = 0; b < batch; ++b) {
        int32_t bad = -1;
        int st = mro_validate_indices(indices + (int64_t)b * n_idx, n_idx, n_ctx, &bad);
        if (st != MRO_OK) return st;
    }
    threads = pick_threads(threads);
    int32_t *valid = (int32_t *)malloc(sizeof(int32_t) * (size_t)batch * (size_t)(n_idx + 1));
    int32_t *nvalid = (int32_t *)malloc(sizeof(int32_t) * (size_t)batch);
    for (int32_t b = 0; b < batch; ++b) {
        int32_t n = 0;
        for (int32_t i = 0; i < n_idx; ++i) {
            int32_t v = indices[(int64_t)b * n_idx + i];
            if (v != -1) valid[(int64_t)b * (n_idx + 1) + n++] = v;
        }
        nvalid[b] = n;
    }
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t bh = 0; bh < (int64_t)batch * heads; ++bh) {
        int64_t b = bh / heads, h = bh % heads;
        const uint16_t *ql = q_lat + bh * kv_rank;
        const uint16_t *qr = q_rope ? q_rope + bh * rope_dim : NULL;
        const float *sink = sinks ? sinks + h : NULL;
        const int32_t *sel = valid + b * (n_idx + 1);
        if (acc)
            decode_head_f64(ql, qr, cache + b * batch_stride, row_stride, sel, nvalid[b], kv_rank,
                            rope_dim, sink, scale, out + bh * kv_rank);
        else
            decode_head_f32(ql, qr, cache + b * batch_stride, row_stride, sel, nvalid[b], kv_rank,
                            rope_dim, sink, scale, out + bh * kv_rank);
    }
    free(valid);
    free(nvalid);
    return MRO_OK;
}

/* MLA.swift:231-245 (expand) + 198-206 (eager attention) + 257-275 (mask),
 * evaluated for selected (query, head) pairs in double.  Masked keys are
 * skipped: their -FLT_MAX score underflows to probability 0 exactly. */
void mro_mla_prefill_rows(const uint16_t *q, const uint16_t *cache, int64_t row_stride,
                          const uint16_t *w_uk, const uint16_t *w_uv, int32_t T, int32_t P,
                          int32_t heads, int32_t kv_rank, int32_t rope_dim, int32_t nope_dim,
                          int32_t v_dim, float scale, int round_kv, const int32_t *sel_t,
                          const int32_t *sel_h, int32_t n_sel, float *out, int threads) {
    threads = pick_threads(threads);
    int32_t dq = nope_dim + rope_dim;
    /* group by head so each head's keys/values are formed once */
    for (int32_t h = 0; h < heads; ++h) {
        int any = 0;
        for (int32_t i = 0; i < n_sel; ++i)
            if (sel_h[i] == h) any = 1;
        if (!any) continue;
        double *K = (double *)malloc(sizeof(double) * (size_t)P * (size_t)nope_dim);
        double *V = (double *)malloc(sizeof(double) * (size_t)P * (size_t)v_dim);
#pragma omp parallel for num_threads(threads) schedule(static)
        for (int32_t p = 0; p < P; ++p) {
            const uint16_t *c = cache + (int64_t)p * row_stride;
            for (int32_t d = 0; d < nope_dim; ++d) {
                double a = 0;
                for (int32_t r = 0; r < kv_rank; ++r)
                    a += (double)mro_bf16_to_f32(c[r]) *
                         (double)mro_bf16_to_f32(w_uk[(int64_t)r * heads * nope_dim + (int64_t)h * nope_dim + d]);
                K[(int64_t)p * nope_dim + d] = round_kv ? (double)mro_bf16_to_f32(mro_f32_to_bf16((float)a)) : a;
            }
            for (int32_t d = 0; d < v_dim; ++d) {
                double a = 0;
                for (int32_t r = 0; r < kv_rank; ++r)
                    a += (double)mro_bf16_to_f32(c[r]) *
                         (double)mro_bf16_to_f32(w_uv[(int64_t)r * heads * v_dim + (int64_t)h * v_dim + d]);
                V[(int64_t)p * v_dim + d] = round_kv ? (double)mro_bf16_to_f32(mro_f32_to_bf16((float)a)) : a;
            }
        }
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
        for (int32_t i = 0; i < n_sel; ++i) {
            if (sel_h[i] != h) continue;
            int32_t t = sel_t[i];
            int32_t last = t + (P - T); /* key > query + offset is masked */
            const uint16_t *qv = q + ((int64_t)t * heads + h) * dq;
            double *s = (double *)malloc(sizeof(double) * (size_t)P);
            double m = -INFINITY;
            for (int32_t p = 0; p <= last && p < P; ++p) {
                const uint16_t *c = cache + (int64_t)p * row_stride;
                double a = 0;
                for (int32_t d = 0; d < nope_dim; ++d)
                    a += (double)mro_bf16_to_f32(qv[d]) * K[(int64_t)p * nope_dim + d];
                for (int32_t j = 0; j < rope_dim; ++j)
                    a += (double)mro_bf16_to_f32(qv[nope_dim + j]) *
                         (double)mro_bf16_to_f32(c[kv_rank + j]);
                s[p] = a * (double)scale;
                if (s[p] > m) m = s[p];
            }
            double l = 0;
            double acc[1024];
            for (int32_t d = 0; d < v_dim; ++d) acc[d] = 0;
            for (int32_t p = 0; p <= last && p < P; ++p) {
                double e = exp(s[p] - m);
                l += e;
                for (int32_t d = 0; d < v_dim; ++d) acc[d] += e * V[(int64_t)p * v_dim + d];
            }
            for (int32_t d = 0; d < v_dim; ++d) out[(int64_t)i * v_dim + d] = (float)(acc[d] / l);
            free(s);
        }
        free(K);
        free(V);
    }
}

/* AffineWeights.swift:104-147: the shape rules, in the reference's order. */
int mro_affine_validate(int64_t out_features, int64_t packed_cols, int64_t scale_cols,
                        int32_t group, int32_t bits, int64_t *in_features_out) {
    if (out_features < 0 || packed_cols < 0 || scale_cols < 0) return MRO_INVALID_SHAPE;
    if (bits <= 0 || (32 % bits) != 0) return MRO_INVALID_SHAPE;
    if (group <= 0) return MRO_INVALID_SHAPE;
    int64_t in_features = packed_cols * (32 / bits);
    if (in_features % group != 0) return MRO_INVALID_SHAPE;
    if (scale_cols != in_features / group) return MRO_INVALID_SHAPE;
    if (in_features_out) *in_features_out = in_features;
    return MRO_OK;
}

static inline float scale_at(const uint16_t *p, int32_t dtype, int64_t i) {
    if (dtype == MRO_BF16) return mro_bf16_to_f32(p[i]);
    if (dtype == MRO_F16) return mro_f16_to_f32(p[i]);
    float f;
    memcpy(&f, (const char *)p + 4 * i, 4);
    return f;
}

/* AffineWeights.swift:320-342 + MXFP4Weights.swift:42-48: element j of a
 * word sits at bit offset bits*j (element 0 in the low bits);
 * w = scale * q + bias, two float roundings (the product is exact for
 * bf16/f16 scales, so this equals the fused form too). */
int mro_affine_dequantize(const uint32_t *packed, const uint16_t *scales,
                          const uint16_t *biases, int32_t scale_dtype, int64_t out_features,
                          int64_t in_features, int32_t group, int32_t bits, float *out,
                          int threads) {
    if (scale_dtype < MRO_BF16 || scale_dtype > MRO_F32) return MRO_INVALID_DTYPE;
    if (bits <= 0 || 32 % bits != 0 || group <= 0 || in_features % group != 0)
        return MRO_INVALID_SHAPE;
    threads = pick_threads(threads);
    int32_t per_word = 32 / bits;
    uint32_t mask = bits == 32 ? 0xffffffffu : ((1u << bits) - 1u);
    int64_t words = in_features / per_word;
    int64_t groups = in_features / group;
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t o = 0; o < out_features; ++o) {
        for (int64_t i = 0; i < in_features; ++i) {
            uint32_t w = packed[o * words + i / per_word];
            uint32_t q = (w >> (bits * (i % per_word))) & mask;
            float s = scale_at(scales, scale_dtype, o * groups + i / group);
            float b = scale_at(biases, scale_dtype, o * groups + i / group);
            float prod = s * (float)q;
            out[o * in_features + i] = prod + b;
        }
    }
    return MRO_OK;
}

int mro_affine_matmul(const float *x, int64_t M, const uint32_t *packed, const uint16_t *scales,
                      const uint16_t *biases, int32_t scale_dtype, int64_t out_features,
                      int64_t in_features, int32_t group, int32_t bits, int acc, float *y,
                      int threads) {
    float *w = (float *)malloc(sizeof(float) * (size_t)out_features * (size_t)in_features);
    if (!w) return MRO_INVALID_SHAPE;
    int st = mro_affine_dequantize(packed, scales, biases, scale_dtype, out_features, in_features,
                                   group, bits, w, threads);
    if (st != MRO_OK) {
        free(w);
        return st;
    }
    threads = pick_threads(threads);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t o = 0; o < out_features; ++o) {
        for (int64_t m = 0; m < M; ++m) {
            const float *xr = x + m * in_features;
            const float *wr = w + o * in_features;
            if (acc) {
                double a = 0;
                for (int64_t i = 0; i < in_features; ++i) a += (double)xr[i] * (double)wr[i];
                y[m * out_features + o] = (float)a;
            } else {
                float a = 0;
                for (int64_t i = 0; i < in_features; ++i) a += xr[i] * wr[i];
                y[m * out_features + o] = a;
            }
        }
    }
    free(w);
    return MRO_OK;
}

/* DeepSeekV4Attention.swift:545-548: perHead = einsum("shd,td->sht") in
 * fp32, then sum over h of maximum(perHead, 0) * w[s, h]. */
int mro_indexer_scores(const float *q, int32_t S, int32_t H, int32_t D, const float *k, int32_t T,
                       const float *w, float *out) {
    if (!(S > 0 && H > 0 && D > 0 && T >= 0)) return MRO_INVALID_SHAPE;
#pragma omp parallel for schedule(static)
    for (int64_t st = 0; st < (int64_t)S * T; ++st) {
        const int64_t s = st / T, t = st % T;
        float acc = 0.f;
        for (int32_t h = 0; h < H; ++h) {
            const float *qr = q + (s * H + h) * D, *kr = k + t * D;
            float d = 0.f;
            for (int32_t i = 0; i < D; ++i) d += qr[i] * kr[i];
            const float r = d > 0.f ? d : (d != d ? d : 0.f);
            acc += r * w[s * H + h];
        }
        out[st] = acc;
    }
    return MRO_OK;
}

/* DeepSeekV4Attention.swift:630-634: descending score, ties by ascending
 * key id, keys at or past `visible` compare as -infinity. */
static const float *g_sort_scores;
static int32_t g_sort_visible;
static int topk_cmp(const void *a, const void *b) {
    int32_t l = *(const int32_t *)a, r = *(const int32_t *)b;
    float lv = l < g_sort_visible ? g_sort_scores[l] : -INFINITY;
    float rv = r < g_sort_visible ? g_sort_scores[r] : -INFINITY;
    if (lv == rv) return (l > r) - (l < r);
    return lv > rv ? -1 : 1;
}

/* DeepSeekV4Attention.swift:582-645 */
int mro_topk_select(const float *scores, int32_t rows, int32_t cols, int32_t top_k,
                    int32_t ratio, int32_t start_pos, int32_t offset, int32_t *out,
                    int32_t *out_count) {
    if (!(rows > 0 && top_k > 0 && ratio > 0 && start_pos >= 0 && offset >= 0))
        return MRO_INVALID_SHAPE;
    if (start_pos > 0 && rows != 1) return MRO_INVALID_SHAPE;
    int64_t end = (int64_t)start_pos + rows;
    if (end > 0x7fffffffLL) return MRO_INVALID_SHAPE;
    int32_t available = (int32_t)(end / ratio);
    if (available > cols) return MRO_INVALID_SHAPE;
    int32_t selected = top_k < available ? top_k : available;
    *out_count = selected;
    if (selected == 0) return MRO_OK;
    for (int64_t i = 0; i < (int64_t)rows * cols; ++i)
        if (isnan(scores[i])) return MRO_NONFINITE;
    int32_t *order = (int32_t *)malloc(sizeof(int32_t) * (size_t)available);
    for (int32_t row = 0; row < rows; ++row) {
        int32_t visible = start_pos == 0 ? (row + 1) / ratio : available;
        for (int32_t k = 0; k < available; ++k) order[k] = k;
        g_sort_scores = scores + (int64_t)row * cols;
        g_sort_visible = visible;
        qsort(order, (size_t)available, sizeof(int32_t), topk_cmp);
        for (int32_t k = 0; k < selected; ++k) {
            int32_t key = order[k];
            if (key >= visible) {
                out[(int64_t)row * selected + k] = -1;
            } else {
                int64_t v = (int64_t)offset + key;
                if (v > 0x7fffffffLL) {
                    free(order);
                    return MRO_INVALID_SHAPE;
                }
                out[(int64_t)row * selected + k] = (int32_t)v;
            }
        }
    }
    free(order);
    return MRO_OK;
}

/* DeepSeekV4Attention.swift:170-198 */
int mro_window_indices(int32_t window, int32_t seq_len, int32_t start_pos, int32_t *out,
                       int32_t *out_rows, int32_t *out_cols) {
    if (!(window > 0 && seq_len > 0 && start_pos >= 0)) return MRO_INVALID_SHAPE;
    if (start_pos > 0) {
        if (seq_len != 1) return MRO_INVALID_SHAPE;
        *out_rows = 1;
        *out_cols = window;
        if (start_pos >= window - 1) {
            int32_t cursor = start_pos % window, n = 0;
            for (int32_t k = cursor + 1; k < window; ++k) out[n++] = k;
            for (int32_t k = 0; k <= cursor; ++k) out[n++] = k;
        } else {
            int32_t n = 0;
            for (int32_t k = 0; k <= start_pos; ++k) out[n++] = k;
            for (int32_t k = 0; k < window - start_pos - 1; ++k) out[n++] = -1;
        }
        return MRO_OK;
    }
    int32_t width = seq_len < window ? seq_len : window;
    *out_rows = seq_len;
    *out_cols = width;
    for (int32_t pos = 0; pos < seq_len; ++pos) {
        int32_t first = pos - window + 1;
        if (first < 0) first = 0;
        for (int32_t col = 0; col < width; ++col) {
            int32_t cand = first + col;
            out[(int64_t)pos * width + col] = cand <= pos ? cand : -1;
        }
    }
    return MRO_OK;
}

/* DeepSeekV4Attention.swift:200-228 */
int mro_compressed_indices(int32_t ratio, int32_t seq_len, int32_t start_pos, int32_t offset,
                           int32_t *out, int32_t *out_rows, int32_t *out_cols) {
    if (!(ratio > 0 && seq_len > 0 && start_pos >= 0 && offset >= 0)) return MRO_INVALID_SHAPE;
    if (start_pos > 0) {
        if (seq_len != 1) return MRO_INVALID_SHAPE;
        int32_t count = (int32_t)(((int64_t)start_pos + 1) / ratio);
        *out_rows = 1;
        *out_cols = count;
        for (int32_t k = 0; k < count; ++k) {
            if ((int64_t)offset + k > 0x7fffffffLL) return MRO_INVALID_SHAPE;
            out[k] = offset + k;
        }
        return MRO_OK;
    }
    int32_t width = seq_len / ratio;
    *out_rows = seq_len;
    *out_cols = width;
    for (int32_t pos = 0; pos < seq_len; ++pos) {
        int32_t visible = (pos + 1) / ratio;
        for (int32_t key = 0; key < width; ++key) {
            if (key < visible && (int64_t)offset + key > 0x7fffffffLL) return MRO_INVALID_SHAPE;
            out[(int64_t)pos * width + key] = key < visible ? offset + key : -1;
        }
    }
    return MRO_OK;
}

/* Linear.swift:55-57: matmul(x, weight.transposed(1, 0)), weight [out, in]. */
void mro_linear(const float *x, int64_t M, const void *w, int w_f32, int64_t out_features,
                int64_t in_features, int64_t w_rs, int acc, float *y, int threads) {
    threads = pick_threads(threads);
#pragma omp parallel for num_threads(threads) schedule(static)
    for (int64_t o = 0; o < out_features; ++o) {
        for (int64_t m = 0; m < M; ++m) {
            const float *xr = x + m * in_features;
            double a64 = 0;
            float a32 = 0.f;
            for (int64_t i = 0; i < in_features; ++i) {
                const float wv = w_f32 ? ((const float *)w)[o * w_rs + i]
                                       : mro_bf16_to_f32(((const uint16_t *)w)[o * w_rs + i]);
                if (acc)
                    a64 += (double)xr[i] * (double)wv;
                else
                    a32 += xr[i] * wv;
            }
            y[m * out_features + o] = acc ? (float)a64 : a32;
        }
    }
}

/* MLA.swift:209-211: merged * sigmoid(k3Linear(x, gProj)). */
void mro_sigmoid_gate(const float *merged, const float *g, int64_t n, float *out) {
    for (int64_t i = 0; i < n; ++i) {
        const float s = 1.0f / (1.0f + expf(-g[i]));
        out[i] = merged[i] * s;
    }
}
