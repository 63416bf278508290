// C-ABI: affine weights, RMSNorm, rotary, cache append, absorption, the
// composed decode block, and the V4 index tables.  Validation first, with
// the reference's messages where it has them; no device memory allocation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <string>

#include "../../include/minirun_hip.h"
#include "capi_util.hpp"
#include "mr_kernels.hpp"

using mrc::aligned16;
using mrc::align256;
using mrc::dtype_name;
using mrc::fail;
using mrc::hip_fail;
using mrc::WS_LIMIT;
using mrc::ws_add;
using mrc::ws_mul;

namespace {

std::string shape_str(int32_t rank, const int64_t* dims) {
    std::string s = "[";
    for (int32_t i = 0; i < rank; ++i) {
        if (i) s += ", ";
        s += std::to_string(dims[i]);
    }
    return s + "]";
}

bool is_float_dtype(mr_dtype d) { return d == MR_BF16 || d == MR_F16 || d == MR_F32; }
int scale_code(mr_dtype d) { return d == MR_BF16 ? 0 : (d == MR_F16 ? 1 : 2); }

mr_status check_weight(const mr_affine_weight* w, const char* what) {
    if (!w) return fail(MR_INVALID_ARGUMENT, "%s: weight descriptor is NULL", what);
    if (!w->packed || !w->scales || !w->biases)
        return fail(MR_INVALID_ARGUMENT, "%s: packed, scales and biases must be non-NULL", what);
    if (!is_float_dtype(w->scale_dtype))
        return fail(MR_INVALID_DTYPE,
                    "affine scales must be a floating-point type — .bfloat16 for this checkpoint, .float16 or "
                    ".float32 for others — got %s", dtype_name(w->scale_dtype));
    if (w->bits <= 0 || 32 % w->bits != 0)
        return fail(MR_INVALID_SHAPE, "bits %d must divide 32 for the uint32 packing", w->bits);
    if (w->group <= 0) return fail(MR_INVALID_SHAPE, "group size must be positive");
    if (w->out_features <= 0 || w->in_features <= 0)
        return fail(MR_INVALID_SHAPE, "%s: out_features %lld and in_features %lld must be positive", what,
                    (long long)w->out_features, (long long)w->in_features);
    if (w->in_features % w->group != 0)
        return fail(MR_INVALID_SHAPE,
                    "inFeatures %lld is not a multiple of the group size %d; partial final groups are not supported",
                    (long long)w->in_features, w->group);
    if (w->in_features % (32 / w->bits) != 0)
        return fail(MR_INVALID_SHAPE, "%s: in_features %lld does not fill whole uint32 words", what,
                    (long long)w->in_features);
    if (!mrc::aligned4(w->packed) || !mrc::aligned4(w->scales) || !mrc::aligned4(w->biases))
        return fail(MR_INVALID_ARGUMENT, "%s: packed, scales and biases must be 4-byte aligned", what);
    return MR_OK;
}

bool act_dtype_ok(mr_dtype d) { return d == MR_BF16 || d == MR_F32; }

mr::AffineGemvParams gemv_params(const mr_affine_weight* w);

// y = W . RMSNorm(x) (norm_w non-null) or y = W . x for one bf16 token:
// the norm rides in the GEMV's staging of x when the 4-bit fast path takes
// the weight, else it runs as its own stage into `norm_buf`.
mr_status block_gemv(const void* x, int64_t in, const mr_affine_weight* w, void* y, const void* norm_w,
                     mr_dtype norm_dtype, float eps, void* norm_buf, void* stream) {
    mr::AffineGemvParams g = gemv_params(w);
    g.x = x;
    g.x_f32 = 0;
    g.x_stride = in;
    g.m = 1;
    g.y = y;
    g.y_f32 = 0;
    g.y_stride_row = 1;
    g.y_stride_token = w->out_features;
    g.force_generic = !aligned16(w->packed);
    g.norm_w = norm_w;
    g.norm_w_f32 = norm_dtype == MR_F32;
    g.norm_eps = eps;
    if (norm_w && !mr::affine_gemv_fast_ok(g)) {
        mr_status st = mr_rmsnorm(x, MR_BF16, 1, (int32_t)in, in, norm_w, norm_dtype, eps, norm_buf, MR_BF16, in, stream);
        if (st != MR_OK) return st;
        g.x = norm_buf;
        g.norm_w = nullptr;
    }
    const hipError_t e = mr::launch_affine_gemv(g, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "affine matmul launch");
}

// The same for two weights of one activation vector (q_a and kv_a of the
// block input) as one launch when both take the fast path, sharing the
// norm: fused in both, or one stage into `norm_buf` for both.
mr_status block_gemv_pair(const void* x, int64_t in, const mr_affine_weight* wa, void* ya, const mr_affine_weight* wb,
                          void* yb, const void* norm_w, mr_dtype norm_dtype, float eps, void* norm_buf, void* stream) {
    mr::AffineGemvParams g[2] = {gemv_params(wa), gemv_params(wb)};
    const mr_affine_weight* w[2] = {wa, wb};
    void* y[2] = {ya, yb};
    for (int i = 0; i < 2; ++i) {
        g[i].x = x;
        g[i].x_f32 = 0;
        g[i].x_stride = in;
        g[i].m = 1;
        g[i].y = y[i];
        g[i].y_f32 = 0;
        g[i].y_stride_row = 1;
        g[i].y_stride_token = w[i]->out_features;
        g[i].force_generic = !aligned16(w[i]->packed);
        g[i].norm_w = norm_w;
        g[i].norm_w_f32 = norm_dtype == MR_F32;
        g[i].norm_eps = eps;
    }
    if (norm_w && !(mr::affine_gemv_fast_ok(g[0]) && mr::affine_gemv_fast_ok(g[1]))) {
        mr_status st = mr_rmsnorm(x, MR_BF16, 1, (int32_t)in, in, norm_w, norm_dtype, eps, norm_buf, MR_BF16, in, stream);
        if (st != MR_OK) return st;
        for (auto& gi : g) {
            gi.x = norm_buf;
            gi.norm_w = nullptr;
        }
    }
    const hipError_t e = mr::launch_affine_gemv_pair(g[0], g[1], (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "affine matmul launch");
}

mr_status check_dense(const mr_dense_weight* w, const char* what) {
    if (!w) return fail(MR_INVALID_ARGUMENT, "%s: weight descriptor is NULL", what);
    if (!w->weight) return fail(MR_INVALID_ARGUMENT, "%s: weight is NULL", what);
    if (w->dtype != MR_BF16 && w->dtype != MR_F32)
        return fail(MR_INVALID_DTYPE, "%s: a dense weight is bf16 or f32, got %s", what, dtype_name(w->dtype));
    if (w->out_features <= 0 || w->in_features <= 0 || w->out_features > INT32_MAX || w->in_features > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "%s: out_features %lld and in_features %lld must be positive int32", what,
                    (long long)w->out_features, (long long)w->in_features);
    const int vpc = w->dtype == MR_F32 ? 4 : 8;  // values per 16-byte chunk
    if (w->in_features % vpc)
        return fail(MR_INVALID_SHAPE, "%s: in_features %lld must be a multiple of %d (16-byte row chunks)", what,
                    (long long)w->in_features, vpc);
    if (w->row_stride < w->in_features || w->row_stride % vpc || !aligned16(w->weight))
        return fail(MR_INVALID_ARGUMENT, "%s: rows must be 16-byte aligned with a row stride >= in_features", what);
    return MR_OK;
}

mr_status check_projection(const mr_projection* p, const char* what) {
    if (!p) return fail(MR_INVALID_ARGUMENT, "%s: projection is NULL", what);
    if (p->kind == MR_PROJ_AFFINE) return check_weight(&p->affine, what);
    if (p->kind == MR_PROJ_DENSE) return check_dense(&p->dense, what);
    return fail(MR_INVALID_ARGUMENT, "%s: projection kind %d is not MR_PROJ_AFFINE or MR_PROJ_DENSE", what,
                (int)p->kind);
}

int64_t proj_out(const mr_projection* p) { return p->kind == MR_PROJ_AFFINE ? p->affine.out_features : p->dense.out_features; }
int64_t proj_in(const mr_projection* p) { return p->kind == MR_PROJ_AFFINE ? p->affine.in_features : p->dense.in_features; }

mr::DenseGemvParams dense_params(const mr_dense_weight* w) {
    mr::DenseGemvParams g{};
    g.w = w->weight;
    g.w_f32 = w->dtype == MR_F32;
    g.w_rs = w->row_stride;
    g.out_rows = (int)w->out_features;
    g.in = (int)w->in_features;
    g.map_a = (int)w->out_features;
    g.m = 1;
    return g;
}

// x_eff = x * sigmoid(g) as bf16 into out (the gate as its own stage, for
// projections whose kernel cannot apply it while staging x)
mr_status gate_stage(const void* x, const void* g, int64_t n, void* out, void* stream) {
    const hipError_t e = mr::launch_gate_mul((const uint16_t*)x, (const uint16_t*)g, n, (uint16_t*)out,
                                             (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "gate launch");
}

// y = W . x_eff for one bf16 token, x_eff = x, RMSNorm(x) (norm_w) or
// x * sigmoid(gate) (gate): fused into the projection's staging of x where
// its kernel can, else as a stage of its own into `stage_buf` (in elements).
mr_status block_proj(const void* x, int64_t in, const mr_projection* w, void* y, const void* norm_w,
                     mr_dtype norm_dtype, float eps, const void* gate, void* stage_buf, void* stream) {
    if (w->kind == MR_PROJ_AFFINE) {
        if (gate) {
            mr_status st = gate_stage(x, gate, in, stage_buf, stream);
            if (st != MR_OK) return st;
            x = stage_buf;
        }
        return block_gemv(x, in, &w->affine, y, norm_w, norm_dtype, eps, stage_buf, stream);
    }
    mr::DenseGemvParams g = dense_params(&w->dense);
    g.x = x;
    g.x_f32 = 0;
    g.x_stride = in;
    g.y = y;
    g.y_f32 = 0;
    g.y_stride_row = 1;
    g.y_stride_token = w->dense.out_features;
    const bool staged = in * 2 <= mr::DENSE_STAGE_BYTES;  // one bf16 vector in LDS
    if (staged) {
        g.norm_w = norm_w;
        g.norm_w_f32 = norm_dtype == MR_F32;
        g.norm_eps = eps;
        g.gate = gate;
        g.gate_f32 = 0;
        g.gate_stride = in;
    } else if (norm_w || gate) {
        mr_status st = norm_w ? mr_rmsnorm(x, MR_BF16, 1, (int32_t)in, in, norm_w, norm_dtype, eps, stage_buf, MR_BF16,
                                           in, stream)
                              : gate_stage(x, gate, in, stage_buf, stream);
        if (st != MR_OK) return st;
        g.x = stage_buf;
    }
    const hipError_t e = mr::launch_dense_gemv(g, staged, mrc::cu_count(), (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "dense projection launch");
}

// Dense projections of one bf16 activation vector stacked into one staged
// launch (x_eff = x or RMSNorm(x) staged once): true when every weight is
// dense with the same dtype and width and the vector fits the staging.
bool dense_stack_ok(const mr_projection* const* w, int n, int64_t in) {
    if (n < 1 || n > 3 || in * 2 > mr::DENSE_STAGE_BYTES) return false;
    int64_t rows = 0;
    for (int i = 0; i < n; ++i) {
        if (w[i]->kind != MR_PROJ_DENSE || w[i]->dense.dtype != w[0]->dense.dtype || w[i]->dense.in_features != in)
            return false;
        rows += w[i]->dense.out_features;
    }
    return rows <= INT32_MAX;
}

mr_status dense_stack(const void* x, int64_t in, const mr_projection* const* w, void* const* y, int n,
                      const void* norm_w, mr_dtype norm_dtype, float eps, void* stream) {
    mr::DenseGemvParams g = dense_params(&w[0]->dense);
    g.x = x;
    g.x_f32 = 0;
    g.x_stride = in;
    g.y = y[0];
    g.y_f32 = 0;
    g.y_stride_row = 1;
    g.y_stride_token = w[0]->dense.out_features;
    g.norm_w = norm_w;
    g.norm_w_f32 = norm_dtype == MR_F32;
    g.norm_eps = eps;
    g.nseg = n;
    int64_t end = 0;
    for (int i = 0; i < n; ++i) {
        end += w[i]->dense.out_features;
        g.seg_end[i] = (int)end;
        g.seg_w[i] = w[i]->dense.weight;
        g.seg_w_rs[i] = w[i]->dense.row_stride;
        g.seg_y[i] = y[i];
        g.seg_y_ts[i] = w[i]->dense.out_features;
    }
    for (int i = n; i < 3; ++i) g.seg_end[i] = (int)end;
    g.out_rows = (int)end;
    g.map_a = (int)end;
    const hipError_t e = mr::launch_dense_gemv(g, true, mrc::cu_count(), (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "dense projection launch");
}

mr::AffineGemvParams gemv_params(const mr_affine_weight* w) {
    mr::AffineGemvParams g{};
    g.packed = w->packed;
    g.scales = w->scales;
    g.biases = w->biases;
    g.scale_dtype = scale_code(w->scale_dtype);
    g.out_rows = (int)w->out_features;
    g.in_features = (int)w->in_features;
    g.group = w->group;
    g.bits = w->bits;
    g.map_a = (int)w->out_features;
    g.map_b = 0;
    g.map_c = 0;
    g.x_div = 1;
    return g;
}

}  // namespace

extern "C" {

mr_status mr_affine_validate(mr_dtype packed_dtype, int32_t packed_rank, const int64_t* ps, mr_dtype scales_dtype,
                             int32_t scales_rank, const int64_t* ss, mr_dtype biases_dtype, int32_t biases_rank,
                             const int64_t* bs, int32_t group, int32_t bits, int64_t* experts, int64_t* out_features,
                             int64_t* in_features) {
    // AffineWeights.swift:84-157, same order
    if (packed_dtype != MR_U32)
        return fail(MR_INVALID_DTYPE,
                    "packed affine weights must be .uint32 (the little-endian reinterpretation of the checkpoint's "
                    "stream), got %s", dtype_name(packed_dtype));
    if (!is_float_dtype(scales_dtype))
        return fail(MR_INVALID_DTYPE,
                    "affine scales must be a floating-point type — .bfloat16 for this checkpoint, .float16 or "
                    ".float32 for others — got %s", dtype_name(scales_dtype));
    if (scales_dtype != biases_dtype)
        return fail(MR_INVALID_DTYPE, "scales are %s but biases are %s; MLX emits both in one dtype",
                    dtype_name(scales_dtype), dtype_name(biases_dtype));
    if (packed_rank < 0 || scales_rank < 0 || biases_rank < 0 || packed_rank > 8 || scales_rank > 8 || biases_rank > 8 ||
        (packed_rank && !ps) || (scales_rank && !ss) || (biases_rank && !bs))
        return fail(MR_INVALID_ARGUMENT, "affine validation: bad shape arrays");
    bool same = scales_rank == biases_rank;
    for (int32_t i = 0; same && i < scales_rank; ++i) same = ss[i] == bs[i];
    if (!same)
        return fail(MR_INVALID_SHAPE, "scales %s and biases %s must have one shape", shape_str(scales_rank, ss).c_str(),
                    shape_str(biases_rank, bs).c_str());
    if (!(packed_rank == scales_rank && (packed_rank == 2 || packed_rank == 3)))
        return fail(MR_INVALID_SHAPE,
                    "packed %s and scales %s must both be rank 2 (one matrix) or rank 3 (an expert stack), and must agree",
                    shape_str(packed_rank, ps).c_str(), shape_str(scales_rank, ss).c_str());
    if (bits <= 0 || 32 % bits != 0) return fail(MR_INVALID_SHAPE, "bits %d must divide 32 for the uint32 packing", bits);
    if (group <= 0) return fail(MR_INVALID_SHAPE, "group size must be positive");
    const int64_t ex = packed_rank == 3 ? ps[0] : 0;
    if (packed_rank == 3 && ss[0] != ex)
        return fail(MR_INVALID_SHAPE, "expert count differs: packed has %lld, scales has %lld", (long long)ex,
                    (long long)ss[0]);
    const int64_t out = ps[packed_rank - 2];
    if (ss[scales_rank - 2] != out)
        return fail(MR_INVALID_SHAPE, "row count differs: packed has %lld, scales has %lld", (long long)out,
                    (long long)ss[scales_rank - 2]);
    const int64_t in = ps[packed_rank - 1] * (32 / bits);
    if (in % group != 0)
        return fail(MR_INVALID_SHAPE,
                    "inFeatures %lld is not a multiple of the group size %d; partial final groups are not supported",
                    (long long)in, group);
    const int64_t expected = in / group;
    if (ss[scales_rank - 1] != expected)
        return fail(MR_INVALID_SHAPE,
                    "group count differs: %lld input features at group size %d need %lld scales per row, got %lld",
                    (long long)in, group, (long long)expected, (long long)ss[scales_rank - 1]);
    if (experts) *experts = ex;
    if (out_features) *out_features = out;
    if (in_features) *in_features = in;
    return MR_OK;
}

mr_status mr_affine_dequantize(const mr_affine_weight* w, void* out, mr_dtype out_dtype, void* stream) {
    mr_status st = check_weight(w, "affine dequantize");
    if (st != MR_OK) return st;
    if (!out) return fail(MR_INVALID_ARGUMENT, "affine dequantize: out is NULL");
    if (!act_dtype_ok(out_dtype)) return fail(MR_INVALID_DTYPE, "affine dequantize: out dtype must be bf16 or f32");
    mr::AffineDequantParams p{};
    p.packed = w->packed;
    p.scales = w->scales;
    p.biases = w->biases;
    p.scale_dtype = scale_code(w->scale_dtype);
    p.out_features = w->out_features;
    p.in_features = w->in_features;
    p.group = w->group;
    p.bits = w->bits;
    p.out = out;
    p.out_f32 = out_dtype == MR_F32;
    const hipError_t e = mr::launch_affine_dequant(p, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "affine dequantize launch");
}

mr_status mr_affine_matmul(const void* x, mr_dtype x_dtype, int32_t tokens, int64_t x_stride, const mr_affine_weight* w,
                           void* y, mr_dtype y_dtype, int64_t y_stride, void* stream) {
    mr_status st = check_weight(w, "affine matmul");
    if (st != MR_OK) return st;
    if (!x || !y) return fail(MR_INVALID_ARGUMENT, "affine matmul: x and y must be non-NULL");
    if (!act_dtype_ok(x_dtype) || !act_dtype_ok(y_dtype))
        return fail(MR_INVALID_DTYPE, "affine matmul: x and y must be bf16 or f32");
    if (tokens <= 0) return fail(MR_INVALID_SHAPE, "affine matmul: tokens %d must be positive", tokens);
    if (x_stride < w->in_features || y_stride < w->out_features)
        return fail(MR_INVALID_SHAPE, "affine matmul: x rows need %lld features, y rows %lld",
                    (long long)w->in_features, (long long)w->out_features);
    if (w->in_features > INT32_MAX || w->out_features > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "affine matmul: dimensions exceed int32");
    mr::AffineGemvParams g = gemv_params(w);
    g.x = x;
    g.x_f32 = x_dtype == MR_F32;
    g.x_stride = x_stride;
    g.m = tokens;
    g.y = y;
    g.y_f32 = y_dtype == MR_F32;
    g.y_stride_row = 1;
    g.y_stride_token = y_stride;
    g.force_generic = !aligned16(w->packed);  // the fused kernel loads 16-byte row chunks
    if (tokens >= mr::PROJ_GEMM_MIN_TOKENS && x_dtype == MR_BF16) {
        // many tokens: dequantized k-tiles into LDS and MFMA
        mr::ProjGemmParams q{};
        q.x = (const uint16_t*)x;
        q.ldx = x_stride;
        q.packed = w->packed;
        q.scales = w->scales;
        q.biases = w->biases;
        q.scale_dtype = scale_code(w->scale_dtype);
        q.group = w->group;
        q.bits = w->bits;
        q.y = y;
        q.ldy = y_stride;
        q.y_f32 = y_dtype == MR_F32;
        q.M = tokens;
        q.N = (int)w->out_features;
        q.K = (int)w->in_features;
        if (mr::proj_gemm_ok(q)) {
            const hipError_t e = mr::launch_proj_gemm(q, mrc::cu_count(), (hipStream_t)stream);
            return e == hipSuccess ? MR_OK : hip_fail(e, "affine matmul launch");
        }
    }
    const hipError_t e = mr::launch_affine_gemv(g, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "affine matmul launch");
}

mr_status mr_linear(const void* x, mr_dtype x_dtype, int32_t tokens, int64_t x_stride, const mr_dense_weight* w,
                    void* y, mr_dtype y_dtype, int64_t y_stride, void* stream) {
    // k3Linear, Linear.swift:55-57
    mr_status st = check_dense(w, "linear");
    if (st != MR_OK) return st;
    if (!x || !y) return fail(MR_INVALID_ARGUMENT, "linear: x and y must be non-NULL");
    if (!act_dtype_ok(x_dtype) || !act_dtype_ok(y_dtype)) return fail(MR_INVALID_DTYPE, "linear: x and y must be bf16 or f32");
    if (tokens <= 0) return fail(MR_INVALID_SHAPE, "linear: tokens %d must be positive", tokens);
    if (x_stride < w->in_features || y_stride < w->out_features)
        return fail(MR_INVALID_SHAPE, "linear: x rows need %lld features, y rows %lld", (long long)w->in_features,
                    (long long)w->out_features);
    // the GEMV reads activation vectors in 16-byte chunks (past its last row
    // a wave still loads one chunk of the vector): at least one whole chunk
    if (w->in_features * (x_dtype == MR_F32 ? 4 : 2) < 16)
        return fail(MR_INVALID_SHAPE, "linear: an activation row of %lld %s values is under 16 bytes",
                    (long long)w->in_features, dtype_name(x_dtype));
    if (tokens >= mr::PROJ_GEMM_MIN_TOKENS && x_dtype == MR_BF16 && w->dtype == MR_BF16) {
        // many tokens: MFMA tiles
        mr::ProjGemmParams q{};
        q.x = (const uint16_t*)x;
        q.ldx = x_stride;
        q.w = (const uint16_t*)w->weight;
        q.ldw = w->row_stride;
        q.y = y;
        q.ldy = y_stride;
        q.y_f32 = y_dtype == MR_F32;
        q.M = tokens;
        q.N = (int)w->out_features;
        q.K = (int)w->in_features;
        if (mr::proj_gemm_ok(q)) {
            const hipError_t e = mr::launch_proj_gemm(q, mrc::cu_count(), (hipStream_t)stream);
            return e == hipSuccess ? MR_OK : hip_fail(e, "linear launch");
        }
    }
    mr::DenseGemvParams g = dense_params(w);
    g.x = x;
    g.x_f32 = x_dtype == MR_F32;
    g.x_stride = x_stride;
    g.m = tokens;
    g.y = y;
    g.y_f32 = y_dtype == MR_F32;
    g.y_stride_row = 1;
    g.y_stride_token = y_stride;
    const bool staged = w->in_features * (x_dtype == MR_F32 ? 4 : 2) <= mr::DENSE_STAGE_BYTES;
    const hipError_t e = mr::launch_dense_gemv(g, staged, mrc::cu_count(), (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "linear launch");
}

mr_status mr_affine_tile_view(const void* tile, int64_t rows, int64_t cols, int32_t group, int32_t bits,
                              mr_dtype scale_dtype, mr_affine_weight* out, int64_t* tile_bytes) {
    // QuantizedTileContainer.swift:560-620, affine mode, one scale row per row
    constexpr int64_t kAlign = 16384;
    if (!out) return fail(MR_INVALID_ARGUMENT, "affine tile view: out is NULL");
    if (rows <= 0 || cols <= 0 || group <= 0 || bits <= 0 || 32 % bits != 0)
        return fail(MR_INVALID_SHAPE, "affine tile view: rows %lld, cols %lld, group %d, bits %d", (long long)rows,
                    (long long)cols, group, bits);
    if (!is_float_dtype(scale_dtype))
        return fail(MR_INVALID_DTYPE, "affine scales are a floating-point type; e8m0 is an MX encoding");
    if (cols % group != 0)
        return fail(MR_INVALID_SHAPE,
                    "cols %lld must be a multiple of the group size %d; partial final groups are not supported",
                    (long long)cols, group);
    const int per_word = 32 / bits;
    if (cols % per_word != 0)
        return fail(MR_INVALID_SHAPE, "cols %lld must be a multiple of %d (%d %d-bit elements per uint32)",
                    (long long)cols, per_word, per_word, bits);
    const int64_t packed_bytes = rows * cols * bits / 8;
    const int64_t scale_bytes = rows * (cols / group) * (scale_dtype == MR_F32 ? 4 : 2);
    if (packed_bytes % kAlign != 0)
        return fail(MR_INVALID_SHAPE,
                    "packed bytes per tile (%lld) must be a multiple of %lld so the scale sub-region starts aligned "
                    "and can be adopted as its own zero-copy array; try rows*cols*bits divisible by %lld",
                    (long long)packed_bytes, (long long)kAlign, (long long)kAlign * 8);
    if (scale_bytes % kAlign != 0)
        return fail(MR_INVALID_SHAPE,
                    "scale bytes per tile (%lld) must be a multiple of %lld; try rows*cols divisible by %lld",
                    (long long)scale_bytes, (long long)kAlign,
                    (long long)(kAlign * group / (scale_dtype == MR_F32 ? 4 : 2)));
    if (!tile) return fail(MR_INVALID_ARGUMENT, "affine tile view: tile is NULL");
    const char* base = (const char*)tile;
    out->packed = (const uint32_t*)base;
    out->scales = base + packed_bytes;
    out->biases = base + packed_bytes + scale_bytes;
    out->scale_dtype = scale_dtype;
    out->out_features = rows;
    out->in_features = cols;
    out->group = group;
    out->bits = bits;
    if (tile_bytes) *tile_bytes = packed_bytes + 2 * scale_bytes;
    return MR_OK;
}

mr_status mr_tile_upload(void* device_dst, const void* pinned_src, int64_t bytes, void* stream) {
    if (bytes < 0) return fail(MR_INVALID_ARGUMENT, "tile upload: negative size");
    if (bytes == 0) return MR_OK;
    if (!device_dst || !pinned_src) return fail(MR_INVALID_ARGUMENT, "tile upload: NULL pointer");
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, pinned_src) != hipSuccess || at.type != hipMemoryTypeHost) {
        (void)hipGetLastError();  // clear the query's error for the next call
        return fail(MR_INVALID_ARGUMENT, "tile upload: the source is not pinned host memory");
    }
    const hipError_t e = hipMemcpyAsync(device_dst, pinned_src, size_t(bytes), hipMemcpyHostToDevice,
                                        (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "tile upload");
}

mr_status mr_affine_gather_matmul(const void* x, mr_dtype x_dtype, int32_t tokens, int64_t x_stride,
                                  const mr_affine_weight* w, int64_t experts, const int32_t* rhs_indices,
                                  int32_t experts_per_token, void* y, mr_dtype y_dtype, void* stream) {
    // AffineWeights.swift:283-318: the reference's preconditions, as errors
    if (experts <= 0)
        return fail(MR_INVALID_ARGUMENT,
                    "affineGatherMM needs a stacked AffineWeights; use affineMM for a single matrix");
    if (tokens < 0 || experts_per_token <= 0)
        return fail(MR_INVALID_ARGUMENT, "rhsIndices must be [tokens, expertsPerToken] matching x's token count");
    mr_status st = check_weight(w, "affine gather matmul");
    if (st != MR_OK) return st;
    if (tokens == 0) return MR_OK;
    if (!x || !y || !rhs_indices)
        return fail(MR_INVALID_ARGUMENT, "affine gather matmul: x, rhs_indices and y must be non-NULL");
    if (!act_dtype_ok(x_dtype) || !act_dtype_ok(y_dtype))
        return fail(MR_INVALID_DTYPE, "affine gather matmul: x and y must be bf16 or f32");
    if (x_stride < w->in_features)
        return fail(MR_INVALID_SHAPE, "affine gather matmul: x rows need %lld features", (long long)w->in_features);
    const int64_t pairs = int64_t(tokens) * experts_per_token;
    if (w->in_features > INT32_MAX || pairs * w->out_features > INT32_MAX || experts * w->out_features > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "affine gather matmul: dimensions exceed int32");
    mr::AffineGemvParams g = gemv_params(w);
    g.x = x;
    g.x_f32 = x_dtype == MR_F32;
    g.x_stride = x_stride;
    g.x_div = experts_per_token;
    g.m = 1;
    g.out_rows = (int)(pairs * w->out_features);  // [tokens][experts_per_token][out]
    g.rhs_idx = rhs_indices;
    g.experts = experts;
    g.y = y;
    g.y_f32 = y_dtype == MR_F32;
    g.y_stride_row = 1;
    g.y_stride_token = g.out_rows;
    g.force_generic = !aligned16(w->packed);
    const hipError_t e = mr::launch_affine_gemv(g, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "affine gather matmul launch");
}

mr_status mr_rmsnorm(const void* x, mr_dtype x_dtype, int64_t rows, int32_t dim, int64_t x_stride, const void* weight,
                     mr_dtype w_dtype, float eps, void* out, mr_dtype out_dtype, int64_t out_stride, void* stream) {
    if (!x || !weight || !out) return fail(MR_INVALID_ARGUMENT, "rmsnorm: NULL pointer");
    if (!act_dtype_ok(x_dtype) || !act_dtype_ok(w_dtype) || !act_dtype_ok(out_dtype))
        return fail(MR_INVALID_DTYPE, "rmsnorm: dtypes must be bf16 or f32");
    if (rows <= 0 || dim <= 0 || x_stride < dim || out_stride < dim || rows > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "rmsnorm: rows %lld, dim %d, strides %lld/%lld", (long long)rows, dim,
                    (long long)x_stride, (long long)out_stride);
    if (!(eps >= 0) || !std::isfinite(eps)) return fail(MR_INVALID_ARGUMENT, "rmsnorm: eps must be finite, >= 0");
    mr::RmsNormParams p{x, x_dtype == MR_F32, x_stride, weight, w_dtype == MR_F32, out, out_dtype == MR_F32,
                        out_stride, rows, dim, eps};
    const hipError_t e = mr::launch_rmsnorm(p, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "rmsnorm launch");
}

mr_status mr_rope_frequencies(int32_t dim, int32_t original_len, double base, double factor, double beta_fast,
                              double beta_slow, double* freqs) {
    // DeepSeekV4Attention.swift:36-99
    if (!(dim > 0 && dim % 2 == 0))
        return fail(MR_INVALID_SHAPE, "rotary dimension must be positive and even, got %d", dim);
    if (original_len < 0) return fail(MR_INVALID_SHAPE, "original rotary sequence length cannot be negative");
    if (!(std::isfinite(base) && base > 1 && std::isfinite(factor) && factor > 0 && std::isfinite(beta_fast) &&
          beta_fast > 0 && std::isfinite(beta_slow) && beta_slow > 0))
        return fail(MR_INVALID_SHAPE, "rotary base, factor, and correction rotations must be finite and positive");
    if (!freqs) return fail(MR_INVALID_ARGUMENT, "rotary frequencies: output is NULL");
    const int half = dim / 2;
    for (int i = 0; i < half; ++i) freqs[i] = 1.0 / std::pow(base, double(i * 2) / double(dim));
    if (original_len > 0) {
        auto corr = [&](double rot) {
            return double(dim) * std::log(double(original_len) / (rot * 2.0 * M_PI)) / (2.0 * std::log(base));
        };
        const int64_t low = std::max<int64_t>(int64_t(std::floor(corr(beta_fast))), 0);
        const int64_t high = std::min<int64_t>(int64_t(std::ceil(corr(beta_slow))), dim - 1);
        const double den = low == high ? 0.001 : double(high - low);
        for (int i = 0; i < half; ++i) {
            const double ramp = std::min(std::max((double(i) - double(low)) / den, 0.0), 1.0);
            const double smooth = 1.0 - ramp;
            freqs[i] = freqs[i] / factor * (1.0 - smooth) + freqs[i] * smooth;
        }
    }
    for (int i = 0; i < half; ++i)
        if (!(std::isfinite(freqs[i]) && freqs[i] > 0))
            return fail(MR_NONFINITE, "rotary frequency table is not finite and positive");
    return MR_OK;
}

mr_status mr_rope_table(const int64_t* positions, int64_t n_pos, const double* freqs, int32_t half, int32_t inverse,
                        float* cos_out, float* sin_out) {
    // DeepSeekV4Attention.swift:126-149
    if (n_pos < 0 || half <= 0 || (n_pos && (!positions || !freqs || !cos_out || !sin_out)))
        return fail(MR_INVALID_ARGUMENT, "rotary table: bad arguments");
    for (int64_t i = 0; i < n_pos; ++i)
        if (positions[i] < 0) return fail(MR_INVALID_SHAPE, "rotary positions cannot be negative");
    const double dir = inverse ? -1.0 : 1.0;
    for (int64_t i = 0; i < n_pos; ++i)
        for (int32_t k = 0; k < half; ++k) {
            const double a = dir * double(positions[i]) * freqs[k];
            if (!std::isfinite(a)) return fail(MR_NONFINITE, "rotary angle is not finite");
            cos_out[i * half + k] = float(std::cos(a));
            sin_out[i * half + k] = float(std::sin(a));
        }
    return MR_OK;
}

mr_status mr_rope_apply(void* x, mr_dtype dtype, int64_t n_pos, int64_t inner, int64_t row_stride, int64_t col0,
                        int32_t dim, const float* cos_t, const float* sin_t, void* stream) {
    if (!x || !cos_t || !sin_t) return fail(MR_INVALID_ARGUMENT, "rotary apply: NULL pointer");
    if (!act_dtype_ok(dtype))
        return fail(MR_INVALID_DTYPE, "rotary input must have a real floating-point dtype (bf16 or f32 here)");
    if (!(dim > 0 && dim % 2 == 0) || n_pos < 0 || inner <= 0 || col0 < 0 || col0 + dim > row_stride)
        return fail(MR_INVALID_SHAPE, "rotary input must be [sequence, ..., %d] with one position per sequence row", dim);
    if (n_pos == 0) return MR_OK;
    mr::RopeParams p{x, dtype == MR_F32, n_pos, inner, row_stride, col0, dim, cos_t, sin_t};
    const hipError_t e = mr::launch_rope(p, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "rotary launch");
}

mr_status mr_mla_cache_append(const void* kv, mr_dtype kv_dtype, int64_t kv_stride, int64_t tokens, const void* norm_w,
                              mr_dtype w_dtype, float eps, int32_t kv_rank, int32_t rope_dim, const float* cos_t,
                              const float* sin_t, void* latent, int64_t latent_row_stride, void* rope,
                              int64_t rope_row_stride, int64_t start_row, void* stream) {
    if (!kv || !norm_w || !latent || (rope_dim && !rope))
        return fail(MR_INVALID_ARGUMENT, "cache append: NULL pointer");
    if (!cos_t != !sin_t) return fail(MR_INVALID_ARGUMENT, "cache append: give both rotary tables or neither (NoPE)");
    if (!act_dtype_ok(kv_dtype) || !act_dtype_ok(w_dtype)) return fail(MR_INVALID_DTYPE, "cache append: dtypes");
    if (tokens <= 0 || kv_rank <= 0 || rope_dim < 0 || rope_dim % 2 || kv_stride < kv_rank + rope_dim ||
        latent_row_stride < kv_rank || (rope_dim && rope_row_stride < rope_dim) || start_row < 0 || tokens > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "cache append: bad geometry");
    const mr::CacheAppendParams p{kv,      kv_dtype == MR_F32, kv_stride,         norm_w,       w_dtype == MR_F32,
                                  eps,     kv_rank,            rope_dim,          cos_t,        sin_t,
                                  (uint16_t*)latent, latent_row_stride, (uint16_t*)rope, rope_row_stride, start_row,
                                  tokens};
    const hipError_t e = mr::launch_cache_append(p, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "cache append launch");
}

static mr_status check_kv_b(const mr_projection* kv_b, int32_t heads, int32_t nope_dim, int32_t v_dim) {
    mr_status st = check_projection(kv_b, "kv_b_proj");
    if (st != MR_OK) return st;
    if (kv_b->kind == MR_PROJ_AFFINE) {
        const mr_affine_weight* w = &kv_b->affine;
        if (w->bits != 4 || w->group != 64)
            return fail(MR_INVALID_SHAPE, "kv_b_proj: the absorbed path needs a 4-bit, group-64 affine weight (got %d/%d)",
                        w->bits, w->group);
    }
    if (proj_in(kv_b) != 512)
        return fail(MR_INVALID_SHAPE, "kv_b_proj: in_features must be kv_rank 512, got %lld", (long long)proj_in(kv_b));
    if (heads <= 0 || nope_dim <= 0 || v_dim <= 0 || proj_out(kv_b) != int64_t(heads) * (nope_dim + v_dim))
        return fail(MR_INVALID_SHAPE, "kv_b_proj has %lld rows; heads %d x (nope %d + v %d) expected",
                    (long long)proj_out(kv_b), heads, nope_dim, v_dim);
    return MR_OK;
}

// q_lat[h] = q_nope[h] . W_UK[h], optionally rotating q's rope slice
// (rope_cos non-null) and appending one cache row (app non-null) in the
// same launch
static mr_status absorb(const void* q, int64_t q_head_stride, int32_t heads, int32_t nope_dim, int32_t v_dim,
                        const mr_projection* kv_b, void* q_lat, int64_t q_lat_head_stride, const float* rope_cos,
                        const float* rope_sin, int32_t rope_dim, void* stream,
                        const mr::CacheAppendParams* app = nullptr) {
    hipError_t e;
    if (kv_b->kind == MR_PROJ_AFFINE) {
        const mr_affine_weight* w = &kv_b->affine;
        mr::AbsorbParams p{(const uint16_t*)q, q_head_stride, w->packed, w->scales, w->biases,
                           scale_code(w->scale_dtype), heads, nope_dim, v_dim, 512, (uint16_t*)q_lat, q_lat_head_stride};
        p.rope_cos = rope_cos;
        p.rope_sin = rope_sin;
        p.rope_dim = rope_dim;
        p.rope_col0 = nope_dim;
        if (app) {
            p.app = *app;
            p.app_on = 1;
        }
        e = mr::launch_absorb_q(p, (hipStream_t)stream);
    } else {
        const mr_dense_weight* w = &kv_b->dense;
        mr::DenseAbsorbParams p{};
        p.q = (uint16_t*)q;
        p.q_head_stride = q_head_stride;
        p.w = w->weight;
        p.w_f32 = w->dtype == MR_F32;
        p.w_rs = w->row_stride;
        p.heads = heads;
        p.nope_dim = nope_dim;
        p.v_dim = v_dim;
        p.q_lat = (uint16_t*)q_lat;
        p.q_lat_head_stride = q_lat_head_stride;
        p.rope_cos = rope_cos;
        p.rope_sin = rope_sin;
        p.rope_dim = rope_dim;
        p.rope_col0 = nope_dim;
        if (app) {
            p.app = *app;
            p.app_on = 1;
        }
        e = mr::launch_dense_absorb(p, (hipStream_t)stream);
    }
    return e == hipSuccess ? MR_OK : hip_fail(e, "absorb launch");
}

mr_status mr_mla_absorb_query(const void* q, int64_t q_head_stride, int32_t heads, int32_t nope_dim, int32_t v_dim,
                              const mr_projection* kv_b, void* q_lat, int64_t q_lat_head_stride, void* stream) {
    mr_status st = check_kv_b(kv_b, heads, nope_dim, v_dim);
    if (st != MR_OK) return st;
    if (!q || !q_lat || q_head_stride < nope_dim || q_lat_head_stride < 512)
        return fail(MR_INVALID_ARGUMENT, "absorb query: bad q / q_lat");
    if (kv_b->kind == MR_PROJ_DENSE && nope_dim > 1024)
        return fail(MR_INVALID_SHAPE, "absorb query: nope_dim %d exceeds 1024", nope_dim);
    return absorb(q, q_head_stride, heads, nope_dim, v_dim, kv_b, q_lat, q_lat_head_stride, nullptr, nullptr, 0, stream);
}

mr_status mr_mla_unabsorb_values(const void* ctx, int64_t ctx_head_stride, int32_t heads, int32_t nope_dim,
                                 int32_t v_dim, const mr_projection* kv_b, void* out, mr_dtype out_dtype,
                                 void* stream) {
    mr_status st = check_kv_b(kv_b, heads, nope_dim, v_dim);
    if (st != MR_OK) return st;
    if (!ctx || !out || ctx_head_stride < 512) return fail(MR_INVALID_ARGUMENT, "unabsorb values: bad ctx / out");
    if (!act_dtype_ok(out_dtype)) return fail(MR_INVALID_DTYPE, "unabsorb values: out must be bf16 or f32");
    hipError_t e;
    if (kv_b->kind == MR_PROJ_AFFINE) {
        mr::AffineGemvParams g = gemv_params(&kv_b->affine);
        g.out_rows = heads * v_dim;
        g.map_a = v_dim;
        g.map_b = nope_dim + v_dim;
        g.map_c = nope_dim;
        g.x = ctx;
        g.x_f32 = 0;
        g.x_stride = ctx_head_stride;
        g.m = 1;
        g.y = out;
        g.y_f32 = out_dtype == MR_F32;
        g.y_stride_row = 1;
        g.y_stride_token = int64_t(heads) * v_dim;
        e = mr::launch_affine_gemv(g, (hipStream_t)stream);
    } else {
        mr::DenseGemvParams g = dense_params(&kv_b->dense);
        g.out_rows = heads * v_dim;
        g.map_a = v_dim;
        g.map_b = nope_dim + v_dim;
        g.map_c = nope_dim;
        g.x = ctx;
        g.x_f32 = 0;
        g.x_vec_stride = ctx_head_stride;
        g.m = 1;
        g.y = out;
        g.y_f32 = out_dtype == MR_F32;
        g.y_stride_row = 1;
        g.y_stride_token = int64_t(heads) * v_dim;
        e = mr::launch_dense_gemv(g, false, mrc::cu_count(), (hipStream_t)stream);
    }
    return e == hipSuccess ? MR_OK : hip_fail(e, "unabsorb launch");
}

// ---------------------------------------------------------------- decode block
namespace {

// The split merge and W_UV run as one launch (mla_combine_unabsorb) for a
// 4-bit group-64 affine kv_b with bf16 scales and biases, or a dense bf16
// one, 16-byte aligned, with at most 128 value rows per head (a multiple of
// 64); other weights take the decode's own combine and the grouped GEMV.
bool unabsorb_fuses(const mr_projection* kv_b, int32_t v_dim) {
    if (v_dim % 64 != 0 || v_dim > mr::UNABSORB_MAX_V) return false;
    if (kv_b->kind == MR_PROJ_AFFINE) {
        const mr_affine_weight* w = &kv_b->affine;
        return w->bits == 4 && w->group == 64 && w->scale_dtype == MR_BF16 && aligned16(w->packed) &&
               aligned16(w->scales) && aligned16(w->biases);
    }
    const mr_dense_weight* w = &kv_b->dense;
    return kv_b->kind == MR_PROJ_DENSE && w->dtype == MR_BF16 && aligned16(w->weight) && w->row_stride % 8 == 0;
}

struct BlockLayout {
    size_t h, h_kv, q_lora, q_lora_n, q, q_lat, kv, ctx, attn, gate, stage, dec, total;
    mr_mla_decode_args dec_args;
};

bool block_layout(const mr_mla_block_args* a, BlockLayout* L) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = ws_add(off, align256(bytes));
        return at;
    };
    auto dim = [](int64_t v) { return size_t(std::max<int64_t>(v, 0)); };
    const size_t dq = dim(int64_t(a->qk_nope_dim) + a->qk_rope_dim);
    const size_t H = dim(a->heads);
    const size_t hv = ws_mul(H, dim(a->v_head_dim));
    L->h = take(ws_mul(dim(a->hidden), 2));
    L->h_kv = take(ws_mul(dim(a->hidden), 2));  // the key path's (and the gate's) normed x
    L->q_lora = take(ws_mul(dim(a->q_lora_rank), 2));
    L->q_lora_n = take(ws_mul(dim(a->q_lora_rank), 2));
    L->q = take(ws_mul(ws_mul(H, dq), 2));
    L->q_lat = take(ws_mul(ws_mul(H, dim(a->kv_rank)), 2));
    L->kv = take(ws_mul(dim(int64_t(a->kv_rank) + a->qk_rope_dim), 2));
    L->ctx = take(ws_mul(ws_mul(H, dim(a->kv_rank)), 2));
    L->attn = take(ws_mul(hv, 2));
    L->gate = take(ws_mul(hv, 2));
    L->stage = take(ws_mul(hv, 2));  // the gated o_proj input when the gate is its own stage
    const int dqi = int(std::min<size_t>(dq, INT32_MAX));
    mr_mla_decode_args& d = L->dec_args;
    d = mr_mla_decode_args{};
    d.batch = 1;
    d.heads = a->heads;
    d.n_ctx = a->position + 1;
    d.kv_rank = a->kv_rank;
    d.rope_dim = a->qk_rope_dim;
    d.scale = a->scale;
    d.q_lat_head_stride = a->kv_rank;
    d.q_rope_head_stride = dqi;
    d.latent_row_stride = a->latent_row_stride;
    d.rope_row_stride = a->rope_row_stride;
    d.out_dtype = MR_BF16;
    d.out_head_stride = a->kv_rank;
    L->dec = off;
    const size_t dec_bytes = mr_mla_decode_workspace_size(&d);
    take(dec_bytes);
    L->total = off;
    return true;
}

}  // namespace

size_t mr_mla_decode_block_workspace_size(const mr_mla_block_args* a) {
    if (!a || a->hidden <= 0 || a->q_lora_rank <= 0 || a->heads <= 0 || a->qk_nope_dim < 0 || a->qk_rope_dim < 0 ||
        a->v_head_dim <= 0 || a->kv_rank <= 0 || a->position < 0)
        return 0;
    BlockLayout L;
    block_layout(a, &L);
    return L.total < WS_LIMIT ? L.total : 0;
}

mr_status mr_mla_decode_block(const mr_mla_block_args* a, void* stream) {
    if (!a) return fail(MR_INVALID_ARGUMENT, "mla block: args is NULL");
    if (a->kv_rank != 512 || a->qk_rope_dim != 64 || a->heads <= 0 || a->qk_nope_dim <= 0 || a->v_head_dim <= 0 ||
        a->hidden <= 0 || a->q_lora_rank <= 0)
        return fail(MR_INVALID_SHAPE, "mla block: kv_rank 512, rope 64 and positive dims required");
    if (a->position < 0 || a->position >= a->capacity)
        return fail(MR_INVALID_SHAPE, "mla block: position %d outside the cache capacity %d", a->position, a->capacity);
    if (!a->x || !a->q_a_norm_w || !a->kv_a_norm_w || !a->cache_latent || !a->cache_rope || !a->out || !a->workspace)
        return fail(MR_INVALID_ARGUMENT, "mla block: NULL pointer");
    if (!a->rope_cos != !a->rope_sin)
        return fail(MR_INVALID_ARGUMENT, "mla block: give both rotary tables (rotated MLA) or neither (NoPE)");
    if (a->latent_row_stride < a->kv_rank || a->rope_row_stride < a->qk_rope_dim)  // before any cache write
        return fail(MR_INVALID_SHAPE, "mla block: cache row strides %lld / %lld are below %d / %d",
                    (long long)a->latent_row_stride, (long long)a->rope_row_stride, a->kv_rank, a->qk_rope_dim);
    if (!act_dtype_ok(a->norm_w_dtype)) return fail(MR_INVALID_DTYPE, "mla block: norm weights must be bf16 or f32");
    const int dq = a->qk_nope_dim + a->qk_rope_dim;
    const bool gated = a->g_proj.kind != MR_PROJ_NONE;
    const int64_t hv = int64_t(a->heads) * a->v_head_dim;
    struct {
        const mr_projection* w;
        int64_t out, in;
        const char* name;
    } ws[] = {{&a->q_a, a->q_lora_rank, a->hidden, "q_a_proj"},
              {&a->q_b, int64_t(a->heads) * dq, a->q_lora_rank, "q_b_proj"},
              {&a->kv_a, a->kv_rank + a->qk_rope_dim, a->hidden, "kv_a_proj_with_mqa"},
              {&a->o_proj, a->hidden, hv, "o_proj"},
              {&a->g_proj, hv, a->hidden, "g_proj"}};
    for (auto& e : ws) {
        if (e.w == &a->g_proj && !gated) continue;
        mr_status st = check_projection(e.w, e.name);
        if (st != MR_OK) return st;
        if (proj_out(e.w) != e.out || proj_in(e.w) != e.in)
            return fail(MR_INVALID_SHAPE, "mla block: %s is [%lld, %lld], expected [%lld, %lld]", e.name,
                        (long long)proj_out(e.w), (long long)proj_in(e.w), (long long)e.out, (long long)e.in);
    }
    mr_status st = check_kv_b(&a->kv_b, a->heads, a->qk_nope_dim, a->v_head_dim);
    if (st != MR_OK) return st;
    if (a->kv_b.kind == MR_PROJ_DENSE && a->qk_nope_dim > 1024)
        return fail(MR_INVALID_SHAPE, "mla block: nope dim %d exceeds 1024", a->qk_nope_dim);
    BlockLayout L;
    block_layout(a, &L);
    if (L.total >= WS_LIMIT) return fail(MR_INVALID_SHAPE, "mla block: the workspace these widths need overflows");
    if (a->workspace_bytes < L.total)
        return fail(MR_WORKSPACE_TOO_SMALL, "mla block: workspace %zu bytes < %zu", a->workspace_bytes, L.total);
    if (!aligned16(a->workspace)) return fail(MR_INVALID_ARGUMENT, "mla block: workspace must be 16-byte aligned");
    char* W = (char*)a->workspace;
    void* h = W + L.h;
    void* h_kv = W + L.h_kv;
    void* q_lora = W + L.q_lora;
    void* q_lora_n = W + L.q_lora_n;
    uint16_t* q = (uint16_t*)(W + L.q);
    void* q_lat = W + L.q_lat;
    void* kv = W + L.kv;
    void* ctx = W + L.ctx;
    void* attn = W + L.attn;
    void* gate = W + L.gate;
    void* stage = W + L.stage;
    const mr_dtype nd = a->norm_w_dtype;

    // One stream, in order: the projections of the block input (q_a, kv_a
    // and, gated, g_proj; one stacked launch when they are dense, q_a and
    // kv_a as one launch when they are 4-bit), q_b with
    // its RMSNorm, the absorption (query rotary and the cache append of row
    // `position` ride in it), the decode, W_UV and o_proj (the gate rides in
    // its staging).  A side stream for the key path and the gate cost more
    // in cross-stream waits than it overlapped.
    const mr_projection* xw[3] = {&a->q_a, &a->kv_a, &a->g_proj};
    void* xy[3] = {q_lora, kv, gate};
    void* xs[3] = {h, h_kv, h_kv};  // stage buffers for an input norm that no kernel fuses
    const int nx = gated ? 3 : 2;
    if (dense_stack_ok(xw, nx, a->hidden)) {
        if ((st = dense_stack(a->x, a->hidden, xw, xy, nx, a->input_norm_w, nd, a->eps, stream)) != MR_OK) return st;
    } else if (a->q_a.kind == MR_PROJ_AFFINE && a->kv_a.kind == MR_PROJ_AFFINE) {
        if ((st = block_gemv_pair(a->x, a->hidden, &a->q_a.affine, q_lora, &a->kv_a.affine, kv, a->input_norm_w, nd,
                                  a->eps, h, stream)) != MR_OK)
            return st;
        if (gated && (st = block_proj(a->x, a->hidden, &a->g_proj, gate, a->input_norm_w, nd, a->eps, nullptr, h_kv,
                                      stream)) != MR_OK)
            return st;
    } else {
        for (int i = 0; i < nx; ++i)
            if ((st = block_proj(a->x, a->hidden, xw[i], xy[i], a->input_norm_w, nd, a->eps, nullptr, xs[i], stream)) !=
                MR_OK)
                return st;
    }
    if ((st = block_proj(q_lora, a->q_lora_rank, &a->q_b, q, a->q_a_norm_w, nd, a->eps, nullptr, q_lora_n, stream)) !=
        MR_OK)
        return st;
    const mr::CacheAppendParams app{kv,
                                    0,
                                    a->kv_rank + a->qk_rope_dim,
                                    a->kv_a_norm_w,
                                    nd == MR_F32,
                                    a->eps,
                                    a->kv_rank,
                                    a->qk_rope_dim,
                                    a->rope_cos,
                                    a->rope_sin,
                                    (uint16_t*)a->cache_latent,
                                    a->latent_row_stride,
                                    (uint16_t*)a->cache_rope,
                                    a->rope_row_stride,
                                    a->position,
                                    1};
    if ((st = absorb(q, dq, a->heads, a->qk_nope_dim, a->v_head_dim, &a->kv_b, q_lat, a->kv_rank, a->rope_cos,
                     a->rope_sin, a->qk_rope_dim, stream, &app)) != MR_OK)
        return st;
    mr_mla_decode_args d = L.dec_args;
    d.q_lat = q_lat;
    d.q_rope = q + a->qk_nope_dim;
    d.latent = a->cache_latent;
    d.rope_keys = a->cache_rope;
    d.out = ctx;
    d.workspace = W + L.dec;
    d.workspace_bytes = L.total - L.dec;
    if (unabsorb_fuses(&a->kv_b, a->v_head_dim)) {
        // the split kernel alone, then one launch that merges the splits of
        // each head and un-absorbs them (W_UV) into the o_proj input
        d.flags |= MR_DECODE_SPLIT_ONLY;
        if ((st = mr_mla_decode(&d, stream)) != MR_OK) return st;
        const mrc::DecodePartials dp = mrc::decode_partials(&d);
        mr::CombineUnabsorbParams u{};
        u.ws_o = d.workspace;
        u.ws_f32 = dp.ws_f32;
        u.ws_ml = (const float*)((const char*)d.workspace + dp.ml_offset);
        u.splits = dp.splits;
        u.h_pad = dp.h_pad;
        u.heads = a->heads;
        u.affine = a->kv_b.kind == MR_PROJ_AFFINE;
        if (u.affine) {
            u.packed = a->kv_b.affine.packed;
            u.scales = (const uint16_t*)a->kv_b.affine.scales;
            u.biases = (const uint16_t*)a->kv_b.affine.biases;
        } else {
            u.w = (const uint16_t*)a->kv_b.dense.weight;
            u.w_rs = a->kv_b.dense.row_stride;
        }
        u.row_step = a->qk_nope_dim + a->v_head_dim;
        u.row0 = a->qk_nope_dim;
        u.v_dim = a->v_head_dim;
        u.out = (uint16_t*)attn;
        const hipError_t e = mr::launch_combine_unabsorb(u, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "mla block: merge + W_UV launch");
    } else {
        if ((st = mr_mla_decode(&d, stream)) != MR_OK) return st;
        if ((st = mr_mla_unabsorb_values(ctx, a->kv_rank, a->heads, a->qk_nope_dim, a->v_head_dim, &a->kv_b, attn,
                                         MR_BF16, stream)) != MR_OK)
            return st;
    }
    return block_proj(attn, hv, &a->o_proj, a->out, nullptr, nd, a->eps, gated ? gate : nullptr, stage, stream);
}

// ---------------------------------------------------------------- prefill block
namespace {

// y[t] = W . x[t] for `tokens` bf16 rows into bf16 rows: MFMA tiles from
// 64 tokens, the token-tiled GEMV below that
mr_status proj_rows(const void* x, int32_t tokens, int64_t x_stride, const mr_projection* w, void* y, int64_t y_stride,
                    void* stream) {
    return w->kind == MR_PROJ_AFFINE
               ? mr_affine_matmul(x, MR_BF16, tokens, x_stride, &w->affine, y, MR_BF16, y_stride, stream)
               : mr_linear(x, MR_BF16, tokens, x_stride, &w->dense, y, MR_BF16, y_stride, stream);
}

// Projections of the same bf16 rows into bf16 rows (n of them, up to 3):
// one stacked MFMA launch when every weight takes the MFMA path and all are
// dense bf16 or all affine, else one call each.
mr_status proj_rows_stacked(const void* x, int32_t tokens, int64_t x_stride, const mr_projection* const* w,
                            void* const* y, const int64_t* y_stride, int n, void* stream) {
    mr::ProjGemmParams q[3];
    bool stack = n > 1 && tokens >= mr::PROJ_GEMM_MIN_TOKENS;
    for (int i = 0; stack && i < n; ++i) {
        q[i] = mr::ProjGemmParams{};
        q[i].x = (const uint16_t*)x;
        q[i].ldx = x_stride;
        q[i].y = y[i];
        q[i].ldy = y_stride[i];
        q[i].M = tokens;
        q[i].N = (int)proj_out(w[i]);
        q[i].K = (int)proj_in(w[i]);
        if (w[i]->kind == MR_PROJ_AFFINE) {
            const mr_affine_weight* a = &w[i]->affine;
            q[i].packed = a->packed;
            q[i].scales = a->scales;
            q[i].biases = a->biases;
            q[i].scale_dtype = scale_code(a->scale_dtype);
            q[i].group = a->group;
            q[i].bits = a->bits;
        } else {
            if (w[i]->dense.dtype != MR_BF16) stack = false;
            q[i].w = (const uint16_t*)w[i]->dense.weight;
            q[i].ldw = w[i]->dense.row_stride;
        }
        stack = stack && w[i]->kind == w[0]->kind && mr::proj_gemm_ok(q[i]);
    }
    if (stack) {
        const hipError_t e = mr::launch_proj_gemm_stack(q, n, mrc::cu_count(), (hipStream_t)stream);
        return e == hipSuccess ? MR_OK : hip_fail(e, "stacked projection launch");
    }
    for (int i = 0; i < n; ++i) {
        mr_status st = proj_rows(x, tokens, x_stride, w[i], y[i], y_stride[i], stream);
        if (st != MR_OK) return st;
    }
    return MR_OK;
}

// Workspace regions, 256-byte aligned, each [T][width] bf16 unless noted:
// the normed input (with an input norm), q_lora and its norm, q, the kv_a
// rows, the gate (gated), the attention output, the dequantized kv_b
// (affine kv_b, [H*(nope+v)][kv_rank]) and mr_mla_prefill's own workspace.
struct PrefillBlockLayout {
    size_t h, q_lora, q_lora_n, q, kv, gate, attn, kv_b, pre, total;
    mr_mla_prefill_args pre_args;
};

void prefill_block_layout(const mr_mla_prefill_block_args* a, PrefillBlockLayout* L) {
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t at = off;
        off = ws_add(off, align256(bytes));
        return at;
    };
    auto dim = [](int64_t v) { return size_t(std::max<int64_t>(v, 0)); };
    const size_t T = dim(a->tokens), H = dim(a->heads);
    const int dq = int(std::min<int64_t>(std::max<int64_t>(int64_t(a->qk_nope_dim) + a->qk_rope_dim, 0), INT32_MAX));
    const size_t hv = ws_mul(H, dim(a->v_head_dim));
    L->h = take(a->input_norm_w ? ws_mul(ws_mul(T, dim(a->hidden)), 2) : 0);
    L->q_lora = take(ws_mul(ws_mul(T, dim(a->q_lora_rank)), 2));
    L->q_lora_n = take(ws_mul(ws_mul(T, dim(a->q_lora_rank)), 2));
    L->q = take(ws_mul(ws_mul(ws_mul(T, H), size_t(dq)), 2));
    L->kv = take(ws_mul(ws_mul(T, dim(int64_t(a->kv_rank) + a->qk_rope_dim)), 2));
    L->gate = take(a->g_proj.kind != MR_PROJ_NONE ? ws_mul(ws_mul(T, hv), 2) : 0);
    L->attn = take(ws_mul(ws_mul(T, hv), 2));
    L->kv_b = take(a->kv_b.kind == MR_PROJ_AFFINE
                       ? ws_mul(ws_mul(ws_mul(H, dim(int64_t(a->qk_nope_dim) + a->v_head_dim)), dim(a->kv_rank)), 2)
                       : 0);
    mr_mla_prefill_args& p = L->pre_args;
    p = mr_mla_prefill_args{};
    p.tokens = a->tokens;
    p.n_ctx = int32_t(std::min<int64_t>(int64_t(a->position) + a->tokens, INT32_MAX));
    p.heads = a->heads;
    p.qk_nope_dim = a->qk_nope_dim;
    p.qk_rope_dim = a->qk_rope_dim;
    p.v_head_dim = a->v_head_dim;
    p.kv_rank = a->kv_rank;
    p.scale = a->scale;
    p.q_token_stride = int64_t(a->heads) * dq;
    p.q_head_stride = dq;
    p.latent = a->cache_latent;
    p.latent_row_stride = a->latent_row_stride;
    p.rope_keys = a->cache_rope;
    p.rope_row_stride = a->rope_row_stride;
    if (a->kv_b.kind == MR_PROJ_DENSE) {
        p.kv_b = a->kv_b.dense.weight;
        p.kv_b_row_stride = a->kv_b.dense.row_stride;
    } else {
        p.kv_b_row_stride = a->kv_rank;
    }
    p.out_dtype = MR_BF16;
    p.out_token_stride = int64_t(hv);
    p.out_head_stride = a->v_head_dim;
    L->pre = off;
    take(mr_mla_prefill_workspace_size(&p));
    L->total = off;
}

// Every check the stages would make, before the first launch: a call that
// fails leaves the cache as it was.
mr_status check_prefill_block(const mr_mla_prefill_block_args* a) {
    if (!a) return fail(MR_INVALID_ARGUMENT, "mla prefill block: args is NULL");
    if (a->tokens <= 0 || a->hidden <= 0 || a->q_lora_rank <= 0 || a->heads <= 0 || a->qk_nope_dim < 0 ||
        a->qk_rope_dim < 0 || a->qk_rope_dim % 2 || a->v_head_dim <= 0 || a->kv_rank <= 0)
        return fail(MR_INVALID_SHAPE, "mla prefill block: positive tokens and dims required, an even rope width");
    if (a->position < 0 || int64_t(a->position) + a->tokens > a->capacity)
        return fail(MR_INVALID_SHAPE, "mla prefill block: rows %d .. %lld outside the cache capacity %d", a->position,
                    (long long)a->position + a->tokens - 1, a->capacity);
    if (!a->x || !a->q_a_norm_w || !a->kv_a_norm_w || !a->cache_latent || (a->qk_rope_dim && !a->cache_rope) ||
        !a->out || !a->workspace)
        return fail(MR_INVALID_ARGUMENT, "mla prefill block: NULL pointer");
    if (!a->rope_cos != !a->rope_sin)
        return fail(MR_INVALID_ARGUMENT, "mla prefill block: give both rotary tables (rotated MLA) or neither (NoPE)");
    if (a->x_token_stride < a->hidden || a->out_token_stride < a->hidden)
        return fail(MR_INVALID_SHAPE, "mla prefill block: x / out token strides %lld / %lld are below hidden %d",
                    (long long)a->x_token_stride, (long long)a->out_token_stride, a->hidden);
    if (a->latent_row_stride < a->kv_rank || (a->qk_rope_dim && a->rope_row_stride < a->qk_rope_dim))
        return fail(MR_INVALID_SHAPE, "mla prefill block: cache row strides %lld / %lld are below %d / %d",
                    (long long)a->latent_row_stride, (long long)a->rope_row_stride, a->kv_rank, a->qk_rope_dim);
    if (!act_dtype_ok(a->norm_w_dtype))
        return fail(MR_INVALID_DTYPE, "mla prefill block: norm weights must be bf16 or f32");
    if (!(a->eps >= 0) || !std::isfinite(a->eps))
        return fail(MR_INVALID_ARGUMENT, "mla prefill block: eps must be finite, >= 0");
    const int dq = a->qk_nope_dim + a->qk_rope_dim;
    const int64_t hv = int64_t(a->heads) * a->v_head_dim;
    const bool gated = a->g_proj.kind != MR_PROJ_NONE;
    struct {
        const mr_projection* w;
        int64_t out, in;
        const char* name;
    } ws[] = {{&a->q_a, a->q_lora_rank, a->hidden, "q_a_proj"},
              {&a->q_b, int64_t(a->heads) * dq, a->q_lora_rank, "q_b_proj"},
              {&a->kv_a, a->kv_rank + a->qk_rope_dim, a->hidden, "kv_a_proj_with_mqa"},
              {&a->kv_b, int64_t(a->heads) * (a->qk_nope_dim + a->v_head_dim), a->kv_rank, "kv_b_proj"},
              {&a->o_proj, a->hidden, hv, "o_proj"},
              {&a->g_proj, hv, a->hidden, "g_proj"}};
    for (auto& e : ws) {
        if (e.w == &a->g_proj && !gated) continue;
        mr_status st = check_projection(e.w, e.name);
        if (st != MR_OK) return st;
        if (proj_out(e.w) != e.out || proj_in(e.w) != e.in)
            return fail(MR_INVALID_SHAPE, "mla prefill block: %s is [%lld, %lld], expected [%lld, %lld]", e.name,
                        (long long)proj_out(e.w), (long long)proj_in(e.w), (long long)e.out, (long long)e.in);
    }
    if (a->kv_b.kind == MR_PROJ_DENSE && a->kv_b.dense.dtype != MR_BF16)
        return fail(MR_INVALID_DTYPE, "mla prefill block: a dense kv_b_proj must be bf16");
    PrefillBlockLayout L;
    prefill_block_layout(a, &L);
    mr_mla_prefill_args p = L.pre_args;
    char* W = (char*)a->workspace;
    p.q = W + L.q;
    p.out = W + L.attn;
    if (a->kv_b.kind == MR_PROJ_AFFINE) p.kv_b = W + L.kv_b;
    if (int64_t(a->position) + a->tokens > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "mla prefill block: position + tokens exceeds int32");
    mr_status st = mrc::check_prefill(&p);
    if (st != MR_OK) return st;
    if (L.total >= WS_LIMIT)
        return fail(MR_INVALID_SHAPE, "mla prefill block: the workspace these widths need overflows");
    if (a->workspace_bytes < L.total)
        return fail(MR_WORKSPACE_TOO_SMALL, "mla prefill block: workspace %zu bytes < %zu", a->workspace_bytes, L.total);
    if (!aligned16(a->workspace))
        return fail(MR_INVALID_ARGUMENT, "mla prefill block: workspace must be 16-byte aligned");
    return MR_OK;
}

}  // namespace

size_t mr_mla_prefill_block_workspace_size(const mr_mla_prefill_block_args* a) {
    if (!a || a->tokens <= 0 || a->hidden <= 0 || a->q_lora_rank <= 0 || a->heads <= 0 || a->qk_nope_dim < 0 ||
        a->qk_rope_dim < 0 || a->v_head_dim <= 0 || a->kv_rank <= 0 || a->position < 0)
        return 0;
    PrefillBlockLayout L;
    prefill_block_layout(a, &L);
    return L.total < WS_LIMIT ? L.total : 0;
}

mr_status mr_mla_prefill_block(const mr_mla_prefill_block_args* a, void* stream) {
    mr_status st = check_prefill_block(a);
    if (st != MR_OK) return st;
    PrefillBlockLayout L;
    prefill_block_layout(a, &L);
    char* W = (char*)a->workspace;
    const int32_t T = a->tokens;
    const int dq = a->qk_nope_dim + a->qk_rope_dim;
    const int64_t hv = int64_t(a->heads) * a->v_head_dim;
    const int kv_w = a->kv_rank + a->qk_rope_dim;
    const mr_dtype nd = a->norm_w_dtype;
    const bool gated = a->g_proj.kind != MR_PROJ_NONE;
    void* q_lora = W + L.q_lora;
    void* q_lora_n = W + L.q_lora_n;
    void* q = W + L.q;
    void* kv = W + L.kv;
    void* gate = W + L.gate;
    void* attn = W + L.attn;

    // the block input, through the input norm when one is given
    const void* h = a->x;
    int64_t h_stride = a->x_token_stride;
    if (a->input_norm_w) {
        if ((st = mr_rmsnorm(a->x, MR_BF16, T, a->hidden, a->x_token_stride, a->input_norm_w, nd, a->eps, W + L.h,
                             MR_BF16, a->hidden, stream)) != MR_OK)
            return st;
        h = W + L.h;
        h_stride = a->hidden;
    }
    // the projections of h over all T tokens (MLA.swift:131,141,207), one
    // stacked launch where they allow it
    {
        const mr_projection* xw[3] = {&a->q_a, &a->kv_a, &a->g_proj};
        void* xy[3] = {q_lora, kv, gate};
        const int64_t ys[3] = {a->q_lora_rank, kv_w, hv};
        if ((st = proj_rows_stacked(h, T, h_stride, xw, xy, ys, gated ? 3 : 2, stream)) != MR_OK) return st;
    }
    // q = q_b(RMSNorm(q_lora)), its rope slice rotated at each token's position
    if ((st = mr_rmsnorm(q_lora, MR_BF16, T, a->q_lora_rank, a->q_lora_rank, a->q_a_norm_w, nd, a->eps, q_lora_n,
                         MR_BF16, a->q_lora_rank, stream)) != MR_OK)
        return st;
    if ((st = proj_rows(q_lora_n, T, a->q_lora_rank, &a->q_b, q, int64_t(a->heads) * dq, stream)) != MR_OK) return st;
    if (a->rope_cos && a->qk_rope_dim &&
        (st = mr_rope_apply(q, MR_BF16, T, a->heads, dq, a->qk_nope_dim, a->qk_rope_dim, a->rope_cos, a->rope_sin,
                            stream)) != MR_OK)
        return st;
    // the T new cache rows: RMSNorm(latent) and the shared key (:142-157)
    const mr::CacheAppendParams app{kv,
                                    0,
                                    kv_w,
                                    a->kv_a_norm_w,
                                    nd == MR_F32,
                                    a->eps,
                                    a->kv_rank,
                                    a->qk_rope_dim,
                                    a->rope_cos,
                                    a->rope_sin,
                                    (uint16_t*)a->cache_latent,
                                    a->latent_row_stride,
                                    (uint16_t*)a->cache_rope,
                                    a->rope_row_stride,
                                    a->position,
                                    T};
    hipError_t e = mr::launch_cache_append(app, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "mla prefill block: cache append launch");
    // causal attention over rows 0 .. position + T - 1 (:159-206)
    mr_mla_prefill_args p = L.pre_args;
    p.q = q;
    p.out = attn;
    if (a->kv_b.kind == MR_PROJ_AFFINE) {
        if ((st = mr_affine_dequantize(&a->kv_b.affine, W + L.kv_b, MR_BF16, stream)) != MR_OK) return st;
        p.kv_b = W + L.kv_b;
    }
    p.workspace = W + L.pre;
    p.workspace_bytes = L.total - L.pre;
    // the output gate (:207-211) rides in the attention's row stores
    if ((st = mrc::mla_prefill_gated(&p, gated ? gate : nullptr, hv, stream)) != MR_OK) return st;
    return proj_rows(attn, T, hv, &a->o_proj, a->out, a->out_token_stride, stream);
}

// ---------------------------------------------------------------- V4 index tables (host)
mr_status mr_attention_indices_window(int32_t window, int32_t seq_len, int32_t start_pos, int32_t* out, int32_t* rows,
                                      int32_t* cols) {
    // DeepSeekV4Attention.swift:170-198
    if (!(window > 0 && seq_len > 0 && start_pos >= 0))
        return fail(MR_INVALID_SHAPE, "window size and sequence length must be positive and start position nonnegative");
    if (!out || !rows || !cols) return fail(MR_INVALID_ARGUMENT, "window indices: NULL output");
    if (start_pos > 0) {
        if (seq_len != 1) return fail(MR_INVALID_SHAPE, "incremental window indexing accepts exactly one token");
        *rows = 1;
        *cols = window;
        int n = 0;
        if (start_pos >= window - 1) {
            const int32_t cursor = start_pos % window;
            for (int32_t k = cursor + 1; k < window; ++k) out[n++] = k;
            for (int32_t k = 0; k <= cursor; ++k) out[n++] = k;
        } else {
            for (int32_t k = 0; k <= start_pos; ++k) out[n++] = k;
            for (int32_t k = 0; k < window - start_pos - 1; ++k) out[n++] = -1;
        }
        return MR_OK;
    }
    const int32_t width = std::min(seq_len, window);
    *rows = seq_len;
    *cols = width;
    for (int32_t pos = 0; pos < seq_len; ++pos) {
        const int32_t first = std::max(0, pos - window + 1);
        for (int32_t c = 0; c < width; ++c) {
            const int32_t cand = first + c;
            out[int64_t(pos) * width + c] = cand <= pos ? cand : -1;
        }
    }
    return MR_OK;
}

mr_status mr_attention_indices_compressed(int32_t ratio, int32_t seq_len, int32_t start_pos, int32_t offset,
                                          int32_t* out, int32_t* rows, int32_t* cols) {
    // DeepSeekV4Attention.swift:200-236
    if (!(ratio > 0 && seq_len > 0 && start_pos >= 0 && offset >= 0))
        return fail(MR_INVALID_SHAPE,
                    "compression ratio and sequence length must be positive; position and offset must be nonnegative");
    if (!out || !rows || !cols) return fail(MR_INVALID_ARGUMENT, "compressed indices: NULL output");
    if (start_pos > 0) {
        if (seq_len != 1) return fail(MR_INVALID_SHAPE, "incremental compressed indexing accepts exactly one token");
        const int64_t count = (int64_t(start_pos) + 1) / ratio;
        *rows = 1;
        *cols = int32_t(count);
        for (int64_t k = 0; k < count; ++k) {
            if (int64_t(offset) + k > INT32_MAX) return fail(MR_INVALID_SHAPE, "cache index overflows Int");
            out[k] = int32_t(offset + k);
        }
        return MR_OK;
    }
    const int32_t width = seq_len / ratio;
    *rows = seq_len;
    *cols = width;
    for (int32_t pos = 0; pos < seq_len; ++pos) {
        const int32_t visible = (pos + 1) / ratio;
        for (int32_t k = 0; k < width; ++k) {
            if (k < visible && int64_t(offset) + k > INT32_MAX) return fail(MR_INVALID_SHAPE, "cache index overflows Int");
            out[int64_t(pos) * width + k] = k < visible ? offset + k : -1;
        }
    }
    return MR_OK;
}

}  // extern "C"
