// C-ABI of the causal MLA prefill: validation, workspace layout, launches.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "../../include/minirun_hip.h"
#include "capi_util.hpp"
#include "mr_kernels.hpp"

namespace {
using mrc::aligned16;
using mrc::align256;
using mrc::fail;
using mrc::hip_fail;

// the widths the MFMA kernels take; others run the any-width kernels
bool prefill_fast_dims(const mr_mla_prefill_args* a) {
    return a->qk_nope_dim == 128 && a->qk_rope_dim == 64 && a->v_head_dim == 128 && a->kv_rank == 512;
}

size_t kv_bytes(const mr_mla_prefill_args* a) {
    if (!prefill_fast_dims(a))  // fp32 keys and values, [heads][n_ctx][nope + v]
        return align256(size_t(a->n_ctx) * size_t(a->heads) *
                        size_t(std::max<int64_t>(int64_t(a->qk_nope_dim) + a->v_head_dim, 0)) * 4);
    return align256(size_t(a->n_ctx) * size_t(a->heads) * 256 * 2);
}

// Other widths: the any-width kernels read elements one by one, so only
// element alignment and strides that cover the rows are required.
mr_status check_prefill_any(const mr_mla_prefill_args* a) {
    if (a->kv_rank <= 0 || a->kv_rank > mr::ANY_MAX_RANK || a->qk_nope_dim < 0 || a->qk_nope_dim > mr::ANY_MAX_NOPE ||
        a->qk_rope_dim < 0 || a->qk_rope_dim > mr::ANY_MAX_ROPE || a->v_head_dim <= 0 || a->v_head_dim > mr::ANY_MAX_RANK)
        return fail(MR_INVALID_SHAPE,
                    "mla prefill: widths kv_rank %d (1..%d), qk_nope %d (0..%d), qk_rope %d (0..%d), v_head %d (1..%d)",
                    a->kv_rank, mr::ANY_MAX_RANK, a->qk_nope_dim, mr::ANY_MAX_NOPE, a->qk_rope_dim, mr::ANY_MAX_ROPE,
                    a->v_head_dim, mr::ANY_MAX_RANK);
    if (a->tokens <= 0 || a->heads <= 0)
        return fail(MR_INVALID_SHAPE, "mla prefill: tokens %d and heads %d must be positive", a->tokens, a->heads);
    if (a->n_ctx < a->tokens)
        return fail(MR_INVALID_SHAPE, "mla prefill: n_ctx %d must cover the %d query tokens", a->n_ctx, a->tokens);
    if (int64_t(a->n_ctx) * a->heads > INT32_MAX || int64_t(a->tokens) * a->heads > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "mla prefill: n_ctx * heads and tokens * heads must fit in int32");
    if (!(std::isfinite(a->scale) && a->scale > 0))
        return fail(MR_INVALID_SHAPE, "mla prefill: scale %g must be finite and positive", double(a->scale));
    if (!a->q || !a->latent || (a->qk_rope_dim && !a->rope_keys) || !a->kv_b || !a->out)
        return fail(MR_INVALID_ARGUMENT, "mla prefill: q, latent, rope_keys, kv_b and out must be non-NULL");
    auto al2 = [](const void* q) { return ((uintptr_t)q & 1) == 0; };
    if (!al2(a->q) || !al2(a->latent) || !al2(a->rope_keys) || !al2(a->kv_b) || !al2(a->out))
        return fail(MR_INVALID_ARGUMENT, "mla prefill: q, latent, rope_keys, kv_b and out must be element-aligned");
    const int64_t qw = a->qk_nope_dim + a->qk_rope_dim;
    if (a->q_head_stride < qw || a->q_token_stride < qw || a->latent_row_stride < a->kv_rank ||
        a->rope_row_stride < a->qk_rope_dim || a->kv_b_row_stride < a->kv_rank || a->out_head_stride < a->v_head_dim ||
        a->out_token_stride < a->v_head_dim)
        return fail(MR_INVALID_ARGUMENT, "mla prefill: strides are smaller than the rows they step over");
    if (a->out_dtype != MR_BF16 && a->out_dtype != MR_F32)
        return fail(MR_INVALID_DTYPE, "mla prefill: out_dtype must be MR_BF16 or MR_F32");
    return MR_OK;
}

}  // namespace

mr_status mrc::check_prefill(const mr_mla_prefill_args* a) {
    if (!a) return fail(MR_INVALID_ARGUMENT, "mr_mla_prefill: args is NULL");
    if (!prefill_fast_dims(a)) return check_prefill_any(a);
    if (a->tokens <= 0 || a->heads <= 0)
        return fail(MR_INVALID_SHAPE, "mla prefill: tokens %d and heads %d must be positive", a->tokens, a->heads);
    if (a->n_ctx < a->tokens)
        return fail(MR_INVALID_SHAPE, "mla prefill: n_ctx %d must cover the %d query tokens", a->n_ctx, a->tokens);
    if (double(a->heads) * 256.0 * double(a->n_ctx) >= 2147483648.0 || a->heads > 65536)
        return fail(MR_INVALID_SHAPE, "mla prefill: n_ctx * heads * 256 must stay below 2^31");
    if (!(std::isfinite(a->scale) && a->scale > 0))
        return fail(MR_INVALID_SHAPE, "mla prefill: scale %g must be finite and positive", double(a->scale));
    if (!a->q || !a->latent || !a->rope_keys || !a->kv_b || !a->out)
        return fail(MR_INVALID_ARGUMENT, "mla prefill: q, latent, rope_keys, kv_b and out must be non-NULL");
    if (!aligned16(a->q) || !aligned16(a->latent) || !aligned16(a->rope_keys) || !aligned16(a->kv_b) ||
        !aligned16(a->out))
        return fail(MR_INVALID_ARGUMENT, "mla prefill: q, latent, rope_keys, kv_b and out must be 16-byte aligned");
    const int64_t st[] = {a->q_token_stride, a->q_head_stride, a->latent_row_stride, a->rope_row_stride,
                          a->kv_b_row_stride};
    for (int64_t s : st)
        if (s < 0 || s % 8)
            return fail(MR_INVALID_ARGUMENT, "mla prefill: input strides must be non-negative multiples of 8 elements");
    if (a->q_head_stride < 192 || a->q_token_stride < 192 || a->latent_row_stride < 512 || a->rope_row_stride < 64 ||
        a->kv_b_row_stride < 512)
        return fail(MR_INVALID_ARGUMENT, "mla prefill: strides are smaller than the rows they step over");
    if (a->rope_row_stride > (int64_t)(INT32_MAX / 64))  // a 64-key tile's offsets stay 32-bit
        return fail(MR_INVALID_ARGUMENT, "mla prefill: rope_row_stride %lld too large", (long long)a->rope_row_stride);
    if (a->out_dtype != MR_BF16 && a->out_dtype != MR_F32)
        return fail(MR_INVALID_DTYPE, "mla prefill: out_dtype must be MR_BF16 or MR_F32");
    const int64_t vec = a->out_dtype == MR_F32 ? 4 : 8;  // 16-byte output pieces
    if (a->out_head_stride < 128 || a->out_token_stride < 128 || a->out_head_stride % vec || a->out_token_stride % vec)
        return fail(MR_INVALID_ARGUMENT, "mla prefill: out strides must be >= 128 and multiples of %lld elements",
                    (long long)vec);
    return MR_OK;
}

extern "C" {

size_t mr_mla_prefill_workspace_size(const mr_mla_prefill_args* a) {
    // 0 for the widths and counts the call refuses (check_prefill_any's
    // limits; the fixed widths are inside them)
    if (!a || a->n_ctx <= 0 || a->heads <= 0 || a->kv_rank <= 0 || a->kv_rank > mr::ANY_MAX_RANK ||
        a->qk_nope_dim < 0 || a->qk_nope_dim > mr::ANY_MAX_NOPE || a->qk_rope_dim < 0 ||
        a->qk_rope_dim > mr::ANY_MAX_ROPE || a->v_head_dim <= 0 || a->v_head_dim > mr::ANY_MAX_RANK ||
        int64_t(a->n_ctx) * a->heads > INT32_MAX)
        return 0;
    return kv_bytes(a);
}

mr_status mr_mla_prefill(const mr_mla_prefill_args* a, void* stream) { return mrc::mla_prefill_gated(a, nullptr, 0, stream); }

}  // extern "C"

mr_status mrc::mla_prefill_gated(const mr_mla_prefill_args* a, const void* gate, int64_t gate_ts, void* stream) {
    mr_status st = mrc::check_prefill(a);
    if (st != MR_OK) return st;
    if (gate && (a->out_dtype != MR_BF16 || a->out_head_stride != a->v_head_dim ||
                 a->out_token_stride != int64_t(a->heads) * a->v_head_dim || gate_ts != a->out_token_stride ||
                 !aligned16(gate)))
        return fail(MR_INVALID_ARGUMENT, "mla prefill: a gated prefill writes contiguous bf16 rows");
    const size_t need = kv_bytes(a);
    if (!a->workspace || a->workspace_bytes < need)
        return fail(MR_WORKSPACE_TOO_SMALL, "mla prefill: workspace %zu bytes < %zu required", a->workspace_bytes, need);
    if (!aligned16(a->workspace)) return fail(MR_INVALID_ARGUMENT, "mla prefill: workspace must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    hipEvent_t const* ev = (hipEvent_t const*)a->phase_events;
    if (!prefill_fast_dims(a)) {
        mr::AnyPrefillParams q{};
        q.q = (const uint16_t*)a->q;
        q.q_ts = a->q_token_stride;
        q.q_hs = a->q_head_stride;
        q.latent = (const uint16_t*)a->latent;
        q.lat_rs = a->latent_row_stride;
        q.rope = (const uint16_t*)a->rope_keys;
        q.rope_rs = a->rope_row_stride;
        q.kv_b = (const uint16_t*)a->kv_b;
        q.kvb_rs = a->kv_b_row_stride;
        q.kv = (float*)a->workspace;
        q.out = a->out;
        q.out_ts = a->out_token_stride;
        q.out_hs = a->out_head_stride;
        q.out_f32 = a->out_dtype == MR_F32;
        q.T = a->tokens;
        q.P = a->n_ctx;
        q.H = a->heads;
        q.R = a->kv_rank;
        q.DR = a->qk_rope_dim;
        q.NOPE = a->qk_nope_dim;
        q.V = a->v_head_dim;
        q.scale_log2 = float(double(a->scale) * 1.4426950408889634);
        hipError_t e = mr::launch_mla_prefill_any(q, ev, s);
        if (e == hipSuccess && gate)
            e = mr::launch_gate_mul((const uint16_t*)a->out, (const uint16_t*)gate, int64_t(a->tokens) * gate_ts,
                                    (uint16_t*)a->out, s);
        return e == hipSuccess ? MR_OK : hip_fail(e, "mla prefill (any width) launch");
    }
    uint16_t* kv = (uint16_t*)a->workspace;
    // keys/values head-major: head h's [n_ctx][256] block is contiguous
    const int64_t kv_hs = int64_t(a->n_ctx) * 256;

    mr::UpProjParams u{};
    u.a = (const uint16_t*)a->latent;
    u.lda = a->latent_row_stride;
    u.b = (const uint16_t*)a->kv_b;
    u.ldb = a->kv_b_row_stride;
    u.c = kv;
    u.ldc = 256;
    u.c_hs = kv_hs;
    u.M = a->n_ctx;
    u.N = a->heads * 256;
    u.K = 512;

    mr::PrefillAttnParams p{};
    p.q = (const uint16_t*)a->q;
    p.q_ts = a->q_token_stride;
    p.q_hs = a->q_head_stride;
    p.kv = kv;
    p.kv_rs = 256;
    p.kv_hs = kv_hs;
    p.rope = (const uint16_t*)a->rope_keys;
    p.rope_rs = a->rope_row_stride;
    p.out = a->out;
    p.out_ts = a->out_token_stride;
    p.out_hs = a->out_head_stride;
    p.out_f32 = a->out_dtype == MR_F32;
    p.T = a->tokens;
    p.P = a->n_ctx;
    p.H = a->heads;
    p.scale_log2 = float(double(a->scale) * 1.4426950408889634);
    p.gate = (const uint16_t*)gate;
    p.gate_ts = gate_ts;

    hipError_t e = hipSuccess;
    if (ev) e = hipEventRecord(ev[0], s);
    if (e == hipSuccess) e = mr::launch_upproj(u, s);
    if (e == hipSuccess && ev) e = hipEventRecord(ev[1], s);
    if (e == hipSuccess) e = mr::launch_prefill_attn(p, s);
    if (e == hipSuccess && ev) e = hipEventRecord(ev[2], s);
    return e == hipSuccess ? MR_OK : hip_fail(e, "mla prefill launch");
}
