// C-ABI of the lightning indexer: the scores (DeepSeekV4Attention.swift:
// 530-549) and the top-k selection, with the reference's geometry checks
// (:533-541, :590-612) on the host and the work on the device.
#include <hip/hip_runtime.h>

#include <vector>

#include "../../include/minirun_hip.h"
#include "capi_util.hpp"
#include "mr_kernels.hpp"

namespace {
using mrc::fail;
using mrc::hip_fail;
}  // namespace

extern "C" {

mr_status mr_indexer_scores(const void* queries, mr_dtype q_dtype, int32_t seq, int32_t heads, int32_t dim,
                            int64_t q_seq_stride, int64_t q_head_stride, const void* keys, mr_dtype k_dtype,
                            int32_t n_keys, int32_t key_dim, int64_t k_row_stride, const void* weights,
                            mr_dtype w_dtype, int32_t w_rows, int32_t w_cols, int64_t w_row_stride, float* scores,
                            int64_t out_row_stride, void* stream) {
    // DeepSeekV4Attention.swift:533-541
    if (!(seq > 0 && heads > 0 && dim > 0 && n_keys >= 0 && key_dim == dim && w_rows == seq && w_cols == heads))
        return fail(MR_INVALID_SHAPE, "index queries, keys, and weights have incompatible geometry");
    auto act = [](mr_dtype d) { return d == MR_BF16 || d == MR_F32; };
    if (!act(q_dtype) || !act(k_dtype) || !act(w_dtype))
        return fail(MR_INVALID_DTYPE, "lightning-index scores: queries, keys and weights must be bf16 or f32");
    if (n_keys == 0) return MR_OK;  // :542-544
    if (!queries || !keys || !weights || !scores)
        return fail(MR_INVALID_ARGUMENT, "lightning-index scores: NULL pointer");
    if (q_head_stride < dim || q_seq_stride < int64_t(heads) * q_head_stride || k_row_stride < dim ||
        w_row_stride < heads || out_row_stride < n_keys)
        return fail(MR_INVALID_ARGUMENT, "lightning-index scores: strides are smaller than the rows");
    mr::IndexerParams p{};
    p.q = queries;
    p.q_f32 = q_dtype == MR_F32;
    p.q_ss = q_seq_stride;
    p.q_hs = q_head_stride;
    p.k = keys;
    p.k_f32 = k_dtype == MR_F32;
    p.k_rs = k_row_stride;
    p.w = weights;
    p.w_f32 = w_dtype == MR_F32;
    p.w_ss = w_row_stride;
    p.out = scores;
    p.out_ss = out_row_stride;
    p.S = seq;
    p.H = heads;
    p.D = dim;
    p.T = n_keys;
    const hipError_t e = mr::launch_indexer_scores(p, (hipStream_t)stream);
    return e == hipSuccess ? MR_OK : hip_fail(e, "lightning-index scores launch");
}

mr_status mr_topk_geometry(int32_t rows, int32_t cols, int32_t top_k, int32_t ratio, int32_t start_pos,
                           int32_t offset, int32_t* selected) {
    if (!(rows > 0 && cols >= 0 && top_k > 0 && ratio > 0 && start_pos >= 0 && offset >= 0))
        return fail(MR_INVALID_SHAPE, "invalid lightning-index selection geometry");
    if (start_pos > 0 && rows != 1)
        return fail(MR_INVALID_SHAPE, "incremental lightning indexing accepts exactly one token");
    const int64_t end = int64_t(start_pos) + rows;
    if (end > INT32_MAX) return fail(MR_INVALID_SHAPE, "lightning-index end position overflows Int");
    const int32_t available = int32_t(end / ratio);
    if (available > cols)
        return fail(MR_INVALID_SHAPE, "score matrix has fewer compressed keys than the sequence position requires");
    const int32_t sel = top_k < available ? top_k : available;
    if (available > 0 && int64_t(offset) + available - 1 > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "lightning cache index overflows Int");
    if (selected) *selected = sel;
    return MR_OK;
}

// Score matrices whose workspace could reach 2^56 bytes (every buffer is at
// most 64 bytes per score plus a slice's worth per row) have no size; the
// selection refuses them.
static bool topk_ws_fits(int32_t rows, int32_t cols) {
    return double(rows) * (double(cols) + 8192.0) * 64.0 < double(mrc::WS_LIMIT);
}

size_t mr_topk_workspace_size(int32_t rows, int32_t cols, int32_t top_k) {
    if (rows <= 0 || cols < 0 || top_k <= 0 || !topk_ws_fits(rows, cols)) return 0;
    // a row selects at most min(top_k, cols) keys (cols bounds the keys any
    // start position makes available); the size grows with that count
    return mr::topk_workspace_bytes(rows, cols, top_k < cols ? top_k : cols);
}

mr_status mr_topk_select(const mr_topk_args* a, void* stream) {
    if (!a) return fail(MR_INVALID_ARGUMENT, "mr_topk_select: args is NULL");
    int32_t selected = 0;
    mr_status st = mr_topk_geometry(a->rows, a->cols, a->top_k, a->ratio, a->start_pos, a->offset, &selected);
    if (st != MR_OK) return st;
    if (!topk_ws_fits(a->rows, a->cols))
        return fail(MR_INVALID_SHAPE, "top-k selection: %d rows of %d scores overflow a workspace", a->rows, a->cols);
    if (!a->scores || (selected > 0 && !a->out))
        return fail(MR_INVALID_ARGUMENT, "top-k selection: scores and out must be non-NULL");
    if (a->score_row_stride < a->cols || (selected > 0 && a->out_row_stride < selected))
        return fail(MR_INVALID_ARGUMENT, "top-k selection: row strides are smaller than the rows");
    const size_t need = mr::topk_workspace_bytes(a->rows, a->cols, selected);
    if (!a->workspace || a->workspace_bytes < need)
        return fail(MR_WORKSPACE_TOO_SMALL, "top-k selection: workspace %zu bytes < %zu required", a->workspace_bytes,
                    need);
    if (selected == 0) return MR_OK;  // every row is empty (:613-616)
    hipStream_t s = (hipStream_t)stream;
    mr::TopkParams p{};
    p.scores = a->scores;
    p.row_stride = a->score_row_stride;
    p.rows = a->rows;
    p.cols = a->cols;
    p.available = int32_t((int64_t(a->start_pos) + a->rows) / a->ratio);
    p.selected = selected;
    p.ratio = a->ratio;
    p.start_pos = a->start_pos;
    p.offset = a->offset;
    p.out = a->out;
    p.out_stride = a->out_row_stride;
    p.nan_flags = (int32_t*)a->workspace;
    hipError_t e = mr::launch_topk_select(p, a->workspace, a->status, s);
    if (e != hipSuccess) return hip_fail(e, "top-k selection launch");
    // the reference throws on a NaN score: check on the host unless the
    // caller takes the device status or opts out
    if ((a->flags & MR_TOPK_CHECK) || (!a->status && !(a->flags & MR_TOPK_UNCHECKED))) {
        std::vector<int32_t> flags(size_t(a->rows));
        e = hipMemcpyAsync(flags.data(), p.nan_flags, size_t(a->rows) * 4, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        if (e != hipSuccess) return hip_fail(e, "top-k selection check");
        for (int32_t f : flags)
            if (f) return fail(MR_NONFINITE, "lightning-index score contains NaN");
    }
    return MR_OK;
}

}  // extern "C"
