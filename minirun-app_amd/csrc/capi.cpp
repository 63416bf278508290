// C-ABI layer: argument validation with named errors, workspace layout,
// launch-shape choice.  No device memory is allocated here.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/minirun_hip.h"
#include "capi_util.hpp"
#include "mr_kernels.hpp"

namespace {
thread_local std::string g_last_error;
}  // namespace

namespace mrc {

mr_status fail(mr_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

mr_status hip_fail(hipError_t e, const char* what) {
    return fail(MR_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
}

const char* dtype_name(mr_dtype d) {
    switch (d) {
        case MR_BF16: return "bfloat16";
        case MR_F16: return "float16";
        case MR_F32: return "float32";
        case MR_U32: return "uint32";
        case MR_I32: return "int32";
    }
    return "unknown";
}

}  // namespace mrc

namespace {
using mrc::aligned16;
using mrc::aligned4;
using mrc::align256;
using mrc::fail;
using mrc::hip_fail;

constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];

}  // namespace

namespace mrc {
int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int v = g_cu_count[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_cu_count[dev].store(n, std::memory_order_relaxed);
    return n;
}
}  // namespace mrc

namespace {
using mrc::cu_count;

struct DecodePlan {
    int n_rows, hg_size, head_groups, h_pad, splits, rows_per_split;
    bool ws_f32;
    bool checked, sync_check;  // index checks, and whether they run before the launch
    size_t o_bytes, ml_bytes, table_bytes, total;
};

// 0 for counts the checks refuse, and for tables of WS_LIMIT bytes or more
size_t validate_ws_bytes(int32_t batch, int32_t n_idx) {
    if (batch <= 0 || n_idx < 0 || n_idx > mr::validate_max_indices()) return 0;
    const size_t total = align256(size_t(batch) * 3 * sizeof(int32_t)) + align256(mr::validate_table_bytes(batch, n_idx));
    return total < mrc::WS_LIMIT ? total : 0;
}

// the widths the split kernel takes; others run the any-width kernel
bool decode_fast_dims(const mr_mla_decode_args* a) { return a->kv_rank == 512 && (a->rope_dim == 64 || a->rope_dim == 0); }

// the counts and widths both kernels accept (the checks below refuse the
// rest): the workspace sizes are reported for these only, and stay far
// below 2^56 for them
bool decode_counts_ok(const mr_mla_decode_args* a) {
    if (a->batch <= 0 || a->heads <= 0 || int64_t(a->batch) * (int64_t(a->heads) + 63) > INT32_MAX) return false;
    if (a->kv_rank <= 0 || a->kv_rank > mr::ANY_MAX_RANK || a->rope_dim < 0 || a->rope_dim > mr::ANY_MAX_ROPE)
        return false;
    if (a->n_ctx <= 0) return false;
    if (!a->indices) return true;
    if (a->n_idx < 0) return false;
    if (!(a->flags & MR_DECODE_UNCHECKED) &&
        (a->n_idx > mr::validate_max_indices() || validate_ws_bytes(a->batch, a->n_idx) == 0))
        return false;
    return !decode_fast_dims(a) || int64_t(a->n_idx) <= int64_t(mr::MAX_GATHER_ROWS) * mr::MAX_COMBINE_SPLITS;
}

DecodePlan plan_decode(const mr_mla_decode_args* a) {
    DecodePlan pl{};
    pl.n_rows = a->indices ? a->n_idx : a->n_ctx;
    pl.checked = a->indices && !(a->flags & MR_DECODE_UNCHECKED);
    pl.sync_check = pl.checked && (!a->index_status || (a->flags & MR_DECODE_VALIDATE_INDICES));
    if (!decode_fast_dims(a)) {
        // any-width kernel: no partials; the index checks' result words and
        // long lists' tables (laid out as mr_validate_indices lays them out)
        pl.total = pl.checked ? validate_ws_bytes(a->batch, a->n_idx) : 0;
        return pl;
    }
    pl.hg_size = mr::decode_head_group_size(a->heads);
    pl.head_groups = (a->heads + pl.hg_size - 1) / pl.hg_size;
    pl.h_pad = pl.head_groups * pl.hg_size;
    const int rows = std::max(pl.n_rows, 0);
    int splits;
    if (a->num_splits > 0) {
        splits = a->num_splits;
    } else {
        const double per = double(cu_count()) / double(std::max(1, a->batch * pl.head_groups));
        splits = std::max(1, int(std::lround(per)));
    }
    const int max_splits = std::max(1, (rows + 63) / 64);
    splits = std::min(splits, max_splits);
    int rps = (rows + splits - 1) / splits;
    rps = std::max(64, (rps + 63) / 64 * 64);
    // gathered rows: a split of 64 rows writes as many partial bytes as it
    // reads rows, so take at least 128 while the grid keeps half the CUs busy
    // (measured at B=4, H=128, K=2048: 22.1 us per layer against 23.7 at 64)
    if (a->indices && a->num_splits <= 0 && rps < 128 &&
        int64_t(a->batch) * pl.head_groups * ((rows + 127) / 128) >= cu_count() / 2)
        rps = 128;
    if (a->indices && rps > mr::MAX_GATHER_ROWS) rps = mr::MAX_GATHER_ROWS;
    splits = std::max(1, (rows + rps - 1) / rps);
    if (splits > mr::MAX_COMBINE_SPLITS) {  // very long contexts: fewer, longer splits
        rps = ((rows + mr::MAX_COMBINE_SPLITS - 1) / mr::MAX_COMBINE_SPLITS + 63) / 64 * 64;
        splits = std::max(1, (rows + rps - 1) / rps);
    }
    pl.splits = splits;
    pl.rows_per_split = rps;
    const size_t recs = size_t(std::max(a->batch, 0)) * size_t(splits) * size_t(pl.h_pad);
    // split partials in fp32 for f32 output and for small grids (up to 4096
    // records, 8 MB: short contexts, where each partial carries a large share
    // of the output), else bf16 (half the bytes the combine reads back)
    pl.ws_f32 = a->out_dtype == MR_F32 || recs <= 4096;
    pl.o_bytes = align256(recs * 512 * (pl.ws_f32 ? sizeof(float) : sizeof(uint16_t)));
    pl.ml_bytes = align256(recs * 2 * sizeof(float));
    // index checks in the split launch keep long lists' tables after the
    // partials; a check before the launch uses the workspace first
    pl.table_bytes = (pl.checked && !pl.sync_check) ? align256(mr::validate_table_bytes(a->batch, a->n_idx)) : 0;
    pl.total = pl.o_bytes + pl.ml_bytes + pl.table_bytes;
    if (pl.sync_check) pl.total = std::max(pl.total, validate_ws_bytes(a->batch, a->n_idx));
    return pl;
}

}  // namespace

mrc::DecodePartials mrc::decode_partials(const mr_mla_decode_args* a) {
    const DecodePlan pl = plan_decode(a);
    return DecodePartials{pl.splits, pl.h_pad, pl.ws_f32, pl.o_bytes};
}

namespace {

// Widths the split kernel does not take (kv_rank other than 512, rope_dim
// other than 64 or 0): the any-width kernel reads elements one by one, so
// only element alignment and strides that cover the rows are required.
mr_status check_decode_any(const mr_mla_decode_args* a) {
    if (!(std::isfinite(a->scale) && a->scale > 0))
        return fail(MR_INVALID_SHAPE, "sparse attention queries, shared KV, sinks, indices, or scale are invalid: "
                                      "scale %g must be finite and positive", double(a->scale));
    if (a->indices) {
        if (a->n_idx < 0) return fail(MR_INVALID_SHAPE, "mla decode: n_idx %d is negative", a->n_idx);
        if (a->n_ctx <= 0) return fail(MR_INVALID_SHAPE, "mla decode: the cache has no rows (n_ctx %d)", a->n_ctx);
        if (!(a->flags & MR_DECODE_UNCHECKED) && a->n_idx > mr::validate_max_indices())
            return fail(MR_INVALID_SHAPE, "mla decode: index checks take at most %d entries per token, got %d "
                        "(MR_DECODE_UNCHECKED skips them)", mr::validate_max_indices(), a->n_idx);
    } else if (a->n_ctx <= 0) {
        return fail(MR_INVALID_SHAPE, "mla decode: n_ctx %d must be positive", a->n_ctx);
    }
    if (!a->q_lat || !a->latent || !a->out)
        return fail(MR_INVALID_ARGUMENT, "mla decode: q_lat, latent and out must be non-NULL");
    if (a->rope_dim && (!a->q_rope || !a->rope_keys))
        return fail(MR_INVALID_ARGUMENT, "mla decode: rope_dim %d needs q_rope and rope_keys", a->rope_dim);
    auto al2 = [](const void* q) { return ((uintptr_t)q & 1) == 0; };
    if (!al2(a->q_lat) || !al2(a->latent) || !al2(a->out) || (a->rope_dim && (!al2(a->q_rope) || !al2(a->rope_keys))))
        return fail(MR_INVALID_ARGUMENT, "mla decode: q, cache and out pointers must be element-aligned");
    if (a->q_lat_batch_stride < 0 || a->latent_batch_stride < 0 || a->out_batch_stride < 0 ||
        a->q_lat_head_stride < a->kv_rank || a->latent_row_stride < a->kv_rank || a->out_head_stride < a->kv_rank)
        return fail(MR_INVALID_ARGUMENT, "mla decode: strides must be non-negative and cover kv_rank %d", a->kv_rank);
    if (a->rope_dim && (a->q_rope_batch_stride < 0 || a->rope_batch_stride < 0 || a->q_rope_head_stride < a->rope_dim ||
                        a->rope_row_stride < a->rope_dim))
        return fail(MR_INVALID_ARGUMENT, "mla decode: rope strides must be non-negative and cover rope_dim %d",
                    a->rope_dim);
    if (a->out_dtype != MR_BF16 && a->out_dtype != MR_F32)
        return fail(MR_INVALID_DTYPE, "mla decode: out_dtype must be MR_BF16 or MR_F32");
    if (a->num_splits < 0) return fail(MR_INVALID_ARGUMENT, "mla decode: num_splits must be >= 0");
    if (int64_t(a->batch) * a->heads > INT32_MAX) return fail(MR_INVALID_SHAPE, "mla decode: batch * heads too large");
    return MR_OK;
}

mr_status check_decode(const mr_mla_decode_args* a) {
    if (!a) return fail(MR_INVALID_ARGUMENT, "mr_mla_decode: args is NULL");
    if (a->batch <= 0 || a->heads <= 0)
        return fail(MR_INVALID_SHAPE, "mla decode: batch %d and heads %d must be positive", a->batch, a->heads);
    if (a->kv_rank <= 0 || a->kv_rank > mr::ANY_MAX_RANK || a->rope_dim < 0 || a->rope_dim > mr::ANY_MAX_ROPE)
        return fail(MR_INVALID_SHAPE, "mla decode: kv_rank %d must be in [1, %d] and rope_dim %d in [0, %d]", a->kv_rank,
                    mr::ANY_MAX_RANK, a->rope_dim, mr::ANY_MAX_ROPE);
    // head counts padded to whole head groups (64) stay in 32 bits
    if (int64_t(a->batch) * (int64_t(a->heads) + 63) > INT32_MAX)
        return fail(MR_INVALID_SHAPE, "mla decode: batch %d * heads %d too large", a->batch, a->heads);
    if (a->indices && !(a->flags & MR_DECODE_UNCHECKED) && a->n_idx >= 0 && a->n_idx <= mr::validate_max_indices() &&
        validate_ws_bytes(a->batch, a->n_idx) == 0)
        return fail(MR_INVALID_SHAPE, "mla decode: index check tables for batch %d x %d entries overflow a workspace",
                    a->batch, a->n_idx);
    if (!decode_fast_dims(a)) return check_decode_any(a);
    if (!(std::isfinite(a->scale) && a->scale > 0))
        return fail(MR_INVALID_SHAPE, "sparse attention queries, shared KV, sinks, indices, or scale are invalid: "
                                      "scale %g must be finite and positive", double(a->scale));
    if (a->indices) {
        if (a->n_idx < 0) return fail(MR_INVALID_SHAPE, "mla decode: n_idx %d is negative", a->n_idx);
        if (a->n_ctx <= 0) return fail(MR_INVALID_SHAPE, "mla decode: the cache has no rows (n_ctx %d)", a->n_ctx);
        // a gathered split stages at most MAX_GATHER_ROWS indices in LDS and
        // the combine merges at most MAX_COMBINE_SPLITS splits
        if (int64_t(a->n_idx) > int64_t(mr::MAX_GATHER_ROWS) * mr::MAX_COMBINE_SPLITS)
            return fail(MR_INVALID_SHAPE, "mla decode: n_idx %d exceeds %d", a->n_idx,
                        mr::MAX_GATHER_ROWS * mr::MAX_COMBINE_SPLITS);
        if (!(a->flags & MR_DECODE_UNCHECKED) && a->n_idx > mr::validate_max_indices())
            return fail(MR_INVALID_SHAPE, "mla decode: index checks take at most %d entries per token, got %d "
                        "(MR_DECODE_UNCHECKED skips them)", mr::validate_max_indices(), a->n_idx);
    } else if (a->n_ctx <= 0) {
        return fail(MR_INVALID_SHAPE, "mla decode: n_ctx %d must be positive", a->n_ctx);
    }
    if (!a->q_lat || !a->latent || !a->out)
        return fail(MR_INVALID_ARGUMENT, "mla decode: q_lat, latent and out must be non-NULL");
    if (a->rope_dim && (!a->q_rope || !a->rope_keys))
        return fail(MR_INVALID_ARGUMENT, "mla decode: rope_dim %d needs q_rope and rope_keys", a->rope_dim);
    if (!aligned16(a->q_lat) || !aligned16(a->latent) || (a->rope_dim && (!aligned16(a->q_rope) || !aligned16(a->rope_keys))))
        return fail(MR_INVALID_ARGUMENT, "mla decode: q and cache base pointers must be 16-byte aligned");
    const int64_t strides[] = {a->q_lat_head_stride, a->q_lat_batch_stride, a->latent_row_stride, a->latent_batch_stride};
    for (int64_t s : strides)
        if (s < 0 || s % 8) return fail(MR_INVALID_ARGUMENT, "mla decode: q/latent strides must be non-negative multiples of 8 elements");
    if (a->latent_row_stride < 512 || a->q_lat_head_stride < 512)
        return fail(MR_INVALID_ARGUMENT, "mla decode: latent_row_stride and q_lat_head_stride must be >= 512");
    if (a->rope_dim) {
        const int64_t rs[] = {a->q_rope_head_stride, a->q_rope_batch_stride, a->rope_row_stride, a->rope_batch_stride};
        for (int64_t s : rs)
            if (s < 0 || s % 8) return fail(MR_INVALID_ARGUMENT, "mla decode: rope strides must be non-negative multiples of 8 elements");
        if (a->rope_row_stride < 64 || a->q_rope_head_stride < 64)
            return fail(MR_INVALID_ARGUMENT, "mla decode: rope strides must be >= 64");
    }
    if (a->out_dtype != MR_BF16 && a->out_dtype != MR_F32)
        return fail(MR_INVALID_DTYPE, "mla decode: out_dtype must be MR_BF16 or MR_F32");
    // the combine stores 16 bytes per lane: 8 bf16 or 4 f32 elements
    const int64_t ovec = a->out_dtype == MR_F32 ? 4 : 8;
    if (a->out_head_stride < 512 || a->out_batch_stride < 0 || a->out_head_stride % ovec || a->out_batch_stride % ovec)
        return fail(MR_INVALID_ARGUMENT, "mla decode: out strides must be multiples of %lld elements, head stride >= 512",
                    (long long)ovec);
    if (!aligned16(a->out)) return fail(MR_INVALID_ARGUMENT, "mla decode: out must be 16-byte aligned");
    if (a->num_splits < 0) return fail(MR_INVALID_ARGUMENT, "mla decode: num_splits must be >= 0");
    // row offsets inside one batch element's cache are formed in 32 bits
    if (double(a->n_ctx) * double(a->latent_row_stride) * 2.0 >= 4294967296.0)
        return fail(MR_INVALID_SHAPE, "mla decode: n_ctx * latent_row_stride * 2 bytes must be < 4 GiB per batch element");
    return MR_OK;
}

}  // namespace

// The any-width decode: the device-status index check as a launch of its
// own (long lists' tables where mr_validate_indices keeps them), then one
// workgroup per (batch, head).
static mr_status decode_any(const mr_mla_decode_args* a, bool device_check, void* stream) {
    hipStream_t s = (hipStream_t)stream;
    hipEvent_t const* ev = (hipEvent_t const*)a->phase_events;
    hipError_t e = hipSuccess;
    if (ev) e = hipEventRecord(ev[0], s);
    if (e == hipSuccess && device_check && a->n_idx > 0) {
        int32_t* tables = (int32_t*)((char*)a->workspace + align256(size_t(a->batch) * 3 * sizeof(int32_t)));
        e = mr::launch_validate_indices(a->indices, a->batch, a->n_idx, a->n_ctx, tables, a->index_status, s);
    }
    mr::AnyDecodeParams q{};
    q.q_lat = (const uint16_t*)a->q_lat;
    q.q_lat_bs = a->q_lat_batch_stride;
    q.q_lat_hs = a->q_lat_head_stride;
    q.q_rope = (const uint16_t*)a->q_rope;
    q.q_rope_bs = a->q_rope_batch_stride;
    q.q_rope_hs = a->q_rope_head_stride;
    q.latent = (const uint16_t*)a->latent;
    q.lat_rs = a->latent_row_stride;
    q.lat_bs = a->latent_batch_stride;
    q.rope = (const uint16_t*)a->rope_keys;
    q.rope_rs = a->rope_row_stride;
    q.rope_bs = a->rope_batch_stride;
    q.indices = a->indices;
    q.n_idx = a->n_idx;
    q.sinks = a->sinks;
    q.out = a->out;
    q.out_bs = a->out_batch_stride;
    q.out_hs = a->out_head_stride;
    q.out_f32 = a->out_dtype == MR_F32;
    q.batch = a->batch;
    q.heads = a->heads;
    q.n_ctx = a->n_ctx;
    q.R = a->kv_rank;
    q.DR = a->rope_dim;
    q.scale_log2 = float(double(a->scale) * 1.4426950408889634);
    if (e == hipSuccess) e = mr::launch_mla_decode_any(q, s);
    if (e == hipSuccess && ev) e = hipEventRecord(ev[1], s);
    if (e == hipSuccess && ev) e = hipEventRecord(ev[2], s);
    return e == hipSuccess ? MR_OK : hip_fail(e, "mla decode (any width) launch");
}

extern "C" {

const char* mr_version(void) { return "minirun-hip 0.1.0 gfx950"; }

const char* mr_get_last_error(void) { return g_last_error.c_str(); }

size_t mr_mla_decode_workspace_size(const mr_mla_decode_args* args) {
    if (!args || !decode_counts_ok(args)) return 0;
    return plan_decode(args).total;
}

size_t mr_validate_indices_workspace_size(int32_t batch, int32_t n_idx) { return validate_ws_bytes(batch, n_idx); }

mr_status mr_validate_indices(const int32_t* indices, int32_t batch, int32_t n_idx, int32_t n_rows,
                              void* workspace, size_t workspace_bytes, int32_t* bad_token,
                              int32_t* bad_position, void* stream) {
    if (bad_token) *bad_token = -1;
    if (bad_position) *bad_position = -1;
    if (batch <= 0 || n_idx < 0 || n_rows < 0)
        return fail(MR_INVALID_SHAPE, "index validation: batch %d, n_idx %d, n_rows %d", batch, n_idx, n_rows);
    if (n_idx == 0) return MR_OK;
    if (n_idx > mr::validate_max_indices())
        return fail(MR_INVALID_SHAPE, "index validation: n_idx %d exceeds %d", n_idx, mr::validate_max_indices());
    if (mr_validate_indices_workspace_size(batch, n_idx) == 0)
        return fail(MR_INVALID_SHAPE, "index validation: the tables of %d x %d entries overflow a workspace", batch, n_idx);
    if (!indices || !workspace) return fail(MR_INVALID_ARGUMENT, "index validation: NULL indices or workspace");
    if (workspace_bytes < mr_validate_indices_workspace_size(batch, n_idx))
        return fail(MR_WORKSPACE_TOO_SMALL, "index validation: workspace %zu bytes < %zu", workspace_bytes,
                    mr_validate_indices_workspace_size(batch, n_idx));
    hipStream_t st = (hipStream_t)stream;
    int32_t* res = (int32_t*)workspace;
    int32_t* tables = (int32_t*)((char*)workspace + align256(size_t(batch) * 3 * sizeof(int32_t)));
    hipError_t e = mr::launch_validate_indices(indices, batch, n_idx, n_rows, tables, res, st);
    if (e != hipSuccess) return hip_fail(e, "index validation launch");
    std::vector<int32_t> host(size_t(batch) * 3);
    e = hipMemcpyAsync(host.data(), res, host.size() * sizeof(int32_t), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "index validation readback");
    for (int32_t b = 0; b < batch; ++b) {
        const int32_t code = host[3 * b], pos = host[3 * b + 1], v = host[3 * b + 2];
        if (code == MR_OK) continue;
        if (bad_token) *bad_token = b;
        if (bad_position) *bad_position = pos;
        // DeepSeekV4Attention.swift:888-893
        if (code == MR_INDEX_OUT_OF_RANGE)
            return fail(MR_INDEX_OUT_OF_RANGE, "token %d names KV row %d, outside the cache", b, v);
        return fail(MR_DUPLICATE_INDEX, "token %d names KV row %d more than once", b, v);
    }
    return MR_OK;
}

mr_status mr_mla_decode(const mr_mla_decode_args* a, void* stream) {
    mr_status st = check_decode(a);
    if (st != MR_OK) return st;
    const DecodePlan pl = plan_decode(a);
    if (pl.total && (!a->workspace || a->workspace_bytes < pl.total))
        return fail(MR_WORKSPACE_TOO_SMALL, "mla decode: workspace %zu bytes < %zu required", a->workspace_bytes, pl.total);
    if (!aligned16(a->workspace)) return fail(MR_INVALID_ARGUMENT, "mla decode: workspace must be 16-byte aligned");
    // index checks: on the device in the split launch when the caller gives
    // a status buffer, else synchronously before it (the reference throws)
    const bool checked = pl.checked;
    const bool sync_check = pl.sync_check;
    if (sync_check && a->n_idx > 0) {
        st = mr_validate_indices(a->indices, a->batch, a->n_idx, a->n_ctx, a->workspace, a->workspace_bytes, nullptr,
                                 nullptr, stream);
        if (st != MR_OK) return st;
    }
    if (checked && !sync_check && !aligned4(a->index_status))
        return fail(MR_INVALID_ARGUMENT, "mla decode: index_status must be 4-byte aligned");
    if (!decode_fast_dims(a)) return decode_any(a, checked && !sync_check, stream);
    mr::DecodeParams p{};
    p.q_lat = (const uint16_t*)a->q_lat;
    p.q_lat_bs = a->q_lat_batch_stride;
    p.q_lat_hs = a->q_lat_head_stride;
    p.q_rope = (const uint16_t*)a->q_rope;
    p.q_rope_bs = a->q_rope_batch_stride;
    p.q_rope_hs = a->q_rope_head_stride;
    p.latent = (const uint16_t*)a->latent;
    p.lat_rs = a->latent_row_stride;
    p.lat_bs = a->latent_batch_stride;
    p.rope = (const uint16_t*)a->rope_keys;
    p.rope_rs = a->rope_row_stride;
    p.rope_bs = a->rope_batch_stride;
    p.indices = a->indices;
    p.n_idx = a->n_idx;
    p.batch = a->batch;
    p.heads = a->heads;
    p.n_ctx = a->n_ctx;
    p.rope_dim = a->rope_dim;
    p.n_rows = pl.n_rows;
    p.splits = pl.splits;
    p.rows_per_split = pl.rows_per_split;
    p.head_groups = pl.head_groups;
    p.h_pad = pl.h_pad;
    p.hg_size = pl.hg_size;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    p.ws_o = a->workspace;
    p.ws_f32 = pl.ws_f32;
    p.ws_ml = (float*)((char*)a->workspace + pl.o_bytes);
    // one check workgroup per token, in front of a multiple of 8 so the
    // attention workgroups keep their XCD placement (blockIdx % 8)
    p.check_blocks = (checked && !sync_check) ? (a->batch + 7) / 8 * 8 : 0;
    p.index_status = p.check_blocks ? a->index_status : nullptr;
    p.check_table = (p.check_blocks && pl.table_bytes) ? (int32_t*)((char*)a->workspace + pl.o_bytes + pl.ml_bytes)
                                                       : nullptr;

    mr::CombineParams cp{};
    cp.ws_o = p.ws_o;
    cp.ws_f32 = p.ws_f32;
    cp.ws_ml = p.ws_ml;
    cp.sinks = a->sinks;
    cp.out = a->out;
    cp.out_bs = a->out_batch_stride;
    cp.out_hs = a->out_head_stride;
    cp.batch = a->batch;
    cp.heads = a->heads;
    cp.splits = pl.splits;
    cp.h_pad = pl.h_pad;
    cp.out_f32 = a->out_dtype == MR_F32;

    const hipError_t e =
        mr::launch_mla_decode(p, cp, (a->flags & MR_DECODE_SPLIT_ONLY) != 0, (hipEvent_t const*)a->phase_events,
                              (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "mla decode launch");
    return MR_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- no-allocation decode
// Scratch of mr_mla_decode_noalloc: a file-scope device array, one copy per
// GPU, held until the process ends.  In host code `scratch` names a host-side
// stand-in, not device memory: kernels and copies get the device address
// that hipGetSymbolAddress returns for the current device, looked up once
// per device and kept in g_scratch.  The decode writes every byte of the
// scratch it reads in the same call (split partials, then the combine), so
// nothing in it has to start at zero.
namespace {
static __device__ __align__(256) unsigned char scratch[MR_DECODE_NOALLOC_SCRATCH_BYTES];
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

mr_status scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "mla decode (no-alloc): hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(MR_INVALID_ARGUMENT, "mla decode (no-alloc): device %d", dev);
    void* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_acquire);
        if (!p) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p) return hip_fail(e, "mla decode (no-alloc): hipGetSymbolAddress(scratch)");
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MR_OK;
}
}  // namespace

extern "C" mr_status mr_mla_decode_noalloc(const mr_mla_decode_args* a, void* stream) {
    mr_status st = check_decode(a);
    if (st != MR_OK) return st;
    mr_mla_decode_args d = *a;
    d.workspace = nullptr;
    d.workspace_bytes = 0;
    // a synchronous index check reads its result on the host: not here
    if (d.indices && !(d.flags & MR_DECODE_UNCHECKED) && (!d.index_status || (d.flags & MR_DECODE_VALIDATE_INDICES)))
        return fail(MR_INVALID_ARGUMENT, "mla decode (no-alloc): index lists need index_status (device check) or "
                                         "MR_DECODE_UNCHECKED");
    const size_t need = plan_decode(&d).total;
    if (need > MR_DECODE_NOALLOC_SCRATCH_BYTES)
        return fail(MR_WORKSPACE_TOO_SMALL, "mla decode (no-alloc): needs %zu bytes of scratch, the library holds %zu",
                    need, (size_t)MR_DECODE_NOALLOC_SCRATCH_BYTES);
    void* ptr = nullptr;
    if ((st = scratch_address(&ptr)) != MR_OK) return st;
    d.workspace = ptr;
    d.workspace_bytes = MR_DECODE_NOALLOC_SCRATCH_BYTES;
    return mr_mla_decode(&d, stream);
}
