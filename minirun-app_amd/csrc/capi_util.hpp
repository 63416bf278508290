// Internal helpers of the C-ABI layer: thread-local error text and checks.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../../include/minirun_hip.h"

namespace mrc {

mr_status fail(mr_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
mr_status hip_fail(hipError_t e, const char* what);
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Workspace arithmetic that cannot wrap: products and sums saturate at
// WS_LIMIT, a size no workspace reaches (64 PiB); a layout that reaches it
// is refused, and its *_workspace_size reports 0.
constexpr size_t WS_LIMIT = size_t(1) << 56;
inline size_t ws_mul(size_t a, size_t b) { return (b && a > WS_LIMIT / b) ? WS_LIMIT : std::min(a * b, WS_LIMIT); }
inline size_t ws_add(size_t a, size_t b) {
    return std::min(a, WS_LIMIT) + std::min(b, WS_LIMIT) >= WS_LIMIT ? WS_LIMIT : a + b;
}
const char* dtype_name(mr_dtype d);
int cu_count();  // compute units of the current device (cached per device)

// Where mr_mla_decode leaves its split partials in the workspace (the layout
// its combine reads): records [batch][h_pad][splits][512] at offset 0, bf16
// (f32 when ws_f32), then (m, l) pairs at ml_offset.
struct DecodePartials {
    int32_t splits, h_pad;
    bool ws_f32;
    size_t ml_offset;
};
DecodePartials decode_partials(const mr_mla_decode_args* a);

// Every check mr_mla_prefill makes before its launches, workspace aside.
mr_status check_prefill(const mr_mla_prefill_args* a);
// mr_mla_prefill with the output gate of MLA.swift:207-211 applied to its
// bf16 output (contiguous [T][H * v] rows, gate rows of the same stride);
// gate null: mr_mla_prefill itself.
mr_status mla_prefill_gated(const mr_mla_prefill_args* a, const void* gate, int64_t gate_ts, void* stream);

}  // namespace mrc
