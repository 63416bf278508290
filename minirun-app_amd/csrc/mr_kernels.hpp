// Kernel parameter blocks and launchers shared by the HIP sources and the
// C-ABI layer (capi.cpp).  Internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mr_device.hpp"

namespace mr {

constexpr int MAX_GATHER_ROWS = 1024;     // index rows one decode workgroup stages in LDS
constexpr int MAX_COMBINE_SPLITS = 1024;  // context splits the combine kernel merges

// ---------------------------------------------------------------- decode
struct DecodeParams {
    const uint16_t* q_lat;
    int64_t q_lat_bs, q_lat_hs;
    const uint16_t* q_rope;
    int64_t q_rope_bs, q_rope_hs;
    const uint16_t* latent;
    int64_t lat_rs, lat_bs;
    const uint16_t* rope;
    int64_t rope_rs, rope_bs;
    const int32_t* indices;  // null: dense rows [0, n_ctx)
    int32_t n_idx;
    int32_t batch, heads, n_ctx, rope_dim;
    int32_t n_rows;          // rows attended per batch element (n_ctx or n_idx)
    int32_t splits, rows_per_split, head_groups, h_pad;
    float scale_log2;        // softmax scale * log2(e)
    float* ws_o;             // [batch*splits][h_pad][512]
    float* ws_ml;            // [batch*splits][h_pad][2]
    int32_t* err_flag;       // optional: bit 0 set on an out-of-range index
};

struct CombineParams {
    const float* ws_o;
    const float* ws_ml;
    const float* sinks;  // [heads] or null
    void* out;
    int64_t out_bs, out_hs;
    int32_t batch, heads, splits, h_pad;
    int32_t out_f32;
};

int decode_head_groups(int heads);
hipError_t launch_validate_indices(const int32_t* indices, int32_t batch, int32_t n_idx, int32_t n_rows,
                                   int32_t* result, hipStream_t st);
hipError_t launch_mla_decode(const DecodeParams& p, const CombineParams& cp, bool transpose_reads,
                             hipEvent_t const* events, hipStream_t st);

}  // namespace mr
