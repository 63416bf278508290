// Kernel parameter blocks and launchers shared by the HIP sources and the
// C-ABI layer (capi.cpp).  Internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mr_device.hpp"

namespace mr {

constexpr int MAX_GATHER_ROWS = 512;      // index rows one decode workgroup stages in LDS
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
    int32_t hg_size;         // heads per workgroup: 32 or 64
    float scale_log2;        // softmax scale * log2(e)
    void* ws_o;              // [batch][h_pad][splits][512]: O_s / l_s, bf16 (or f32 when ws_f32)
    int32_t ws_f32;
    float* ws_ml;            // [batch][h_pad][splits][2]: m_s (base 2), l_s
    // gathered form: the first check_blocks workgroups check the index list
    // of token blockIdx.x (< batch) and write (status, position, value) to
    // index_status[3 * token]; 0 = no check
    int32_t check_blocks;
    int32_t* index_status;
    // the check workgroups' hash tables (2 * slots int32 per token) for lists
    // too long for LDS; null: in LDS
    int32_t* check_table;
    // x / head_groups and x / splits as __umulhi(x, magic) (floor(2^32 / d)
    // + 1, exact while x * d < 2^32; 0: divide), set by launch_mla_decode
    uint32_t hg_magic, split_magic;
};

struct CombineParams {
    const void* ws_o;  // bf16, or f32 when ws_f32
    int32_t ws_f32;
    const float* ws_ml;
    const float* sinks;  // [heads] or null
    void* out;
    int64_t out_bs, out_hs;
    int32_t batch, heads, splits, h_pad;
    int32_t out_f32;
};

// The split merge fused with the value un-absorption of the decode block
// (MLA.swift:198-206): per head h, ctx = bf16(sum_s w_s O_s / sum_s w_s)
// as mla_combine forms it (no sinks), then out[h][j] = bf16(W_UV[h][j] . ctx)
// for j < v_dim, where W_UV[h][j] is row h * row_step + row0 + j of kv_b.
// The weight is a 4-bit group-64 affine one with bf16 scales and biases
// (rows of 512 inputs contiguous, as MLX stores them) or a dense bf16 one
// (rows 16-byte aligned at stride w_rs).  Batch 1, one workgroup per head.
struct CombineUnabsorbParams {
    const void* ws_o;  // split partials, bf16 (or f32 when ws_f32)
    int32_t ws_f32;
    const float* ws_ml;
    int32_t splits, h_pad, heads;
    int32_t affine;  // 1: 4-bit affine, 0: dense bf16
    const uint32_t* packed;
    const uint16_t* scales;
    const uint16_t* biases;
    const uint16_t* w;
    int64_t w_rs;
    int32_t row_step, row0, v_dim;
    uint16_t* out;  // [heads][v_dim] bf16
};
constexpr int UNABSORB_MAX_V = 128;  // value rows of one head the fused kernel stages
hipError_t launch_combine_unabsorb(const CombineUnabsorbParams& p, hipStream_t st);

// Heads per decode workgroup: 64 when there are more than 32 heads, else 32.
int decode_head_group_size(int heads);
// Index checks (DeepSeekV4Attention.swift:884-895), one workgroup per token:
// result[3 * b] = (status, position, value); lists of at most
// validate_max_indices() entries.  Lists too long for a workgroup's LDS keep
// their hash tables in global memory: validate_table_bytes(batch, n_idx)
// bytes at `tables` (0 bytes, and `tables` unused, for short lists).
int validate_max_indices();
size_t validate_table_bytes(int32_t batch, int32_t n_idx);
hipError_t launch_validate_indices(const int32_t* indices, int32_t batch, int32_t n_idx, int32_t n_rows,
                                   int32_t* tables, int32_t* result, hipStream_t st);
hipError_t launch_mla_decode(const DecodeParams& p, const CombineParams& cp, bool split_only,
                             hipEvent_t const* events, hipStream_t st);

// ---------------------------------------------------------------- prefill
// Up-projection (NT GEMM): kv[p][n] = sum_r latent[p][r] * kv_b[n][r], bf16
// in, fp32 accumulation, bf16 out.  M = rows, N = output features (a
// multiple of 128), K = 512.
struct UpProjParams {
    const uint16_t* a;  // latent rows [M][K], row stride lda
    int64_t lda;
    const uint16_t* b;  // kv_b [N][K], row stride ldb
    int64_t ldb;
    uint16_t* c;        // column block n / 256 at c + (n / 256) * c_hs, rows of stride ldc
    int64_t ldc, c_hs;
    int32_t M, N, K;
};

// Causal attention over the up-projected keys/values.  Head h of key p, with
// r = kv + h * kv_hs + p * kv_rs: K = [r[0..127] ++ rope[p][0..63]],
// V = r[128..255].
// Query i (of T, at cache position P - T + i) attends keys 0 .. P - T + i.
struct PrefillAttnParams {
    const uint16_t* q;  // [T][H][192] bf16 (nope 128 ++ rope 64)
    int64_t q_ts, q_hs;
    const uint16_t* kv;  // head h, key p: kv + h * kv_hs + p * kv_rs, 256 values
    int64_t kv_rs, kv_hs;
    const uint16_t* rope;  // [P][64] rows, stride rope_rs
    int64_t rope_rs;
    void* out;  // [T][H][128]
    int64_t out_ts, out_hs;
    int32_t out_f32;
    int32_t T, P, H;
    float scale_log2;  // softmax scale * log2(e)
    // bf16 out only: null, or the output gate (MLA.swift:207-211) applied
    // as the rows are stored, out = bf16(bf16(attn) * sigmoid(gate)) with
    // gate[i][h * 128 + d] at gate + i * gate_ts
    const uint16_t* gate;
    int64_t gate_ts;
};

hipError_t launch_upproj(const UpProjParams& p, hipStream_t st);

// ---------------------------------------------------------------- any-width MLA (generic.hip)
// The decode and the prefill at widths the fixed-width kernels do not take,
// in fp32; elements are read one by one (no alignment beyond 2 bytes).
constexpr int ANY_MAX_RANK = 2048;  // kv_rank (decode), kv_rank and v_head (prefill)
constexpr int ANY_MAX_ROPE = 512;   // rope width
constexpr int ANY_MAX_NOPE = 1024;  // qk_nope width (prefill)

struct AnyDecodeParams {
    const uint16_t* q_lat;
    int64_t q_lat_bs, q_lat_hs;
    const uint16_t* q_rope;
    int64_t q_rope_bs, q_rope_hs;
    const uint16_t* latent;
    int64_t lat_rs, lat_bs;
    const uint16_t* rope;
    int64_t rope_rs, rope_bs;
    const int32_t* indices;  // null: rows 0 .. n_ctx-1
    int32_t n_idx;
    const float* sinks;      // [heads] or null
    void* out;               // [batch][heads][R] with strides out_bs, out_hs
    int64_t out_bs, out_hs;
    int32_t out_f32;
    int32_t batch, heads, n_ctx, R, DR;
    float scale_log2;
};
hipError_t launch_mla_decode_any(const AnyDecodeParams& p, hipStream_t st);

struct AnyPrefillParams {
    const uint16_t* q;  // [T][H][NOPE + DR]
    int64_t q_ts, q_hs;
    const uint16_t* latent;  // [P][R]
    int64_t lat_rs;
    const uint16_t* rope;  // [P][DR]
    int64_t rope_rs;
    const uint16_t* kv_b;  // [H * (NOPE + V)][R]
    int64_t kvb_rs;
    float* kv;  // workspace [H][P][NOPE + V]
    void* out;  // [T][H][V]
    int64_t out_ts, out_hs;
    int32_t out_f32;
    int32_t T, P, H, R, DR, NOPE, V;
    float scale_log2;
};
hipError_t launch_mla_prefill_any(const AnyPrefillParams& p, hipEvent_t const* events, hipStream_t st);

// ---------------------------------------------------------------- token-tiled projections
// y[M][N] = x[M][K] . W[N][K]^T on MFMA (gemm.hip): x bf16 rows of stride
// ldx; W dense bf16 rows of stride ldw (packed null), or 4-bit affine rows
// (packed [N][K/8] uint32, scales / biases [N][K/group] of scale_dtype 0
// bf16, 1 f16, 2 f32); y bf16 or f32 rows of stride ldy.
struct ProjGemmParams {
    const uint16_t* x;
    int64_t ldx;
    const uint16_t* w;
    int64_t ldw;
    const void* packed;
    const void* scales;
    const void* biases;
    int32_t scale_dtype, group, bits;
    void* y;
    int64_t ldy;
    int32_t y_f32;
    int32_t M, N, K;
};
// Up to three projections of the same M tokens in one launch: entry s owns
// the N tiles tile_end[s-1] .. tile_end[s] - 1 (tile_end past nseg: INT32_MAX).
struct ProjGemmStack {
    ProjGemmParams seg[3];
    int32_t nseg;
    int32_t tile_end[3];
};
constexpr int PROJ_GEMM_MIN_TOKENS = 64;  // fewer tokens take the token-tile GEMV kernels
bool proj_gemm_ok(const ProjGemmParams& p);  // shapes, alignment and formats the kernel takes
hipError_t launch_proj_gemm(const ProjGemmParams& p, int cu_count, hipStream_t st);
// n entries with one M, all dense or all affine, one output dtype; each proj_gemm_ok
hipError_t launch_proj_gemm_stack(const ProjGemmParams* segs, int n, int cu_count, hipStream_t st);
hipError_t launch_prefill_attn(const PrefillAttnParams& p, hipStream_t st);

// ---------------------------------------------------------------- top-k
constexpr int TOPK_MAX = 4096;          // selected keys per row
constexpr int TOPK_SLICE = 32768;       // keys one workgroup ranks in registers

struct TopkParams {
    const float* scores;  // [rows][cols], row stride row_stride
    int64_t row_stride;
    int32_t rows, cols;
    int32_t available, selected;  // keys ranked per row, keys emitted per row
    int32_t ratio, start_pos, offset;
    int32_t* out;  // [rows][selected], row stride out_stride
    int64_t out_stride;
    int32_t* nan_flags;  // [rows]: 1 when the row holds a NaN
    // rows of more than TOPK_SLICE keys (or more than TOPK_MAX selected):
    // `slices` workgroups per row each rank a slice of the keys and write
    // their first min(selected, list_len) composites (score image << 32 |
    // key, ascending; ~0 past them) to cand[row][slice][list_len], and their
    // NaN flag to slice_nan[row][slice]; merge rounds then reduce the sorted
    // lists pairwise (set by the launcher)
    int32_t slices, list_len;
    unsigned long long* cand;
    int32_t* slice_nan;
    // one row: the kernel that writes the row's NaN flag also writes the
    // device status (MR_NONFINITE or 0) here, with no status launch; else null
    int32_t* status_direct;
    // spread selection (a row over many workgroups, set by the launcher):
    // per (row, slice of TOPK_SPREAD_SLICE keys) the slice's keys ordered by
    // their first digit, the digit's start offsets and a coarse copy of them
    int32_t sp_slices;
    unsigned short* sp_coarse;        // [rows][sp_slices][TOPK_SPREAD_CO] (8-byte records)
    unsigned short* sp_off;           // [rows][sp_slices][TOPK_SPREAD_OFF]
    unsigned long long* sp_sorted;    // [rows][sp_slices][TOPK_SPREAD_SLICE]
};
constexpr int TOPK_SPREAD_SLICE = 2048;                  // keys per slice workgroup
constexpr int TOPK_SPREAD_BITS = 12;                     // first digit: the score image's top bits
constexpr int TOPK_SPREAD_BINS = 1 << TOPK_SPREAD_BITS;
constexpr int TOPK_SPREAD_OFF = TOPK_SPREAD_BINS + 8;    // u16 per slice: BINS + 1 offsets, 16-byte rows
constexpr int TOPK_SPREAD_COARSE = 64;                   // coarse bins (of BINS / 64 digit values)
constexpr int TOPK_SPREAD_CO = TOPK_SPREAD_COARSE + 8;   // u16 per slice: 65 coarse offsets, the NaN flag,
                                                         // the smallest composite (u64 at u16 68)
constexpr int TOPK_SPREAD_MAX_SLICES = 128;              // rows of up to 262144 keys
constexpr int TOPK_SPREAD_MAX_ROWS = 8;

// Workspace of a selection: per-row NaN flags; for few rows the spread
// selection's per-slice arrays; for rows of more than TOPK_SLICE keys the
// slice flags and two candidate buffers.
size_t topk_workspace_bytes(int32_t rows, int32_t cols, int32_t selected);
hipError_t launch_topk_select(const TopkParams& p, void* workspace, int32_t* status, hipStream_t st);

// ---------------------------------------------------------------- affine
struct AffineDequantParams {
    const uint32_t* packed;
    const void* scales;
    const void* biases;
    int scale_dtype;  // 0 bf16, 1 f16, 2 f32
    int64_t out_features, in_features;
    int group, bits;
    void* out;
    int out_f32;
};

// y[token m][row j] = sum_i x[m, xvec(j)][i] * W[wrow(j)][i]
//   wrow(j) = (j / map_a) * map_b + map_c + (j % map_a),  xvec(j) = j / map_a
struct AffineGemvParams {
    const void* x;
    int x_f32;
    int64_t x_stride;  // elements between activation vectors
    int m;             // tokens
    const uint32_t* packed;
    const void* scales;
    const void* biases;
    int scale_dtype;
    int out_rows;
    int in_features;
    int group, bits;
    int map_a;
    int64_t map_b, map_c;
    void* y;
    int y_f32;
    int64_t y_stride_row, y_stride_token;
    int force_generic;
    // 4-bit fast path: optional RMSNorm of the activation vector, applied
    // while it is staged (null = plain x), and the launch geometry the host
    // chose (threads per output row, rows per workgroup tile)
    const void* norm_w;
    int norm_w_f32;
    float norm_eps;
    int tpr, tile_rows, tiles_per_vec;
    // routed experts (affineGatherMM): activation vector v reads x row
    // v / x_div and the weight rows of expert rhs_idx[v] (map_a rows each);
    // an expert id outside [0, experts) gives zeros.  Null = the map above.
    const int32_t* rhs_idx;
    int32_t x_div;
    int64_t experts;
};

// Lightning-index scores: out[s][t] = sum_h w[s][h] * max(q[s][h] . k[t], 0).
// Strides in elements; k_bytes is set by the launcher.
struct IndexerParams {
    const void* q;  // [S][H][D]
    int q_f32;
    int64_t q_ss, q_hs;
    const void* k;  // [T][D]
    int k_f32;
    int64_t k_rs;
    const void* w;  // [S][H]
    int w_f32;
    int64_t w_ss;
    float* out;     // [S][out_ss]
    int64_t out_ss;
    int32_t S, H, D, T;
    uint32_t k_bytes;
};
bool indexer_mfma_ok(const IndexerParams& p);
hipError_t launch_indexer_scores(const IndexerParams& p, hipStream_t st);

// ---------------------------------------------------------------- dense projections
// y[t][j] = sum_i x_eff[t, xvec(j)][i] * W[wrow(j)][i], W [rows][in] bf16 or
// f32 (row stride w_rs elements), with
//   wrow(j) = (j / map_a) * map_b + map_c + j % map_a,  xvec(j) = j / map_a.
// Staged launches (one activation vector per token: map_a == out_rows)
// apply the optional RMSNorm or sigmoid gate to x once, in LDS.
constexpr int MAX_GEMV_TOKENS = 8;        // tokens per launch tile
constexpr int DENSE_STAGE_BYTES = 65536;  // staged activations per workgroup (bf16 or fp32)
struct DenseGemvParams {
    const void* x;
    int x_f32;
    int64_t x_stride;      // elements between tokens
    int64_t x_vec_stride;  // elements between the activation vectors of a token (direct mode)
    int m;
    const void* w;
    int w_f32;
    int64_t w_rs;
    int out_rows, in;
    int map_a;
    int64_t map_b, map_c;
    void* y;
    int y_f32;
    int64_t y_stride_row, y_stride_token;
    const void* norm_w;  // optional: x_eff = norm_w * (x * rsqrt(mean(x^2) + eps))
    int norm_w_f32;
    float norm_eps;
    const void* gate;    // optional (not with norm_w): x_eff = x * sigmoid(gate[t * gate_stride + i])
    int gate_f32;
    int64_t gate_stride;
    // staged launches: up to 3 weights with the same in_features stacked
    // along the output rows (rows [seg_end[s-1], seg_end[s]) read seg_w[s],
    // row stride seg_w_rs[s], and write seg_y[s], token stride seg_y_ts[s]);
    // nseg 0 = the single weight w / y above
    int nseg;
    int seg_end[3];
    const void* seg_w[3];
    int64_t seg_w_rs[3];
    void* seg_y[3];
    int64_t seg_y_ts[3];
    int tpr, batches, mt, stage_vec;  // set by the launcher
    int64_t units;
};
// staged: map_a == out_rows and one activation vector fits DENSE_STAGE_BYTES
int dense_gemv_tokens_per_tile(int in, int m, bool x_f32);
hipError_t launch_dense_gemv(DenseGemvParams p, bool staged, int cus, hipStream_t st);

// Latent-cache append of one kv_a row per token (layout in cache_append_row).
struct CacheAppendParams {
    const void* kv;  // [tokens, kv_rank + rope_dim]
    int kv_f32;
    int64_t kv_stride;
    const void* norm_w;
    int w_f32;
    float eps;
    int kv_rank, rope_dim;
    const float* cos_t;  // [tokens, rope_dim/2]; null: the key is stored unrotated (NoPE)
    const float* sin_t;
    uint16_t* latent;
    int64_t latent_stride;
    uint16_t* rope;
    int64_t rope_stride;
    int64_t start_row, tokens;
};

// q_lat[h][r] = sum_{d < nope} q[h][d] * W[h*(nope+v) + d][r], r < 512
// (W_UK of a dense kv_b_proj); optional rotation of q's rotary columns.
struct DenseAbsorbParams {
    uint16_t* q;  // bf16 [heads][q_head_stride], nope part first
    int64_t q_head_stride;
    const void* w;
    int w_f32;
    int64_t w_rs;
    int heads, nope_dim, v_dim;
    uint16_t* q_lat;
    int64_t q_lat_head_stride;
    const float* rope_cos;  // [rope_dim/2] or null
    const float* rope_sin;
    int rope_dim;
    int64_t rope_col0;
    CacheAppendParams app;  // app_on: one extra workgroup appends token 0's cache row in the same launch
    int app_on;
};
hipError_t launch_dense_absorb(const DenseAbsorbParams& p, hipStream_t st);
// out[i] = bf16(x[i] * sigmoid(g[i])), bf16 vectors of n elements
hipError_t launch_gate_mul(const uint16_t* x, const uint16_t* g, int64_t n, uint16_t* out, hipStream_t st);

hipError_t launch_affine_dequant(const AffineDequantParams& p, hipStream_t st);
bool affine_gemv_fast_ok(const AffineGemvParams& p);
hipError_t launch_affine_gemv(const AffineGemvParams& p, hipStream_t st);
// two GEMVs (of one activation vector) as one launch when both take the
// 4-bit fast path with the same scale dtype and geometry class, else two
hipError_t launch_affine_gemv_pair(const AffineGemvParams& a, const AffineGemvParams& b, hipStream_t st);

// ---------------------------------------------------------------- block pieces
struct RmsNormParams {
    const void* x;
    int x_f32;
    int64_t x_stride;
    const void* weight;
    int w_f32;
    void* out;
    int out_f32;
    int64_t out_stride;
    int64_t rows;
    int dim;
    float eps;
};

struct RopeParams {
    void* x;
    int x_f32;
    int64_t n_pos, inner, row_stride, col0;
    int dim;
    const float* cos_t;  // [n_pos, dim/2]
    const float* sin_t;
};


struct AbsorbParams {
    const uint16_t* q;  // [heads, q_head_stride], nope part first
    int64_t q_head_stride;
    const uint32_t* packed;  // kv_b [heads*(nope+v), kv_rank], 4-bit group 64
    const void* scales;
    const void* biases;
    int scale_dtype;
    int heads, nope_dim, v_dim, kv_rank;
    uint16_t* q_lat;
    int64_t q_lat_head_stride;
    // optional: rotate each head's rotary part (one position, adjacent pairs,
    // cos/sin [rope_dim/2]) in place in the same launch; null = none
    const float* rope_cos;
    const float* rope_sin;
    int rope_dim;
    int64_t rope_col0;
    CacheAppendParams app;  // app_on: one extra workgroup appends token 0's cache row in the same launch
    int app_on;
};

hipError_t launch_rmsnorm(const RmsNormParams& p, hipStream_t st);
hipError_t launch_rope(const RopeParams& p, hipStream_t st);
hipError_t launch_cache_append(const CacheAppendParams& p, hipStream_t st);
hipError_t launch_absorb_q(const AbsorbParams& p, hipStream_t st);

}  // namespace mr
