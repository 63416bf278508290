// Lightning-indexer top-k selection on gfx950
// (DeepSeekV4LightningIndexer.selecting, DeepSeekV4Attention.swift:582-645).
//
// Per score row: keys 0 .. available-1 ordered by descending score, ties by
// ascending key id, keys at or past `visible` comparing as -infinity; the
// first `selected` keys are emitted as offset + key, or -1 for a key past
// `visible`.  Exact: the order is a total order on (score, key id) and
// floats are compared, never combined.
//
// One 1024-thread workgroup per row:
//   1. radix select over an order-reversing 32-bit image of the score
//      (4 passes of 8 bits, LDS histograms) finds the value D of the
//      selected-th key and how many keys sort strictly before it;
//   2. one chunked sweep collects every key below D and the first keys equal
//      to D in key order (the tie rule) as 64-bit (image << 32 | key);
//   3. a bitonic sort of those composites in LDS gives the final order.
// The row's NaN flag (any NaN among all `cols` scores) goes to nan_flags.
#include <math.h>

#include "mr_kernels.hpp"

namespace mr {

namespace {

constexpr int TK_THREADS = 1024;

// Increasing in the score's order; -0 and +0 map alike.
__device__ __forceinline__ uint32_t ordered_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u << 1) == 0) u = 0;  // -0 -> +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Sorting ascending by this image sorts scores descending.
__device__ __forceinline__ uint32_t desc_image(const float* row, int key, int visible) {
    const float f = key < visible ? row[key] : -INFINITY;
    return ~ordered_bits(f);
}

// Inclusive scan of one value per thread over the block; `sh` holds >= 16
// words.  Every thread of the block must call it.
__device__ __forceinline__ uint32_t block_scan_incl(uint32_t v, uint32_t* sh) {
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(v, o);
        if (l >= o) v += t;
    }
    if (l == 63) sh[w] = v;
    __syncthreads();
    uint32_t base = 0;
    for (int i = 0; i < w; ++i) base += sh[i];
    __syncthreads();
    return v + base;
}

__global__ void __launch_bounds__(TK_THREADS) topk_select_kernel(TopkParams p) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t scan_sh[16];
    __shared__ uint32_t pick[2];  // bin, count before bin
    __shared__ unsigned long long comp[TOPK_MAX];
    __shared__ int nan_seen;

    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* sr = p.scores + (int64_t)row * p.row_stride;
    const int visible = p.start_pos == 0 ? (row + 1) / p.ratio : p.available;
    const int n = p.available;
    const int k = p.selected;

    // NaN anywhere in the row (all columns, as the reference checks the
    // whole matrix)
    if (tid == 0) nan_seen = 0;
    __syncthreads();
    bool nan_here = false;
    for (int i = tid; i < p.cols; i += TK_THREADS) nan_here |= isnan(sr[i]);
    if (nan_here) nan_seen = 1;

    // 1. radix select on the 32-bit image: the k-th smallest value D
    uint32_t prefix = 0, mask = 0;
    uint32_t remaining = (uint32_t)k;  // how many of the still-tied keys to take
#pragma unroll 1
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += TK_THREADS) {
            const uint32_t d = desc_image(sr, i, visible);
            if ((d & mask) == prefix) atomicAdd(&hist[(d >> shift) & 255u], 1u);
        }
        __syncthreads();
        const uint32_t h = tid < 256 ? hist[tid] : 0u;
        const uint32_t incl = block_scan_incl(h, scan_sh);
        if (tid < 256 && incl >= remaining && incl - h < remaining) {
            pick[0] = (uint32_t)tid;
            pick[1] = incl - h;
        }
        __syncthreads();
        prefix |= pick[0] << shift;
        mask |= 255u << shift;
        remaining -= pick[1];
        __syncthreads();
    }
    const uint32_t D = prefix;
    const uint32_t n_less = (uint32_t)k - remaining;  // keys strictly before D

    // 2. collection: thread t sweeps keys [t*C, (t+1)*C) in order
    const int C = (n + TK_THREADS - 1) / TK_THREADS;
    const int lo = min(tid * C, n), hi = min(lo + C, n);
    uint32_t c_less = 0, c_eq = 0;
    for (int i = lo; i < hi; ++i) {
        const uint32_t d = desc_image(sr, i, visible);
        c_less += d < D;
        c_eq += d == D;
    }
    // both counts fit 16 bits (n <= 65535)
    const uint32_t both = block_scan_incl(c_less | (c_eq << 16), scan_sh) - (c_less | (c_eq << 16));
    uint32_t pos_less = both & 0xffffu, rank_eq = both >> 16;
    for (int i = lo; i < hi; ++i) {
        const uint32_t d = desc_image(sr, i, visible);
        const unsigned long long cv = ((unsigned long long)d << 32) | (uint32_t)i;
        if (d < D) {
            comp[pos_less++] = cv;
        } else if (d == D) {
            if (rank_eq < remaining) comp[n_less + rank_eq] = cv;
            ++rank_eq;
        }
    }
    // pad to a power of two for the sort
    int npow = 1;
    while (npow < k) npow <<= 1;
    for (int i = k + tid; i < npow; i += TK_THREADS) comp[i] = ~0ull;
    __syncthreads();

    // 3. bitonic sort, ascending
    for (int size = 2; size <= npow; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < npow; i += TK_THREADS) {
                const int j = i ^ stride;
                if (j > i) {
                    const unsigned long long a = comp[i], b = comp[j];
                    const bool up = (i & size) == 0;
                    if ((a > b) == up) {
                        comp[i] = b;
                        comp[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }

    int32_t* orow = p.out + (int64_t)row * p.out_stride;
    for (int i = tid; i < k; i += TK_THREADS) {
        const int key = (int)(uint32_t)(comp[i] & 0xffffffffull);
        orow[i] = key >= visible ? -1 : p.offset + key;
    }
    if (tid == 0) p.nan_flags[row] = nan_seen;
}

// status = MR_NONFINITE (5) when any row flagged a NaN, else 0
__global__ void __launch_bounds__(256) topk_status_kernel(const int32_t* flags, int32_t rows, int32_t* status) {
    __shared__ int any;
    if (threadIdx.x == 0) any = 0;
    __syncthreads();
    bool f = false;
    for (int i = threadIdx.x; i < rows; i += 256) f |= flags[i] != 0;
    if (f) any = 1;
    __syncthreads();
    if (threadIdx.x == 0) *status = any ? 5 : 0;
}

}  // namespace

hipError_t launch_topk_select(const TopkParams& p, int32_t* status, hipStream_t st) {
    hipLaunchKernelGGL(topk_select_kernel, dim3((unsigned)p.rows), dim3(TK_THREADS), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && status) {
        hipLaunchKernelGGL(topk_status_kernel, dim3(1), dim3(256), 0, st, p.nan_flags, p.rows, status);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace mr
