// Lightning-indexer top-k selection on gfx950
// (DeepSeekV4LightningIndexer.selecting, DeepSeekV4Attention.swift:582-645).
//
// Per score row: keys 0 .. available-1 ordered by descending score, ties by
// ascending key id, keys at or past `visible` comparing as -infinity; the
// first `selected` keys are emitted as offset + key, or -1 for a key past
// `visible`.  Exact: the order is a total order on (score, key id) and
// floats are compared, never combined.
//
// One workgroup per row (1024 threads, or 256 for rows of at most 1024
// keys); thread t holds keys j NT + t (j < KPT) in registers as 48-bit
// composites (order-reversing 32-bit image of the score << 16 | key id), so
// every composite is distinct and ascending composite order is the
// reference's order (descending score, ties by ascending key id):
//   1. radix select over the composites (digits of 11, 11, 10, 8 and 8 bits,
//      LDS histograms; the wide first digit spreads the keys over many bins)
//      finds the selected-th smallest composite D;
//   2. every thread writes its composites <= D to LDS at offsets from one
//      block scan (exactly `selected` of them);
//   3. a bitonic sort of those composites in LDS gives the final order.
// The row's NaN flag (any NaN among all `cols` scores) goes to nan_flags.
#include <math.h>

#include <type_traits>

#include "mr_kernels.hpp"

namespace mr {

namespace {

// Increasing in the score's order; -0 and +0 map alike.
__device__ __forceinline__ uint32_t ordered_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u << 1) == 0) u = 0;  // -0 -> +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Inclusive scan of one value per thread over the block; `sh` holds one
// word per wave.  Every thread of the block must call it.
// Inclusive scan over the 64 lanes of a wave on DPP: row_shr 1, 2, 4, 8
// inside rows of 16 lanes (lanes shifted in from outside the row add 0),
// then row_bcast 15 / 31 carry each row's total into the rows above it.
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xf, 0xf, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xf, 0xf, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xf, 0xf, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xf, 0xf, true);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);
    return v;
}

template <int NT>
__device__ __forceinline__ uint32_t block_scan_incl(uint32_t v, uint32_t* sh) {
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
    v = wave_scan_incl(v);
    if (l == 63) sh[w] = v;
    __syncthreads();
    uint32_t base = 0;
    for (int i = 0; i < w; ++i) base += sh[i];
    __syncthreads();
    return v + base;
}

constexpr int TK_BINS = 2048;
constexpr unsigned long long TK_NONE = ~0ull;  // padding: past every composite

template <int NT, int KPT>
__global__ void __launch_bounds__(NT) topk_select_kernel(TopkParams p) {
    // two histograms: a pass counts into one while the other is cleared for
    // the next pass
    __shared__ __attribute__((aligned(16))) uint32_t hist[2][TK_BINS];
    __shared__ uint32_t scan_sh[NT / 64];
    __shared__ uint32_t pick[3];  // bin, count before it, count in it
    __shared__ unsigned long long comp[TOPK_MAX];
    __shared__ int nan_seen;

    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* sr = p.scores + (int64_t)row * p.row_stride;
    const int visible = p.start_pos == 0 ? (row + 1) / p.ratio : p.available;
    const int n = p.available;
    const int k = p.selected;

    if (tid == 0) nan_seen = 0;
    // this thread's keys j NT + tid (coalesced loads): the 32-bit images in
    // registers; the composite of register j is (img[j] << 16 | j NT + tid)
    uint32_t img[KPT];
    bool nan_here = false;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const int key = NT * j + tid;
        const float f = key < p.cols ? sr[min(key, p.cols - 1)] : 0.f;
        nan_here |= key < p.cols && isnan(f);
        img[j] = ~ordered_bits(key < visible ? f : -INFINITY);
    }
    auto valid = [&](int j) { return NT * j + tid < n; };
    // NaN anywhere in the row (all columns, as the reference checks the
    // whole matrix): columns past the registers' range
    for (int i = KPT * NT + tid; i < p.cols; i += NT) nan_here |= isnan(sr[i]);
    __syncthreads();
    if (nan_here) nan_seen = 1;

    // 1. radix select: the k-th smallest composite D = (dimg << 16 | dkey),
    // digits from the top: image bits 31..21, 20..10, 9..0, then key bits
    // 15..8, 7..0 (all in 32-bit arithmetic)
    uint32_t dimg = 0, dkey = 0;
    uint32_t remaining = (uint32_t)k;  // rank of D among the still-matching composites
    for (int i = tid; i < TK_BINS; i += NT) hist[0][i] = 0;
    __syncthreads();
#pragma unroll 1
    for (int pass = 0; pass < 5; ++pass) {
        const bool on_img = pass < 3;
        const int sh = pass == 0 ? 21 : pass == 1 ? 10 : pass == 2 ? 0 : pass == 3 ? 8 : 0;
        const int wd = pass == 0 ? 11 : pass == 1 ? 11 : pass == 2 ? 10 : 8;
        const int top = sh + wd;  // bits at and above `top` of the current field are fixed
        const uint32_t fixed = top >= 32 ? 0u : (0xffffffffu << top);  // no shift by 32
        uint32_t* hc = hist[pass & 1];
        for (int i = tid; i < TK_BINS; i += NT) hist[(pass & 1) ^ 1][i] = 0;  // the next pass's
        if (pass == 0) {
            // every key counts: no branch, padding keys add 0
#pragma unroll
            for (int j = 0; j < KPT; ++j) atomicAdd(&hc[img[j] >> 21], valid(j) ? 1u : 0u);
        } else if (on_img) {
#pragma unroll
            for (int j = 0; j < KPT; ++j)
                if (valid(j) && ((img[j] ^ dimg) & fixed) == 0u) atomicAdd(&hc[(img[j] >> sh) & ((1u << wd) - 1u)], 1u);
        } else {
#pragma unroll
            for (int j = 0; j < KPT; ++j) {
                const uint32_t key = (uint32_t)(NT * j + tid);
                if (valid(j) && img[j] == dimg && ((key ^ dkey) & fixed) == 0u)
                    atomicAdd(&hc[(key >> sh) & ((1u << wd) - 1u)], 1u);
            }
        }
        __syncthreads();
        // wave 0 finds the bin where the running count reaches `remaining`:
        // lane l sums bins 32l .. 32l+31, a wave scan places the lanes, and
        // the one lane whose range crosses the rank walks its bins
        if (tid < 64) {
            uint32_t tot = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const u32x4 q = *(const u32x4*)(hc + 32 * tid + 4 * i);
                tot += (q[0] + q[1]) + (q[2] + q[3]);
            }
            const uint32_t incl = wave_scan_incl(tot);
            uint32_t before = incl - tot;
            if (before < remaining && remaining <= incl) {
                // this lane's range holds the crossing: walk it, four bins a read
#pragma unroll 1
                for (int i = 0; i < 8; ++i) {
                    const u32x4 q = *(const u32x4*)(hc + 32 * tid + 4 * i);
                    const uint32_t q4 = (q[0] + q[1]) + (q[2] + q[3]);
                    if (before + q4 >= remaining) {
                        int b = 0;
                        uint32_t cb = q[0];
                        if (before + cb < remaining) { before += cb; b = 1; cb = q[1]; }
                        if (b == 1 && before + cb < remaining) { before += cb; b = 2; cb = q[2]; }
                        if (b == 2 && before + cb < remaining) { before += cb; b = 3; cb = q[3]; }
                        pick[0] = (uint32_t)(32 * tid + 4 * i + b);
                        pick[1] = before;
                        pick[2] = cb;
                        break;
                    }
                    before += q4;
                }
            }
        }
        __syncthreads();
        if (on_img)
            dimg |= pick[0] << sh;
        else
            dkey |= pick[0] << sh;
        remaining -= pick[1];
        const uint32_t in_bin = pick[2];
        // image complete and every key with that image is taken: D's key
        // part is past them all (ties need the key digits)
        if (pass == 2 && remaining == in_bin) {
            dkey = 0xffffu;
            break;
        }
    }
    // exactly k composites are <= D

    // 2. collection: each thread's composites <= D at offsets from one scan
    auto le_d = [&](int j) {
        const uint32_t key = (uint32_t)(NT * j + tid);
        return valid(j) && (img[j] < dimg || (img[j] == dimg && key <= dkey));
    };
    uint32_t cnt = 0;
#pragma unroll
    for (int j = 0; j < KPT; ++j) cnt += le_d(j);
    uint32_t pos = block_scan_incl<NT>(cnt, scan_sh) - cnt;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
        if (le_d(j)) {
            if (pos < TOPK_MAX) comp[pos] = ((unsigned long long)img[j] << 16) | (uint32_t)(NT * j + tid);
            ++pos;
        }
    // pad to a power of two (at least 4) for the sort
    int npow = 4;
    while (npow < k) npow <<= 1;
    for (int i = k + tid; i < npow; i += NT) comp[i] = TK_NONE;
    __syncthreads();

    // 3. sort, ascending.  Thread t holds elements 4t .. 4t+3 in registers.
    // Each wave sorts its 256 elements (a bitonic network whose lane
    // exchanges have constant distances), then runs of 256, 512, ... merge
    // pairwise through LDS: each output position finds its split by a
    // merge-path binary search (the composites are distinct).
    constexpr int EPT = 4;
    const bool act = EPT * tid < npow;
    const int lane = tid & 63;
    unsigned long long x[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) x[e] = act ? comp[EPT * tid + e] : TK_NONE;
    auto cswap = [&](unsigned long long& lo, unsigned long long& hi, bool up) {
        // lo sits at the lower index: ascending blocks keep the smaller there
        if ((lo > hi) == up) {
            const unsigned long long t = lo;
            lo = hi;
            hi = t;
        }
    };
    auto xchg = [&](unsigned long long v, auto ld_tag) -> unsigned long long {
        constexpr int LD = decltype(ld_tag)::value;
        const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
        uint32_t rlo, rhi;
        if constexpr (LD == 32) {
            const auto a = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
            const auto c = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
            rlo = (lane & 32) ? a[0] : a[1];
            rhi = (lane & 32) ? c[0] : c[1];
        } else if constexpr (LD == 16) {
            const auto a = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
            const auto c = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
            rlo = (lane & 16) ? a[0] : a[1];
            rhi = (lane & 16) ? c[0] : c[1];
        } else {
            rlo = __shfl_xor(lo, LD);
            rhi = __shfl_xor(hi, LD);
        }
        return ((unsigned long long)rhi << 32) | rlo;
    };
    // one bitonic stage with lane distance LD (element stride 4 LD); blocks
    // of `size` elements, ascending unless the block index bit says
    // otherwise (the last size of the wave sort is all ascending)
    auto lane_stage = [&](auto ld_tag, int size, bool all_up) {
        constexpr int LD = decltype(ld_tag)::value;
        const bool lower = (lane & LD) == 0;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const unsigned long long y = xchg(x[e], ld_tag);
            const bool up = all_up || ((EPT * tid) & size) == 0;
            const bool take_min = lower == up;
            x[e] = take_min ? (x[e] < y ? x[e] : y) : (x[e] > y ? x[e] : y);
        }
    };
    auto thread_stages = [&](int size, bool all_up) {  // element strides 2 and 1
        const bool up0 = all_up || ((EPT * tid) & size) == 0;
        const bool up2 = all_up || ((EPT * tid + 2) & size) == 0;
        if (size >= 4) {
            cswap(x[0], x[2], up0);
            cswap(x[1], x[3], up0);
        }
        cswap(x[0], x[1], up0);
        cswap(x[2], x[3], up2);
    };
    using L1 = std::integral_constant<int, 1>;
    using L2 = std::integral_constant<int, 2>;
    using L4 = std::integral_constant<int, 4>;
    using L8 = std::integral_constant<int, 8>;
    using L16 = std::integral_constant<int, 16>;
    using L32 = std::integral_constant<int, 32>;
    {
        const int wsize = min(npow, 256);  // elements each wave sorts
        // size 2, 4
        thread_stages(2, wsize == 2);
        if (wsize >= 4) thread_stages(4, wsize == 4);
        if (wsize >= 8) { lane_stage(L1{}, 8, wsize == 8); thread_stages(8, wsize == 8); }
        if (wsize >= 16) {
            lane_stage(L2{}, 16, wsize == 16); lane_stage(L1{}, 16, wsize == 16); thread_stages(16, wsize == 16);
        }
        if (wsize >= 32) {
            lane_stage(L4{}, 32, wsize == 32); lane_stage(L2{}, 32, wsize == 32); lane_stage(L1{}, 32, wsize == 32);
            thread_stages(32, wsize == 32);
        }
        if (wsize >= 64) {
            lane_stage(L8{}, 64, wsize == 64); lane_stage(L4{}, 64, wsize == 64); lane_stage(L2{}, 64, wsize == 64);
            lane_stage(L1{}, 64, wsize == 64); thread_stages(64, wsize == 64);
        }
        if (wsize >= 128) {
            lane_stage(L16{}, 128, wsize == 128); lane_stage(L8{}, 128, wsize == 128);
            lane_stage(L4{}, 128, wsize == 128); lane_stage(L2{}, 128, wsize == 128);
            lane_stage(L1{}, 128, wsize == 128); thread_stages(128, wsize == 128);
        }
        if (wsize >= 256) {
            lane_stage(L32{}, 256, true); lane_stage(L16{}, 256, true); lane_stage(L8{}, 256, true);
            lane_stage(L4{}, 256, true); lane_stage(L2{}, 256, true); lane_stage(L1{}, 256, true);
            thread_stages(256, true);
        }
    }
    // merge sorted runs of `run` elements pairwise, in place in LDS
    for (int run = 256; run < npow; run <<= 1) {
        __syncthreads();  // readers of the last round are done
        if (act) {
#pragma unroll
            for (int e = 0; e < EPT; ++e) comp[EPT * tid + e] = x[e];
        }
        __syncthreads();
        if (act) {
            const int q0 = EPT * tid;
            const int base = q0 & ~(2 * run - 1);  // pair start
            const unsigned long long* A = comp + base;
            const unsigned long long* B = A + run;
            const int q = q0 - base;  // output position within the pair
            // i = number of the first q outputs taken from A
            int lo = max(0, q - run), hi = min(q, run);
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (A[mid] < B[q - mid - 1])
                    lo = mid + 1;
                else
                    hi = mid;
            }
            int ia = lo, ib = q - lo;
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                const unsigned long long va = ia < run ? A[ia] : TK_NONE;
                const unsigned long long vb = ib < run ? B[ib] : TK_NONE;
                const bool ta = va < vb;
                x[e] = ta ? va : vb;
                ia += ta;
                ib += !ta;
            }
        }
    }

    int32_t* orow = p.out + (int64_t)row * p.out_stride;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int i = EPT * tid + e;
        if (i < k) {
            const int key = (int)(uint32_t)(x[e] & 0xffffull);
            orow[i] = key >= visible ? -1 : p.offset + key;
        }
    }
    if (tid == 0) p.nan_flags[row] = nan_seen;
}

// Rows of more than 32768 keys (up to 65535): the same selection with the
// row re-read from global memory on every pass (one 1024-thread workgroup,
// 4 radix passes of 8 bits on the 32-bit image, then a chunked sweep that
// takes the keys below the selected value and the first equal ones in key
// order).
constexpr int TK_THREADS = 1024;

// Sorting ascending by this image sorts scores descending.
__device__ __forceinline__ uint32_t desc_image(const float* row, int key, int visible) {
    const float f = key < visible ? row[key] : -INFINITY;
    return ~ordered_bits(f);
}

// Inclusive scan over a 1024-thread block; `sh` holds >= 16 words.
__device__ __forceinline__ uint32_t block_scan_incl_1024(uint32_t v, uint32_t* sh) {
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

__global__ void __launch_bounds__(TK_THREADS) topk_select_gmem_kernel(TopkParams p) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t scan_sh[16];
    __shared__ uint32_t pick[3];  // bin, count before it, count in it
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
        const uint32_t incl = block_scan_incl_1024(h, scan_sh);
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
    const uint32_t both = block_scan_incl_1024(c_less | (c_eq << 16), scan_sh) - (c_less | (c_eq << 16));
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
    // keys per thread: the row's ranked keys in registers
    const dim3 g((unsigned)p.rows);
    if (p.available <= 256 * 4)
        hipLaunchKernelGGL((topk_select_kernel<256, 4>), g, dim3(256), 0, st, p);
    else if (p.available <= 1024 * 16)
        hipLaunchKernelGGL((topk_select_kernel<1024, 16>), g, dim3(1024), 0, st, p);
    else if (p.available <= 1024 * 32)
        hipLaunchKernelGGL((topk_select_kernel<1024, 32>), g, dim3(1024), 0, st, p);
    else
        hipLaunchKernelGGL(topk_select_gmem_kernel, g, dim3(TK_THREADS), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && status) {
        hipLaunchKernelGGL(topk_status_kernel, dim3(1), dim3(256), 0, st, p.nan_flags, p.rows, status);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace mr
