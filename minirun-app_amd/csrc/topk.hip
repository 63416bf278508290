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
//
// A few rows of more than 1024 keys (a decode token's row) spread over many
// workgroups instead: see topk_spread_slice / topk_spread_finish.
//
// Other rows of more than 32768 keys split into slices of 32768, one workgroup
// each (the same kernel, in parallel), which emit their own first
// `selected` keys as sorted 64-bit composites (image << 32 | key); merge
// rounds (topk_merge_kernel) then take the first `selected` of the merge of
// two sorted lists, each output position finding its split by a merge-path
// binary search, until one list is left; the last round writes the keys.
// The order is the same total order, so the result is the same.
#include <math.h>

#include <algorithm>
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
// Rows ranked by 1024 threads take the compacted path when the first digit's
// cut bin holds at most TK_CAND keys: the keys above the cut go straight to
// the selected list and only the cut bin's keys take the remaining digits.
constexpr int TK_CAND = 4096;
// Bucket order of the selected keys: buckets over the span of their score
// images; a bucket of more than TK_BUCKET_MAX keys (ties, a few distinct
// scores) sends the row to the bitonic sort instead.
constexpr int TK_BUCKET_MAX = 32;

// Bitonic sort of the 64 EPT composites one wave holds in registers (lane l:
// elements EPT l .. EPT l + EPT-1), ascending within every run of wsize
// elements (wsize a power of two, 2 <= wsize <= 64 EPT).  The lane exchanges
// have constant distances: DPP moves inside rows of 16 lanes, permlane swaps
// across them (no LDS round trips).
template <int EPT>
__device__ void wave_sort(unsigned long long (&x)[EPT], int wsize) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
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
        } else if constexpr (LD <= 2) {
            // quad_perm 1,0,3,2 / 2,3,0,1
            constexpr int Q = LD == 1 ? 0xB1 : 0x4E;
            rlo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, Q, 0xf, 0xf, false);
            rhi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, Q, 0xf, 0xf, false);
        } else {
            // row_shl:LD for the lower lane of a pair (partner LD up, in
            // the same row of 16), row_shr:LD for the upper one
            constexpr int SHL = 0x100 + LD, SHR = 0x110 + LD;
            const uint32_t ulo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, SHL, 0xf, 0xf, false);
            const uint32_t uhi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, SHL, 0xf, 0xf, false);
            const uint32_t dlo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)lo, SHR, 0xf, 0xf, false);
            const uint32_t dhi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)hi, SHR, 0xf, 0xf, false);
            rlo = (lane & LD) ? dlo : ulo;
            rhi = (lane & LD) ? dhi : uhi;
        }
        return ((unsigned long long)rhi << 32) | rlo;
    };
    // one bitonic stage with lane distance LD (element stride EPT LD);
    // blocks of `size` elements, ascending unless the block index bit
    // says otherwise (the last size of the wave sort is all ascending)
    auto lane_stage = [&](auto ld_tag, int size, bool all_up) {
        constexpr int LD = decltype(ld_tag)::value;
        const bool lower = (lane & LD) == 0;
        const bool up = all_up || ((EPT * tid) & size) == 0;
        const bool take_min = lower == up;
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
            const unsigned long long y = xchg(x[e], ld_tag);
            x[e] = take_min ? (x[e] < y ? x[e] : y) : (x[e] > y ? x[e] : y);
        }
    };
    auto lane_stage_d = [&](int ld, int size, bool all_up) {  // ld wave-uniform
        switch (ld) {
            case 1: lane_stage(std::integral_constant<int, 1>{}, size, all_up); break;
            case 2: lane_stage(std::integral_constant<int, 2>{}, size, all_up); break;
            case 4: lane_stage(std::integral_constant<int, 4>{}, size, all_up); break;
            case 8: lane_stage(std::integral_constant<int, 8>{}, size, all_up); break;
            case 16: lane_stage(std::integral_constant<int, 16>{}, size, all_up); break;
            default: lane_stage(std::integral_constant<int, 32>{}, size, all_up); break;
        }
    };
    // element distances below EPT, inside the thread
    auto thread_stages = [&](int size, bool all_up) {
        if constexpr (EPT == 4) {
            const bool up0 = all_up || ((EPT * tid) & size) == 0;
            const bool up2 = all_up || ((EPT * tid + 2) & size) == 0;
            if (size >= 4) {
                cswap(x[0], x[2], up0);
                cswap(x[1], x[3], up0);
            }
            cswap(x[0], x[1], up0);
            cswap(x[2], x[3], up2);
        } else {
            cswap(x[0], x[1], all_up || ((EPT * tid) & size) == 0);
        }
    };
#pragma unroll 1
    for (int size = 2; size <= wsize; size <<= 1) {
        const bool all_up = size == wsize;
#pragma unroll 1
        for (int d = size >> 1; d >= EPT; d >>= 1) lane_stage_d(d / EPT, size, all_up);
        thread_stages(size, all_up);
    }
}

// Ascending sort of comp[0 .. npow) in LDS (npow a power of two, 4 <= npow
// <= EPT NT, padded with TK_NONE; the composites distinct).  Thread t holds
// elements EPT t .. EPT t + EPT-1 in registers.  Each wave sorts its 64 EPT
// elements (wave_sort), then runs of 64 EPT, 128 EPT, ... merge pairwise
// through LDS: each output position finds its split by a merge-path binary
// search.  On return x[e] is element EPT t + e of the sorted order; comp
// holds the last merge's input.
template <int NT, int EPT>
__device__ void sort_lds(unsigned long long* comp, int npow, unsigned long long (&x)[EPT]) {
    const int tid = threadIdx.x;
    const bool act = EPT * tid < npow;
#pragma unroll
    for (int e = 0; e < EPT; ++e) x[e] = act ? comp[EPT * tid + e] : TK_NONE;
    wave_sort<EPT>(x, min(npow, 64 * EPT));
    // merge sorted runs of `run` elements pairwise, in place in LDS
#pragma unroll 1
    for (int run = 64 * EPT; run < npow; run <<= 1) {
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
}

template <int NT, int KPT>
__global__ void __launch_bounds__(NT) topk_select_kernel(TopkParams p) {
    // two histograms: a pass counts into one while the other is cleared for
    // the next pass
    __shared__ __attribute__((aligned(16))) uint32_t hist[2][TK_BINS];
    __shared__ uint32_t scan_sh[NT / 64];
    __shared__ uint32_t pick[3];  // bin, count before it, count in it
    __shared__ unsigned long long comp[TOPK_MAX];
    constexpr bool FAST = NT == 1024;  // the compacted path (four candidates per thread)
    constexpr int CPT = FAST ? TK_CAND / NT : 1;
    __shared__ unsigned long long cand[FAST ? TK_CAND : 1];
    __shared__ int nan_seen;

    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    // the slice of the row this workgroup ranks (the whole row when slices == 1)
    const int slice = blockIdx.y;
    const int key0 = slice * (NT * KPT);
    const float* sr = p.scores + (int64_t)row * p.row_stride + key0;
    const int visible = (p.start_pos == 0 ? (row + 1) / p.ratio : p.available) - key0;
    const int n = min(max(p.available - key0, 0), NT * KPT);  // keys of this slice
    const int cols = p.cols - key0;
    const int k = min(p.selected, n);

    if (tid == 0) nan_seen = 0;
    // this thread's keys j NT + tid (coalesced loads): the 32-bit images in
    // registers; the composite of register j is (img[j] << 16 | j NT + tid)
    uint32_t img[KPT];
    bool nan_here = false;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const int key = NT * j + tid;
        const float f = key < cols ? sr[min(key, cols - 1)] : 0.f;
        nan_here |= key < cols && isnan(f);
        img[j] = ~ordered_bits(key < visible ? f : -INFINITY);
    }
    auto valid = [&](int j) { return NT * j + tid < n; };
    // NaN anywhere in the row (all columns, as the reference checks the
    // whole matrix): the last slice checks the columns past every slice
    if (slice == (int)gridDim.y - 1)
        for (int i = KPT * NT + tid; i < cols; i += NT) nan_here |= isnan(sr[i]);
    __syncthreads();
    if (nan_here) nan_seen = 1;

    // 1. radix select: the k-th smallest composite D = (dimg << 16 | dkey),
    // digits from the top: image bits 31..21, 20..10, 9..0, then key bits
    // 15..8, 7..0 (all in 32-bit arithmetic)
    uint32_t dimg = 0, dkey = 0;
    uint32_t remaining = (uint32_t)k;  // rank of D among the still-matching composites
    uint32_t cut_count = 0;            // keys in the first digit's cut bin
    bool fast = false;
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
        // few keys share the cut bin: rank them apart from the rest
        if (FAST && pass == 0 && in_bin <= (uint32_t)TK_CAND) {
            cut_count = in_bin;
            fast = true;
            break;
        }
        // image complete and every key with that image is taken: D's key
        // part is past them all (ties need the key digits)
        if (pass == 2 && remaining == in_bin) {
            dkey = 0xffffu;
            break;
        }
    }
    // exactly k composites are <= D

    auto composite = [&](int j) { return ((unsigned long long)img[j] << 16) | (uint32_t)(NT * j + tid); };
    static_assert(TK_BINS % 1024 == 0 && TK_CAND >= TOPK_MAX, "bucket arrays");
    if (FAST && fast) {
        // 2a. keys of bins above the cut bin are all taken: to comp; keys of
        // the cut bin to cand.  One scan places both (counts packed 16:16).
        const uint32_t top = dimg >> 21;
        uint32_t ns = 0, nc = 0;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint32_t b = img[j] >> 21;
            ns += valid(j) && b < top;
            nc += valid(j) && b == top;
        }
        const uint32_t pk = (ns << 16) | nc;
        const uint32_t ex = block_scan_incl<NT>(pk, scan_sh) - pk;
        uint32_t ps = ex >> 16, pc = ex & 0xffffu;
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const uint32_t b = img[j] >> 21;
            if (valid(j) && b < top) comp[ps++] = composite(j);
            if (valid(j) && b == top) cand[pc++] = composite(j);
        }
        __syncthreads();
        const uint32_t before = (uint32_t)k - remaining;
        // 2b. the remaining-th smallest candidate: 8-bit digits of composite
        // bits 36..0 (image bits 20..0, then the key), 256-bin histograms
        unsigned long long cv[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int idx = tid + NT * i;
            cv[i] = idx < (int)cut_count ? cand[idx] : TK_NONE;
        }
        unsigned long long dacc = (unsigned long long)top << 37;
        unsigned long long dsel = dacc | ((1ull << 37) - 1ull);  // the whole bin, unless a digit cuts it
        if (remaining != cut_count) {
#pragma unroll 1
            for (int q = 0; q < 5; ++q) {
                const int sh = q == 0 ? 29 : q == 1 ? 21 : q == 2 ? 16 : q == 3 ? 8 : 0;
                const int wd = q == 2 ? 5 : 8;
                uint32_t* hc = hist[(q + 1) & 1];  // hist[1] was cleared during the first pass
                if (tid < 256) hist[q & 1][tid] = 0;  // the next digit's
#pragma unroll
                for (int i = 0; i < CPT; ++i)
                    if (cv[i] != TK_NONE && ((cv[i] ^ dacc) >> (sh + wd)) == 0ull)
                        atomicAdd(&hc[(uint32_t)(cv[i] >> sh) & ((1u << wd) - 1u)], 1u);
                __syncthreads();
                if (tid < 64) {  // lane l sums bins 4l .. 4l+3; the crossing lane walks them
                    const u32x4 h4 = *(const u32x4*)(hc + 4 * tid);
                    const uint32_t tot = (h4[0] + h4[1]) + (h4[2] + h4[3]);
                    const uint32_t incl = wave_scan_incl(tot);
                    uint32_t bef = incl - tot;
                    if (bef < remaining && remaining <= incl) {
                        int b = 0;
                        uint32_t cb = h4[0];
                        if (bef + cb < remaining) { bef += cb; b = 1; cb = h4[1]; }
                        if (b == 1 && bef + cb < remaining) { bef += cb; b = 2; cb = h4[2]; }
                        if (b == 2 && bef + cb < remaining) { bef += cb; b = 3; cb = h4[3]; }
                        pick[0] = (uint32_t)(4 * tid + b);
                        pick[1] = bef;
                        pick[2] = cb;
                    }
                }
                __syncthreads();
                dacc |= (unsigned long long)pick[0] << sh;
                remaining -= pick[1];
                if (remaining == pick[2]) {  // every candidate with this prefix is taken
                    dsel = dacc | ((1ull << sh) - 1ull);
                    break;
                }
            }
        }
        // 2c. the candidates <= dsel (exactly the remaining ones) after the taken keys
        uint32_t cnt = 0;
#pragma unroll
        for (int i = 0; i < CPT; ++i) cnt += cv[i] <= dsel;
        uint32_t pos = before + block_scan_incl<NT>(cnt, scan_sh) - cnt;
#pragma unroll
        for (int i = 0; i < CPT; ++i)
            if (cv[i] <= dsel) comp[pos++] = cv[i];
    } else {
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
                if (pos < TOPK_MAX) comp[pos] = composite(j);
                ++pos;
            }
    }
    // pad to a power of two (at least 4) for the sort
    int npow = 4;
    while (npow < k) npow <<= 1;
    for (int i = k + tid; i < npow; i += NT) comp[i] = TK_NONE;
    __syncthreads();

    // 3. sort, ascending (sort_lds, EPT = 2 when the padded count fits 2 per
    // thread, so every wave works; else 4).  The sorted keys go out as
    // offsets (or, per slice, as 64-bit composites for the merge rounds).
    auto sort_and_emit = [&](auto ept_tag) {
        constexpr int EPT = decltype(ept_tag)::value;
        unsigned long long x[EPT];
        sort_lds<NT, EPT>(comp, npow, x);
        if (p.slices > 1) {  // this slice's sorted composites, ~0 past its keys
            unsigned long long* crow = p.cand + ((int64_t)row * p.slices + slice) * p.list_len;
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                const int i = EPT * tid + e;
                if (i < p.list_len)
                    crow[i] = i < k ? ((x[e] >> 16) << 32) | (uint32_t)(key0 + (int)(uint32_t)(x[e] & 0xffffull)) : TK_NONE;
            }
            // the list past what the sort held
            for (int i = EPT * NT + tid; i < p.list_len; i += NT) crow[i] = TK_NONE;
            return;
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
    };
    // 3a. bucket order: bucket = (image - smallest image) >> shift, with
    // shift the least that fits the span into TK_BINS buckets; counts, one
    // scan and a scatter place the buckets, and a key's place inside its
    // bucket is the number of its bucket's keys below it
    bool bucketed = false;
    if (FAST && k > 1) {  // cand holds the scattered keys (1024-thread rows)
        uint32_t* cnt_b = hist[0];
        uint32_t* cur_b = hist[1];
        uint32_t mn = 0xffffffffu, mx = 0u;
        for (int i = tid; i < k; i += NT) {
            const uint32_t im = (uint32_t)(comp[i] >> 16);
            mn = min(mn, im);
            mx = max(mx, im);
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            mn = min(mn, (uint32_t)__shfl_xor((int)mn, o));
            mx = max(mx, (uint32_t)__shfl_xor((int)mx, o));
        }
        if ((tid & 63) == 0) {
            cur_b[tid >> 6] = mn;
            cur_b[32 + (tid >> 6)] = mx;
        }
        __syncthreads();
        mn = cur_b[0];
        mx = cur_b[32];
        for (int w = 1; w < NT / 64; ++w) {
            mn = min(mn, cur_b[w]);
            mx = max(mx, cur_b[32 + w]);
        }
        const uint32_t span = mx - mn;
        const int bits = span ? 32 - __builtin_clz(span) : 0;
        const int shift = max(0, bits - 11);  // span >> shift < 2048 = TK_BINS
        auto bucket = [&](unsigned long long c) { return ((uint32_t)(c >> 16) - mn) >> shift; };
        __syncthreads();  // the reduction's words are read
        for (int i = tid; i < TK_BINS; i += NT) {
            cnt_b[i] = 0;
            cur_b[i] = 0;
        }
        __syncthreads();
        for (int i = tid; i < k; i += NT) atomicAdd(&cnt_b[bucket(comp[i])], 1u);
        __syncthreads();
        // the fullest bucket decides; then start offsets by one scan
        constexpr int BPT = TK_BINS / NT;  // buckets per thread (2 or 8)
        uint32_t bc[BPT], tot = 0, big = 0;
#pragma unroll
        for (int e = 0; e < BPT; ++e) {
            bc[e] = cnt_b[BPT * tid + e];
            tot += bc[e];
            big = max(big, bc[e]);
        }
        const bool any_big = __syncthreads_or(big > (uint32_t)TK_BUCKET_MAX);
        if (!any_big) {
            uint32_t st = block_scan_incl<NT>(tot, scan_sh) - tot;
#pragma unroll
            for (int e = 0; e < BPT; ++e) {
                cur_b[BPT * tid + e] = st;
                st += bc[e];
            }
            __syncthreads();
            for (int i = tid; i < k; i += NT) {
                const unsigned long long c = comp[i];
                cand[atomicAdd(&cur_b[bucket(c)], 1u)] = c;
            }
            __syncthreads();
            // cur_b[b] is now the end of bucket b
            for (int i = tid; i < k; i += NT) {
                const unsigned long long c = cand[i];
                const uint32_t b = bucket(c);
                const uint32_t end = cur_b[b], start = end - cnt_b[b];
                uint32_t r = 0;
                for (uint32_t j = start; j < end; ++j) r += cand[j] < c;
                comp[start + r] = c;
            }
            __syncthreads();
            bucketed = true;
        }
    }
    if (bucketed || k <= 1) {
        if (p.slices > 1) {  // this slice's sorted composites, ~0 past its keys
            unsigned long long* crow = p.cand + ((int64_t)row * p.slices + slice) * p.list_len;
            for (int i = tid; i < p.list_len; i += NT)
                crow[i] = i < k ? ((comp[i] >> 16) << 32) | (uint32_t)(key0 + (int)(uint32_t)(comp[i] & 0xffffull)) : TK_NONE;
        } else {
            int32_t* orow = p.out + (int64_t)row * p.out_stride;
            for (int i = tid; i < k; i += NT) {
                const int key = (int)(uint32_t)(comp[i] & 0xffffull);
                orow[i] = key >= visible ? -1 : p.offset + key;
            }
        }
    } else if (npow <= 2 * NT) {
        sort_and_emit(std::integral_constant<int, 2>{});
    } else {
        sort_and_emit(std::integral_constant<int, 4>{});
    }
    if (p.slices > 1) {
        if (tid == 0) p.slice_nan[row * p.slices + slice] = nan_seen;
        return;
    }
    if (tid == 0) {
        p.nan_flags[row] = nan_seen;
        if (p.status_direct) *p.status_direct = nan_seen ? 5 /* MR_NONFINITE */ : 0;
    }
}

// ---------------------------------------------------------------------------
// Spread selection: one row over many workgroups (a decode token's row of
// many keys).  Two launches, the kernel boundary between them the only
// hand-off:
//   1. topk_spread_slice, one workgroup per TOPK_SPREAD_SLICE keys: the keys'
//      composites (image << 32 | key id, 64-bit) ordered by their first digit
//      (the image's top TOPK_SPREAD_BITS bits) by a counting sort (LDS
//      histogram, one scan, a scatter by LDS cursors), written out with the
//      digit's start offsets, every 64th offset (coarse) and the NaN flag;
//   2. topk_spread_finish, one workgroup per row: the coarse offsets summed
//      over the slices give the coarse bin that holds the selected-th key,
//      the fine offsets inside it the cut digit value.  Keys of smaller
//      digits are all taken (each slice's are a prefix of its ordered keys);
//      the cut value's keys (the next run of each slice) are candidates, and
//      a radix select over the rest of their composite (8-bit digits) finds
//      the last one taken.  The selected keys are then ordered: buckets over
//      the span of their composites (counts, one scan, a scatter, the rank
//      inside the bucket), or the bitonic sort when a bucket holds more than
//      TK_BUCKET_MAX keys.
// The order is the same total order as the one-workgroup kernel's.

// 64-bit min / max over the wave (DPP within rows of 16 lanes, then
// permlane swaps across rows); every lane ends with the result.
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((unsigned long long)hi << 32) | lo;
}
template <bool MAX>
__device__ __forceinline__ unsigned long long wave_ext_u64(unsigned long long v) {
    auto f = [](unsigned long long a, unsigned long long b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = f(v, dpp_u64<0xB1>(v));   // quad_perm 1,0,3,2
    v = f(v, dpp_u64<0x4E>(v));   // quad_perm 2,3,0,1
    v = f(v, dpp_u64<0x141>(v));  // row_half_mirror
    v = f(v, dpp_u64<0x140>(v));  // row_mirror
    {
        // one element of each pair is this lane's own value, the other its partner's
        const auto a = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
        const auto b = __builtin_amdgcn_permlane16_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
        v = f(((unsigned long long)b[0] << 32) | a[0], ((unsigned long long)b[1] << 32) | a[1]);
    }
    {
        const auto a = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
        const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
        v = f(((unsigned long long)b[0] << 32) | a[0], ((unsigned long long)b[1] << 32) | a[1]);
    }
    return v;
}

// Called by wave 0: the bin of a 256-bin histogram at which the running
// count reaches `rank` (1 <= rank <= total); pick = {bin, count before it,
// count in it}.  Lane l sums bins 4l .. 4l+3, a wave scan places the lanes
// and the lane whose range crosses the rank walks its four bins.
__device__ __forceinline__ void rank_bin256(const uint32_t* h, uint32_t rank, uint32_t* pick) {
    const int lane = threadIdx.x & 63;
    const u32x4 h4 = *(const u32x4*)(h + 4 * lane);
    const uint32_t tot = (h4[0] + h4[1]) + (h4[2] + h4[3]);
    const uint32_t incl = wave_scan_incl(tot);
    uint32_t bef = incl - tot;
    if (bef < rank && rank <= incl) {
        int b = 0;
        uint32_t cb = h4[0];
        if (bef + cb < rank) { bef += cb; b = 1; cb = h4[1]; }
        if (b == 1 && bef + cb < rank) { bef += cb; b = 2; cb = h4[2]; }
        if (b == 2 && bef + cb < rank) { bef += cb; b = 3; cb = h4[3]; }
        pick[0] = (uint32_t)(4 * lane + b);
        pick[1] = bef;
        pick[2] = cb;
    }
}

constexpr int TK_SLICE_NT = 512;  // threads of a slice workgroup

// atomicAdd(&a[i], 1) for the lanes with `on`, returning each its slot (the
// old value plus its rank): the lanes that share the wave's first active
// index add once, so keys of one score (ties, a dominant value) do not
// serialise on one LDS address.  Lanes outside the branch take no part.
__device__ __forceinline__ uint32_t agg_inc(uint32_t* a, uint32_t i, bool on) {
    const unsigned long long act = __ballot(on);
    if (act == 0ull) return 0u;
    const int lead = __ffsll((long long)act) - 1;
    const uint32_t i0 = (uint32_t)__builtin_amdgcn_readlane((int)i, lead);
    const bool mine = on && i == i0;
    const unsigned long long same = __ballot(mine);
    uint32_t base = 0u;
    if ((int)(threadIdx.x & 63) == lead) base = atomicAdd(&a[i0], (uint32_t)__popcll(same));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, lead);
    if (mine) return base + __builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0u));
    return on ? atomicAdd(&a[i], 1u) : 0u;
}

__global__ void __launch_bounds__(TK_SLICE_NT) topk_spread_slice(TopkParams p) {
    constexpr int NT = TK_SLICE_NT, KPT = TOPK_SPREAD_SLICE / NT, BINS = TOPK_SPREAD_BINS;
    constexpr int SH = 32 - TOPK_SPREAD_BITS;           // image >> SH = first digit
    constexpr int BPT = BINS / NT;                        // digit values per thread
    constexpr int CSTEP = BINS / TOPK_SPREAD_COARSE;      // digit values per coarse bin
    static_assert(BPT % 8 == 0 && CSTEP % BPT == 0 && TOPK_SPREAD_SLICE <= 65535, "offset rows");
    __shared__ __attribute__((aligned(16))) uint32_t hist[BINS];
    __shared__ unsigned long long srt[TOPK_SPREAD_SLICE];
    __shared__ uint32_t scan_sh[NT / 64];
    __shared__ unsigned long long wmin[NT / 64];
    __shared__ int nan_sh;
    static_assert(TOPK_SPREAD_CO % 4 == 0 && TOPK_SPREAD_CO >= TOPK_SPREAD_COARSE + 8, "coarse records");

    const int s = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int S = p.sp_slices;
    const int key0 = s * TOPK_SPREAD_SLICE;
    const float* sr = p.scores + (int64_t)row * p.row_stride;
    const int visible = p.start_pos == 0 ? (row + 1) / p.ratio : p.available;
    const int n = min(p.available - key0, TOPK_SPREAD_SLICE);  // >= 1
    const int64_t slot = (int64_t)row * S + s;

    for (int i = tid; i < BINS / 4; i += NT) ((u32x4*)hist)[i] = u32x4{0u, 0u, 0u, 0u};
    if (tid == 0) nan_sh = 0;
    // key NT j + tid of the slice (coalesced loads) as its 32-bit image
    uint32_t img[KPT];
    bool nan_here = false;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
        const int i = NT * j + tid;
        const float f = i < n ? sr[key0 + i] : 0.f;
        nan_here |= isnan(f);
        img[j] = ~ordered_bits(key0 + i < visible ? f : -INFINITY);
    }
    // NaN anywhere in the row: the columns past the ranked keys, split over the slices
    const int extra = p.cols - p.available;
    if (extra > 0) {
        const int per = (extra + S - 1) / S;
        const int a = p.available + s * per, b = min(a + per, p.cols);
        for (int c = a + tid; c < b; c += NT) nan_here |= isnan(sr[c]);
    }
    __syncthreads();
    if (nan_here) nan_sh = 1;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
        if (NT * j + tid < n) atomicAdd(&hist[img[j] >> SH], 1u);
    __syncthreads();

    // start offset of every digit value (thread t: values BPT t .. BPT t + BPT-1);
    // the counts become the scatter cursors in place
    uint32_t c[BPT], tot = 0;
#pragma unroll
    for (int q = 0; q < BPT / 4; ++q) {
        const u32x4 v = ((const u32x4*)hist)[BPT / 4 * tid + q];
        c[4 * q] = v[0];
        c[4 * q + 1] = v[1];
        c[4 * q + 2] = v[2];
        c[4 * q + 3] = v[3];
        tot += (v[0] + v[1]) + (v[2] + v[3]);
    }
    uint32_t o = block_scan_incl<NT>(tot, scan_sh) - tot;
    uint32_t ov[BPT / 2];
#pragma unroll
    for (int e = 0; e < BPT; ++e) {
        hist[BPT * tid + e] = o;
        if (e & 1)
            ov[e / 2] |= o << 16;
        else
            ov[e / 2] = o;
        o += c[e];
    }
    __syncthreads();
    unsigned long long mn = ~0ull;
#pragma unroll
    for (int j = 0; j < KPT; ++j)
        if (NT * j + tid < n) {
            const uint32_t pos = atomicAdd(&hist[img[j] >> SH], 1u);
            const unsigned long long v = ((unsigned long long)img[j] << 32) | (uint32_t)(key0 + NT * j + tid);
            srt[pos] = v;
            mn = v < mn ? v : mn;
        }
    mn = wave_ext_u64<false>(mn);
    if ((tid & 63) == 0) wmin[tid >> 6] = mn;
    __syncthreads();
    // global stores after the last barrier (a barrier waits for them)
    unsigned short* orow = p.sp_off + slot * TOPK_SPREAD_OFF;
    unsigned short* crow = p.sp_coarse + slot * TOPK_SPREAD_CO;
#pragma unroll
    for (int q = 0; q < BPT / 8; ++q)
        ((u32x4*)orow)[BPT / 8 * tid + q] = u32x4{ov[4 * q], ov[4 * q + 1], ov[4 * q + 2], ov[4 * q + 3]};
    if ((BPT * tid) % CSTEP == 0) crow[BPT * tid / CSTEP] = (unsigned short)(ov[0] & 0xffffu);
    unsigned long long* drow = p.sp_sorted + slot * TOPK_SPREAD_SLICE;
    for (int i = tid; i < n; i += NT) drow[i] = srt[i];
    if (tid == 0) {
        orow[BINS] = (unsigned short)n;
        crow[TOPK_SPREAD_COARSE] = (unsigned short)n;
        crow[TOPK_SPREAD_COARSE + 1] = (unsigned short)nan_sh;
#pragma unroll
        for (int i = 1; i < NT / 64; ++i) mn = wmin[i] < mn ? wmin[i] : mn;
        *(unsigned long long*)(crow + TOPK_SPREAD_COARSE + 4) = mn;  // the slice's smallest composite
    }
}

__global__ void __launch_bounds__(1024) topk_spread_finish(TopkParams p) {
    constexpr int NT = 1024, NW = NT / 64;
    constexpr int CO = TOPK_SPREAD_COARSE;
    constexpr int CSTEP = TOPK_SPREAD_BINS / CO;
    constexpr int FW = CSTEP + 1;        // fine offsets read per slice
    constexpr int CAND = 4096;           // candidates held in LDS
    constexpr int MS = TOPK_SPREAD_MAX_SLICES;
    static_assert(MS <= 128 && CO <= 64 && CSTEP <= 64, "one wave scans the slices and the bins");
    static_assert(TK_BINS == 2 * NT, "two buckets per thread");
    __shared__ uint32_t gco[CO + 1], gfi[FW];
    __shared__ unsigned short fine[MS * FW];
    __shared__ uint32_t pick[3];
    __shared__ __attribute__((aligned(16))) unsigned long long comp[TOPK_MAX];
    __shared__ __attribute__((aligned(16))) unsigned long long aux[CAND];
    __shared__ __attribute__((aligned(16))) uint32_t cnt[TK_BINS], cur[TK_BINS];
    __shared__ __attribute__((aligned(16))) uint32_t dh[2][256];
    __shared__ __attribute__((aligned(16))) uint32_t whist[NW][256];  // a wave's sub-buckets
    __shared__ uint32_t scan_sh[NW];
    __shared__ unsigned long long mn_sh;
    __shared__ uint16_t big[128];  // buckets of TK_BUCKET_MAX+1 .. WAVE_MAX keys
    __shared__ uint32_t nbig;
    __shared__ uint32_t hs[16], hn[16], nhuge;  // fuller buckets: start, keys
    __shared__ uint32_t cpre[MS + 1];
    __shared__ unsigned long long clo_sh, chi_sh;  // smallest and largest candidate
    __shared__ unsigned long long wlo[NW], whi[NW];
    __shared__ int deep;
    __shared__ int nan_sh;
    __shared__ uint32_t ctr;

    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int S = p.sp_slices;
    const uint32_t k = (uint32_t)p.selected;  // 1 <= k <= available
    const int visible = p.start_pos == 0 ? (row + 1) / p.ratio : p.available;
    const int64_t slot0 = (int64_t)row * S;

    if (tid <= CO) gco[tid] = 0;
    if (tid < FW) gfi[tid] = 0;
    if (tid < 256) dh[0][tid] = 0;
    cnt[2 * tid] = 0;
    cnt[2 * tid + 1] = 0;
    if (tid == 0) {
        nan_sh = 0;
        ctr = 0;
        nbig = 0;
        nhuge = 0;
        mn_sh = ~0ull;
        clo_sh = ~0ull;
        chi_sh = 0ull;
    }
    // 1. coarse offsets summed over the slices: the coarse bin holding the
    // k-th key; the row's NaN flag and its smallest composite (each record's
    // first 33 words: 65 offsets and the flag; and its minimum).
    constexpr int CW = (CO + 2) / 2;                  // words of offsets and flag per record
    constexpr int CPT = (MS * CW + NT - 1) / NT;      // of them per thread
    static_assert(TOPK_SPREAD_CO % 4 == 0 && CW * 2 == CO + 2, "coarse records");
    const uint32_t* co32 = (const uint32_t*)(p.sp_coarse + slot0 * TOPK_SPREAD_CO);
    uint32_t cw[CPT];
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
        const int i = tid + NT * e, s = i / CW;
        cw[e] = co32[i < S * CW ? s * (TOPK_SPREAD_CO / 2) + (i - s * CW) : 0];
    }
    const unsigned long long smin =
        *(const unsigned long long*)(p.sp_coarse + (slot0 + (tid < S ? tid : 0)) * TOPK_SPREAD_CO + CO + 4);
    __syncthreads();
#pragma unroll
    for (int e = 0; e < CPT; ++e) {
        const int i = tid + NT * e, s = i / CW, c = 2 * (i - s * CW);  // u16 c and c + 1
        if (i < S * CW) {
            atomicAdd(&gco[c], cw[e] & 0xffffu);
            if (c + 1 <= CO)
                atomicAdd(&gco[c + 1], cw[e] >> 16);
            else if (cw[e] >> 16)
                nan_sh = 1;
        }
    }
    if (tid < S) atomicMin(&mn_sh, smin);
    __syncthreads();
    // every wave finds the coarse bin itself (gco is read-only from here)
    const int c0 = __ffsll((long long)__ballot(lane < CO && gco[lane] < k && k <= gco[lane + 1])) - 1;
    // 2. fine offsets inside it: the cut digit value
    for (int i = tid; i < S * FW; i += NT) {
        const int s = i / FW, j = i - s * FW;
        const uint32_t v = p.sp_off[(slot0 + s) * TOPK_SPREAD_OFF + CSTEP * c0 + j];
        fine[i] = (unsigned short)v;
        atomicAdd(&gfi[j], v);
    }
    __syncthreads();
    const int cb = __ffsll((long long)__ballot(lane < CSTEP && gfi[lane] < k && k <= gfi[lane + 1])) - 1;
    const uint32_t P = gfi[cb], C = gfi[cb + 1] - P;  // keys below the cut value, keys at it
    const uint32_t cut = (uint32_t)(CSTEP * c0 + cb);
    // Usually every key through the cut value fits: all of them are ordered
    // and the first k emitted.  Otherwise the keys below it are gathered and
    // a radix select picks the cut value's taken keys.
    const bool all = P + C <= (uint32_t)TOPK_MAX;
    const bool cand_lds = !all && C <= (uint32_t)CAND;
    // where each slice's keys go: every wave scans the slices itself (slices
    // 2l, 2l+1 on lane l) and reads its own slices' places by readlane
    uint32_t ps0, cs0, pe, ce;
    {
        uint32_t ps[2], cs[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int s = 2 * lane + e;
            const uint32_t lo = s < S ? fine[s * FW + cb] : 0u, hi = s < S ? fine[s * FW + cb + 1] : 0u;
            ps[e] = all ? hi : lo;
            cs[e] = hi - lo;
        }
        const uint32_t pt = ps[0] + ps[1], ct = cs[0] + cs[1];
        pe = wave_scan_incl(pt) - pt;
        ce = wave_scan_incl(ct) - ct;
        ps0 = ps[0];
        cs0 = cs[0];
    }
    // the candidates' flat positions: slice s holds cpre[s] .. cpre[s+1]-1
    // (slices past S hold none, so cpre[S] = C)
    if (w == 0) {
        cpre[2 * lane] = ce;
        cpre[2 * lane + 1] = ce + cs0;
        if (lane == 0) cpre[MS] = C;
    }
    auto place = [&](int s, bool cand) {  // s wave-uniform
        const int l = s >> 1;
        uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)(cand ? ce : pe), l);
        if (s & 1) v += (uint32_t)__builtin_amdgcn_readlane((int)(cand ? cs0 : ps0), l);
        return v;
    };
    // bucket of a key for the final order: (composite - smallest) >> shift,
    // shift the least that fits every key through the cut value into
    // TK_BINS buckets
    const unsigned long long mn = mn_sh;
    const unsigned long long mx = (((unsigned long long)cut + 1ull) << (64 - TOPK_SPREAD_BITS)) - 1ull;
    const unsigned long long span = mx - mn;
    const int shift = max(0, (span ? 64 - __clzll((long long)span) : 0) - 11);  // span >> shift < TK_BINS
    auto bucket = [&](unsigned long long v) { return (uint32_t)((v - mn) >> shift); };
    // 3. gather (wave w: slices w, w + NW, ...; four keys per lane a batch),
    // counting the buckets; the smallest and largest candidate held in LDS
    unsigned long long clo = ~0ull, chi = 0ull;
    auto gather = [&](int s) {
        const uint32_t ps = fine[s * FW + cb], es = fine[s * FW + cb + 1];
        const uint32_t g = (all || cand_lds) ? es : ps;
        const uint32_t dst = place(s, false), dcand = place(s, true);
        const unsigned long long* src = p.sp_sorted + (slot0 + s) * TOPK_SPREAD_SLICE;
        for (uint32_t i0 = 0; i0 < g; i0 += 256) {
            unsigned long long v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t i = i0 + lane + 64 * e;
                v[e] = src[i < g ? i : 0];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t i = i0 + lane + 64 * e;
                if (i < g) {
                    if (all || i < ps) {
                        comp[dst + i] = v[e];
                        atomicAdd(&cnt[bucket(v[e])], 1u);
                    } else {
                        aux[dcand + (i - ps)] = v[e];
                        clo = v[e] < clo ? v[e] : clo;
                        chi = v[e] > chi ? v[e] : chi;
                    }
                }
            }
        }
    };
    for (int s = w; s < S; s += NW) gather(s);
    uint32_t nsort = P + C;
    if (!all) {
        // 4. the (k - P)-th smallest candidate: a radix select, 8-bit digits
        // from the highest bit in which the candidates differ (all share the
        // top TOPK_SPREAD_BITS bits; ties differ only in key id bits).
        // Candidates come from LDS or (too many for it) from the slices'
        // rows, each wave an equal share of the flat candidate range.
        const uint32_t f0 = (uint32_t)((uint64_t)C * w / NW), f1 = (uint32_t)((uint64_t)C * (w + 1) / NW);
        if (cand_lds) {
            clo = wave_ext_u64<false>(clo);
            chi = wave_ext_u64<true>(chi);
            if (lane == 0) {
                atomicMin(&clo_sh, clo);
                atomicMax(&chi_sh, chi);
            }
        }
        __syncthreads();
        int s_first = 0;  // the slice holding flat position f0: the last s with cpre[s] <= f0
        if (!cand_lds) {
            int lo = 0, hi = S - 1;
            while (lo < hi) {
                const int mid = (lo + hi + 1) >> 1;
                if (cpre[mid] <= f0)
                    lo = mid;
                else
                    hi = mid - 1;
            }
            s_first = lo;
        }
        auto for_each_cand = [&](auto&& f) {
            if (cand_lds) {
                for (uint32_t i = tid; i < C; i += NT) f(aux[i]);
            } else {
                uint32_t fp = f0;
                for (int s = s_first; fp < f1; ++s) {  // s < S while fp < f1 <= cpre[S]
                    const uint32_t fe = min(cpre[s + 1], f1);
                    const int64_t adj = (int64_t)fine[s * FW + cb] - (int64_t)cpre[s];  // flat -> row index
                    const unsigned long long* src = p.sp_sorted + (slot0 + s) * TOPK_SPREAD_SLICE;
                    for (uint32_t i0 = fp; i0 < fe; i0 += 512) {  // eight loads in flight per lane
                        unsigned long long v[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const uint32_t i = i0 + lane + 64 * e;
                            v[e] = src[(int64_t)(i < fe ? i : fp) + adj];
                        }
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            if (i0 + lane + 64 * e < fe) f(v[e]);
                    }
                    fp = max(fp, fe);
                }
            }
        };
        if (!cand_lds) {
            for_each_cand([&](unsigned long long v) {
                clo = v < clo ? v : clo;
                chi = v > chi ? v : chi;
            });
            clo = wave_ext_u64<false>(clo);
            chi = wave_ext_u64<true>(chi);
            if (lane == 0) {
                atomicMin(&clo_sh, clo);
                atomicMax(&chi_sh, chi);
            }
            __syncthreads();
        }
        clo = clo_sh;
        chi = chi_sh;
        const uint32_t need = k - P;  // >= 1, < C
        // C >= 2 distinct composites: 1 <= hib <= 64 - TOPK_SPREAD_BITS
        int hib = 64 - __clzll((long long)(clo ^ chi));
        unsigned long long dsel = ~0ull;
        unsigned long long dacc = clo & ~((1ull << hib) - 1ull);
        uint32_t remaining = need;
#pragma unroll 1
        for (int q = 0; q < 8; ++q) {  // each pass fixes up to 8 bits; the last leaves one candidate
            const int sh = max(0, hib - 8), wd = hib - sh;
            uint32_t* h = dh[q & 1];
            if (tid < 256) dh[(q & 1) ^ 1][tid] = 0;  // the next digit's
            for_each_cand([&](unsigned long long v) {
                agg_inc(h, (uint32_t)(v >> sh) & ((1u << wd) - 1u), ((v ^ dacc) >> hib) == 0ull);
            });
            __syncthreads();
            if (tid < 64) rank_bin256(h, remaining, pick);
            __syncthreads();
            dacc |= (unsigned long long)pick[0] << sh;
            remaining -= pick[1];
            if (remaining == pick[2]) {  // every candidate with this prefix is taken
                dsel = dacc | ((1ull << sh) - 1ull);
                break;
            }
            hib = sh;
        }
        // the candidates <= dsel (exactly `need` of them) after the taken keys;
        // their order here is arbitrary, the sort below fixes it
        for_each_cand([&](unsigned long long v) {
            const uint32_t pos = P + agg_inc(&ctr, 0u, v <= dsel);
            const bool take = v <= dsel && pos < k;
            agg_inc(cnt, take ? bucket(v) : 0u, take);
            if (take) comp[pos] = v;
        });
        nsort = k;
    }

    // 5. order the nsort keys by their buckets (counted above: one scan, a
    // scatter, the rank inside the bucket); the first k go out
    int32_t* orow = p.out + (int64_t)row * p.out_stride;
    auto emit = [&](uint32_t i, unsigned long long v) {
        const int key = (int)(uint32_t)v;
        orow[i] = key >= visible ? -1 : p.offset + key;
    };
    __syncthreads();
    // one scan places the buckets; buckets of TK_BUCKET_MAX+1 .. WAVE_MAX
    // keys are listed for a wave's register sort, fuller ones (a value many
    // keys share, few distinct scores) for a second bucket pass over their
    // own span
    constexpr uint32_t WAVE_MAX = 256;  // 64 lanes x 4
    constexpr int HUGE_MAX = TOPK_MAX / (WAVE_MAX + 1);
    static_assert((TOPK_MAX + TK_BUCKET_MAX) / (TK_BUCKET_MAX + 1) <= 128, "listed buckets");
    static_assert(HUGE_MAX <= 16, "full buckets");
    // bucket counts (two per thread) -> their starts in cur, the listings
    // (full buckets only at the first level)
    auto place_buckets = [&](uint32_t b0, uint32_t b1, bool list_full) {
        if (b0 > (uint32_t)TK_BUCKET_MAX && b0 <= WAVE_MAX) big[atomicAdd(&nbig, 1u)] = (uint16_t)(2 * tid);
        if (b1 > (uint32_t)TK_BUCKET_MAX && b1 <= WAVE_MAX) big[atomicAdd(&nbig, 1u)] = (uint16_t)(2 * tid + 1);
        const uint32_t sv = b0 + b1;
        const uint32_t incl = wave_scan_incl(sv);
        if (lane == 63) scan_sh[w] = incl;
        __syncthreads();
        uint32_t before = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) before += i < w ? scan_sh[i] : 0u;
        const uint32_t st = before + incl - sv;
        cur[2 * tid] = st;
        cur[2 * tid + 1] = st + b0;
        if (list_full && b0 > WAVE_MAX) {
            const uint32_t h = atomicAdd(&nhuge, 1u);
            hs[h] = st;
            hn[h] = b0;
        }
        if (list_full && b1 > WAVE_MAX) {
            const uint32_t h = atomicAdd(&nhuge, 1u);
            hs[h] = st + b0;
            hn[h] = b1;
        }
        __syncthreads();
    };
    // rank of every key of a bucket of at most TK_BUCKET_MAX keys (the keys
    // of its bucket below it), then a wave's sort of each listed bucket; the
    // keys were scattered into buf, bucket by bucket, position off onwards
    // A listed bucket (TK_BUCKET_MAX+1 .. WAVE_MAX keys at buf[bstart..]) by
    // one wave: its keys bucketed again into 256 sub-buckets over their own
    // span (a wave's histogram, scanned, the keys scattered to dst at the
    // same positions), each key ranked inside its sub-bucket.  Returns false,
    // with nothing emitted, when a sub-bucket holds more than TK_BUCKET_MAX
    // keys (shared scores); the wave sorts the bucket instead.
    auto sub_sort = [&](const unsigned long long* buf, unsigned long long* dst, uint32_t bstart, uint32_t nb,
                        uint32_t off) -> bool {
        uint32_t* hw = whist[w];
        unsigned long long x[4], lo = ~0ull, hi = 0ull;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t j = lane + 64 * e;
            x[e] = buf[bstart + (j < nb ? j : 0u)];
            if (j < nb) {
                lo = x[e] < lo ? x[e] : lo;
                hi = x[e] > hi ? x[e] : hi;
            }
        }
        lo = wave_ext_u64<false>(lo);
        hi = wave_ext_u64<true>(hi);
        const unsigned long long span = hi - lo;
        const int sh = max(0, (span ? 64 - __clzll((long long)span) : 0) - 8);
        uint32_t sb[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) sb[e] = (uint32_t)((x[e] - lo) >> sh) & 255u;
        *(u32x4*)(hw + 4 * lane) = u32x4{0u, 0u, 0u, 0u};
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (lane + 64 * e < (int)nb) atomicAdd(&hw[sb[e]], 1u);
        __builtin_amdgcn_wave_barrier();
        const u32x4 c4 = *(const u32x4*)(hw + 4 * lane);
        const uint32_t tot = (c4[0] + c4[1]) + (c4[2] + c4[3]);
        const uint32_t cmax = max(max(c4[0], c4[1]), max(c4[2], c4[3]));
        if (__ballot(cmax > (uint32_t)TK_BUCKET_MAX) != 0ull) return false;
        const uint32_t ex = wave_scan_incl(tot) - tot;
        // sub-bucket starts, which the scatter advances to their ends
        *(u32x4*)(hw + 4 * lane) = u32x4{ex, ex + c4[0], ex + c4[0] + c4[1], ex + c4[0] + c4[1] + c4[2]};
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (lane + 64 * e < (int)nb) dst[bstart + atomicAdd(&hw[sb[e]], 1u)] = x[e];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (lane + 64 * e >= (int)nb) continue;
            const uint32_t se = hw[sb[e]], ss = sb[e] ? hw[sb[e] - 1] : 0u;  // [start, end) of its sub-bucket
            uint32_t r = ss;
            for (uint32_t j = ss; j < se; ++j) r += dst[bstart + j] < x[e];
            if (off + bstart + r < k) emit(off + bstart + r, x[e]);
        }
        return true;
    };
    auto order_buckets = [&](unsigned long long* buf, unsigned long long* dst, uint32_t n, uint32_t off,
                             auto&& bkt) {
        unsigned long long kv[4];
        uint32_t kend[4], kstart[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            kv[e] = buf[min(tid + NT * e, TOPK_MAX - 1)];
            const uint32_t b = bkt(kv[e]) & (TK_BINS - 1);
            kend[e] = cur[b];
            kstart[e] = kend[e] - cnt[b];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (tid + NT * e >= (int)n || kend[e] - kstart[e] > (uint32_t)TK_BUCKET_MAX) continue;
            const unsigned long long v = kv[e];
            uint32_t r = off + kstart[e];
            for (uint32_t j0 = kstart[e]; j0 < kend[e]; j0 += 4) {
                unsigned long long u[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) u[q] = j0 + q < kend[e] ? buf[j0 + q] : ~0ull;
#pragma unroll
                for (int q = 0; q < 4; ++q) r += u[q] < v;
            }
            if (r < k) emit(r, v);
        }
        auto sort_bucket = [&](uint32_t b, auto ept_tag) {  // 64 EPT >= the bucket's keys
            constexpr int EPT = decltype(ept_tag)::value;
            const uint32_t bend = cur[b], nb = cnt[b], bstart = bend - nb;
            unsigned long long x[EPT];
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                const uint32_t j = EPT * lane + e;
                x[e] = j < nb ? buf[bstart + j] : TK_NONE;
            }
            wave_sort<EPT>(x, 64 * EPT);
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                const uint32_t j = EPT * lane + e;
                if (j < nb && off + bstart + j < k) emit(off + bstart + j, x[e]);
            }
        };
        for (uint32_t i = w; i < nbig; i += NW) {
            const uint32_t b = big[i], nb = cnt[b];
            if (sub_sort(buf, dst, cur[b] - nb, nb, off)) continue;
            if (nb <= 128)
                sort_bucket(b, std::integral_constant<int, 2>{});
            else
                sort_bucket(b, std::integral_constant<int, 4>{});
        }
    };
    __syncthreads();
    place_buckets(cnt[2 * tid], cnt[2 * tid + 1], true);
    static_assert(TOPK_MAX <= 4 * NT, "four keys per thread");
    {
        unsigned long long kv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) kv[e] = comp[min(tid + NT * e, TOPK_MAX - 1)];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (tid + NT * e < (int)nsort) aux[atomicAdd(&cur[bucket(kv[e])], 1u)] = kv[e];
    }
    __syncthreads();
    // cur[b] is now the end of bucket b
    order_buckets(aux, comp, nsort, 0u, bucket);
    // each full bucket in turn, by the whole workgroup: its keys bucketed
    // again over the span from its smallest to its largest composite (keys
    // of one score differ in the key id only, so they spread)
    const uint32_t nh = nhuge;
    for (uint32_t h = 0; h < nh; ++h) {
        const uint32_t hst = hs[h], hnb = hn[h];
        if (hst >= k) continue;  // nothing of it is emitted
        __syncthreads();  // the last pass's readers of cnt, cur, comp, big are done
        unsigned long long x[4], lo = ~0ull, hi = 0ull;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t i = tid + NT * e;
            x[e] = i < hnb ? aux[hst + i] : TK_NONE;
            if (i < hnb) {
                lo = x[e] < lo ? x[e] : lo;
                hi = x[e] > hi ? x[e] : hi;
            }
        }
        lo = wave_ext_u64<false>(lo);
        hi = wave_ext_u64<true>(hi);
        if (lane == 0) {
            wlo[w] = lo;
            whi[w] = hi;
        }
        cnt[2 * tid] = 0;
        cnt[2 * tid + 1] = 0;
        if (tid == 0) {
            nbig = 0;
            deep = 0;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            lo = wlo[i] < lo ? wlo[i] : lo;
            hi = whi[i] > hi ? whi[i] : hi;
        }
        const unsigned long long hspan = hi - lo;
        const int hshift = max(0, (hspan ? 64 - __clzll((long long)hspan) : 0) - 11);
        auto sub = [&](unsigned long long v) { return (uint32_t)((v - lo) >> hshift); };
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (tid + NT * e < (int)hnb) atomicAdd(&cnt[sub(x[e])], 1u);
        __syncthreads();
        const uint32_t c0 = cnt[2 * tid], c1 = cnt[2 * tid + 1];
        if (c0 > WAVE_MAX || c1 > WAVE_MAX) deep = 1;
        place_buckets(c0, c1, false);
        if (!deep) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (tid + NT * e < (int)hnb) comp[atomicAdd(&cur[sub(x[e])], 1u)] = x[e];
            __syncthreads();
            order_buckets(comp, aux + hst, hnb, hst, sub);
        } else {
            // a sub-bucket still too full (several shared scores in one
            // bucket): the bitonic sort of this bucket's keys
            int npow = 4;
            while (npow < (int)hnb) npow <<= 1;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (tid + NT * e < npow) comp[tid + NT * e] = x[e];
            __syncthreads();
            auto sort_emit = [&](auto ept_tag) {
                constexpr int EPT = decltype(ept_tag)::value;
                unsigned long long y[EPT];
                sort_lds<NT, EPT>(comp, npow, y);
#pragma unroll
                for (int e = 0; e < EPT; ++e) {
                    const uint32_t j = EPT * tid + e;
                    if (j < hnb && hst + j < k) emit(hst + j, y[e]);
                }
            };
            if (npow <= 2 * NT)
                sort_emit(std::integral_constant<int, 2>{});
            else
                sort_emit(std::integral_constant<int, 4>{});
        }
    }
    if (tid == 0) {
        p.nan_flags[row] = nan_sh;
        if (p.status_direct) *p.status_direct = nan_sh ? 5 /* MR_NONFINITE */ : 0;
    }
}

// One merge round over rows of sorted composite lists: list pair q of a row
// (lists 2q and 2q+1 of `lists`, each `len` long; an odd last list passes
// through) -> the first len_out = min(2 len, selected) of their merge (~0
// past an odd list's end).  Output position i takes its split from a
// merge-path binary search over global memory (the lists are short and
// cached).  The last round (one pair left) writes the keys instead, offset
// + key or -1 past `visible`, and the row's NaN flag.
__global__ void __launch_bounds__(256) topk_merge_kernel(TopkParams p, const unsigned long long* in, int lists, int len,
                                                          unsigned long long* outc) {
    const int row = blockIdx.y;
    const int q = blockIdx.x;
    const int len_out = (int)min((int64_t)2 * len, (int64_t)p.selected);
    const unsigned long long* A = in + ((int64_t)row * lists + 2 * q) * len;
    const bool pair = 2 * q + 1 < lists;
    const unsigned long long* B = A + len;
    const int nout = (lists + 1) / 2;
    const bool last = nout == 1;
    const int visible = p.start_pos == 0 ? (row + 1) / p.ratio : p.available;
    for (int i = threadIdx.x; i < len_out; i += 256) {
        unsigned long long v;
        if (pair) {
            // a = number of the first i + 1 outputs taken from A
            int lo = max(0, i + 1 - len), hi = min(i + 1, len);
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (A[mid] < B[i - mid])
                    lo = mid + 1;
                else
                    hi = mid;
            }
            // output i is the larger of A[lo - 1] and B[i - lo] (the last taken)
            const unsigned long long a = lo > 0 ? A[lo - 1] : 0ull;
            const unsigned long long b = i - lo >= 0 ? B[i - lo] : 0ull;
            v = lo == 0 ? b : (i - lo < 0 ? a : (a > b ? a : b));
        } else {
            v = i < len ? A[i] : TK_NONE;
        }
        if (last) {
            const int key = (int)(uint32_t)(v & 0xffffffffull);
            p.out[(int64_t)row * p.out_stride + i] = key >= visible ? -1 : p.offset + key;
        } else {
            outc[((int64_t)row * nout + q) * len_out + i] = v;
        }
    }
    if (last && threadIdx.x == 0) {
        int f = 0;
        for (int sl = 0; sl < p.slices; ++sl) f |= p.slice_nan[row * p.slices + sl];
        p.nan_flags[row] = f;
        if (p.status_direct) *p.status_direct = f ? 5 /* MR_NONFINITE */ : 0;
    }
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

namespace {

size_t a256(size_t x) { return (x + 255) & ~size_t(255); }

// Rows of more keys than this (and few rows) take the spread selection.
constexpr int TOPK_SPREAD_MIN_KEYS = 1024;

bool spread_applies(int32_t rows, int32_t keys) {
    return rows <= TOPK_SPREAD_MAX_ROWS && keys > TOPK_SPREAD_MIN_KEYS &&
           keys <= TOPK_SPREAD_MAX_SLICES * TOPK_SPREAD_SLICE;
}

// Byte offsets of the spread selection's arrays, after the per-row flags.
struct SpreadLayout {
    size_t coarse, off, sorted, end;
};
SpreadLayout spread_layout(int32_t rows, int slices) {
    const size_t rs = size_t(rows) * size_t(slices);
    SpreadLayout L;
    L.coarse = 0;
    L.off = L.coarse + a256(rs * TOPK_SPREAD_CO * 2);
    L.sorted = L.off + a256(rs * TOPK_SPREAD_OFF * 2);
    L.end = L.sorted + a256(rs * TOPK_SPREAD_SLICE * 8);
    return L;
}

// Keys per slice workgroup when more than TOPK_MAX keys are selected: a
// slice sorts all of its keys (at most TOPK_MAX), and the merge rounds
// double the lists' length up to `selected`.
constexpr int TOPK_LARGE_SLICE = TOPK_MAX;

// Bytes of one of the two composite buffers of the merge rounds: the largest
// rows x lists x length over the rounds.
size_t merge_buffer_bytes(int32_t rows, int64_t slices, int64_t len, int64_t selected) {
    size_t most = 0;
    for (int64_t lists = slices;; lists = (lists + 1) / 2, len = std::min(2 * len, selected)) {
        most = std::max(most, size_t(rows) * size_t(lists) * size_t(len) * 8);
        if (lists <= 1) break;
    }
    return a256(most);
}

size_t small_k_bytes(int32_t rows, int32_t cols, int32_t selected) {
    size_t extra = 0;
    if (cols > TOPK_SLICE) {
        const size_t slices = (size_t(cols) + TOPK_SLICE - 1) / TOPK_SLICE;
        extra = a256(size_t(rows) * slices * 4);
        extra += 2 * merge_buffer_bytes(rows, (int64_t)slices, selected, selected);
    }
    if (rows <= TOPK_SPREAD_MAX_ROWS && cols > TOPK_SPREAD_MIN_KEYS) {
        // the ranked keys never exceed the columns
        const int slices = (int)std::min<int64_t>((int64_t(cols) + TOPK_SPREAD_SLICE - 1) / TOPK_SPREAD_SLICE,
                                                  TOPK_SPREAD_MAX_SLICES);
        extra = std::max(extra, spread_layout(rows, slices).end);
    }
    return extra;
}

}  // namespace

size_t topk_workspace_bytes(int32_t rows, int32_t cols, int32_t selected) {
    size_t bytes = a256(size_t(rows) * 4);
    if (selected <= TOPK_MAX) return bytes + small_k_bytes(rows, cols, selected);
    // more than TOPK_MAX keys: slices of TOPK_LARGE_SLICE and merge rounds;
    // a call whose rows turn out to select fewer takes the paths above
    const int64_t slices = (int64_t(cols) + TOPK_LARGE_SLICE - 1) / TOPK_LARGE_SLICE;
    const size_t large = a256(size_t(rows) * size_t(slices) * 4) +
                         2 * merge_buffer_bytes(rows, slices, TOPK_LARGE_SLICE, selected);
    return bytes + std::max(large, small_k_bytes(rows, cols, TOPK_MAX));
}

namespace {

// The pairwise merge rounds over `slices` sorted lists of `len` composites
// per row in buf[0], down to the keys.
hipError_t merge_rounds(const TopkParams& p, unsigned long long* const* buf, int slices, int len, hipStream_t st) {
    int lists = slices, cur = 0;
    while (lists > 1) {
        const int nout = (lists + 1) / 2;
        hipLaunchKernelGGL(topk_merge_kernel, dim3((unsigned)nout, (unsigned)p.rows), dim3(256), 0, st, p,
                           (const unsigned long long*)buf[cur], lists, len, buf[cur ^ 1]);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        lists = nout;
        len = (int)std::min<int64_t>(2 * (int64_t)len, p.selected);
        cur ^= 1;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_topk_select(const TopkParams& p0, void* workspace, int32_t* status, hipStream_t st) {
    TopkParams p = p0;
    p.slices = 1;
    p.list_len = p.selected;
    // a single row's status comes from the kernel that flags its NaN (the
    // selection, or the last merge round), not from a launch of its own
    p.status_direct = p.rows == 1 ? status : nullptr;
    if (p.selected > TOPK_MAX) {
        // more keys than one workgroup orders: every slice of
        // TOPK_LARGE_SLICE keys sorts all of its keys, and the merge rounds
        // keep the first `selected` of each merge
        char* ws = (char*)workspace + a256(size_t(p.rows) * 4);
        const int slices = (p.available + TOPK_LARGE_SLICE - 1) / TOPK_LARGE_SLICE;
        const int64_t max_slices = (int64_t(p.cols) + TOPK_LARGE_SLICE - 1) / TOPK_LARGE_SLICE;
        p.slices = slices;
        p.list_len = TOPK_LARGE_SLICE;
        p.slice_nan = (int32_t*)ws;
        ws += a256(size_t(p.rows) * size_t(max_slices) * 4);
        unsigned long long* buf[2] = {
            (unsigned long long*)ws,
            (unsigned long long*)(ws + merge_buffer_bytes(p.rows, max_slices, TOPK_LARGE_SLICE, p.selected))};
        p.cand = buf[0];
        static_assert(1024 * 4 == TOPK_LARGE_SLICE, "one key per register of a 1024 x 4 slice");
        hipLaunchKernelGGL((topk_select_kernel<1024, 4>), dim3((unsigned)p.rows, (unsigned)slices), dim3(1024), 0, st, p);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = merge_rounds(p, buf, slices, TOPK_LARGE_SLICE, st);
        if (e != hipSuccess) return e;
    } else if (spread_applies(p.rows, p.available)) {
        // a few rows of many keys: each row over many workgroups
        const int slices = (p.available + TOPK_SPREAD_SLICE - 1) / TOPK_SPREAD_SLICE;
        char* ws = (char*)workspace + a256(size_t(p.rows) * 4);
        const SpreadLayout L = spread_layout(p.rows, slices);
        p.sp_slices = slices;
        p.sp_coarse = (unsigned short*)(ws + L.coarse);
        p.sp_off = (unsigned short*)(ws + L.off);
        p.sp_sorted = (unsigned long long*)(ws + L.sorted);
        hipLaunchKernelGGL(topk_spread_slice, dim3((unsigned)slices, (unsigned)p.rows), dim3(TK_SLICE_NT), 0, st, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(topk_spread_finish, dim3((unsigned)p.rows), dim3(1024), 0, st, p);
    } else if (p.available <= 256 * 4) {
        // keys per thread: the row's ranked keys in registers
        hipLaunchKernelGGL((topk_select_kernel<256, 4>), dim3((unsigned)p.rows), dim3(256), 0, st, p);
    } else if (p.available <= 1024 * 16) {
        hipLaunchKernelGGL((topk_select_kernel<1024, 16>), dim3((unsigned)p.rows), dim3(1024), 0, st, p);
    } else if (p.available <= TOPK_SLICE) {
        hipLaunchKernelGGL((topk_select_kernel<1024, 32>), dim3((unsigned)p.rows), dim3(1024), 0, st, p);
    } else {
        // slices of 32768 keys in parallel, then pairwise merge rounds
        char* ws = (char*)workspace + a256(size_t(p.rows) * 4);
        const int slices = (p.available + TOPK_SLICE - 1) / TOPK_SLICE;
        const int max_slices = (p.cols + TOPK_SLICE - 1) / TOPK_SLICE;
        p.slices = slices;
        p.slice_nan = (int32_t*)ws;
        ws += a256(size_t(p.rows) * max_slices * 4);
        unsigned long long* buf[2] = {
            (unsigned long long*)ws,
            (unsigned long long*)(ws + merge_buffer_bytes(p.rows, max_slices, p.selected, p.selected))};
        p.cand = buf[0];
        hipLaunchKernelGGL((topk_select_kernel<1024, 32>), dim3((unsigned)p.rows, (unsigned)slices), dim3(1024), 0, st, p);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = merge_rounds(p, buf, slices, p.selected, st);
        if (e != hipSuccess) return e;
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && status && !p.status_direct) {
        hipLaunchKernelGGL(topk_status_kernel, dim3(1), dim3(256), 0, st, p.nan_flags, p.rows, status);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace mr
