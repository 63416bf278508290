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
// Rows of more than 32768 keys split into slices of 32768, one workgroup
// each (the same kernel, in parallel), which emit their own first
// `selected` keys as sorted 64-bit composites (image << 32 | key); merge
// rounds (topk_merge_kernel) then take the first `selected` of the merge of
// two sorted lists, each output position finding its split by a merge-path
// binary search, until one list is left; the last round writes the keys.
// The order is the same total order, so the result is the same.
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
// Rows ranked by 1024 threads take the compacted path when the first digit's
// cut bin holds at most TK_CAND keys: the keys above the cut go straight to
// the selected list and only the cut bin's keys take the remaining digits.
constexpr int TK_CAND = 4096;
// Bucket order of the selected keys: buckets over the span of their score
// images; a bucket of more than TK_BUCKET_MAX keys (ties, a few distinct
// scores) sends the row to the bitonic sort instead.
constexpr int TK_BUCKET_MAX = 32;

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

    // 3. sort, ascending.  Thread t holds elements EPT t .. EPT t + EPT-1 in
    // registers (EPT = 2 when the padded count fits 2 per thread, so every
    // wave works; else 4).  Each wave sorts its 64 EPT elements (a bitonic
    // network whose lane exchanges have constant distances), then runs of
    // 64 EPT, 128 EPT, ... merge pairwise through LDS: each output position
    // finds its split by a merge-path binary search (the composites are
    // distinct).  The sorted keys go out as offsets (or, per slice, as 64-bit
    // composites for the merge rounds).
    const int lane = tid & 63;
    auto sort_and_emit = [&](auto ept_tag) {
        constexpr int EPT = decltype(ept_tag)::value;
        const bool act = EPT * tid < npow;
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
        const int wsize = min(npow, 64 * EPT);  // elements each wave sorts
#pragma unroll 1
        for (int size = 2; size <= wsize; size <<= 1) {
            const bool all_up = size == wsize;
#pragma unroll 1
            for (int d = size >> 1; d >= EPT; d >>= 1) lane_stage_d(d / EPT, size, all_up);
            thread_stages(size, all_up);
        }
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

        if (p.slices > 1) {  // this slice's sorted composites, ~0 past its keys
            unsigned long long* crow = p.cand + ((int64_t)row * p.slices + slice) * p.selected;
#pragma unroll
            for (int e = 0; e < EPT; ++e) {
                const int i = EPT * tid + e;
                if (i < p.selected)
                    crow[i] = i < k ? ((x[e] >> 16) << 32) | (uint32_t)(key0 + (int)(uint32_t)(x[e] & 0xffffull)) : TK_NONE;
            }
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
            unsigned long long* crow = p.cand + ((int64_t)row * p.slices + slice) * p.selected;
            for (int i = tid; i < p.selected; i += NT)
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

// One merge round over rows of sorted composite lists: list pair q of a row
// (lists 2q and 2q+1 of `lists`, each `len` long; an odd last list passes
// through) -> the first `len` of their merge.  Output position i takes its
// split from a merge-path binary search over global memory (the lists are
// short and cached).  The last round (one pair left) writes the keys
// instead, offset + key or -1 past `visible`, and the row's NaN flag.
__global__ void __launch_bounds__(256) topk_merge_kernel(TopkParams p, const unsigned long long* in, int lists,
                                                          unsigned long long* outc) {
    const int row = blockIdx.y;
    const int q = blockIdx.x;
    const int len = p.selected;
    const unsigned long long* A = in + ((int64_t)row * lists + 2 * q) * len;
    const bool pair = 2 * q + 1 < lists;
    const unsigned long long* B = A + len;
    const int nout = (lists + 1) / 2;
    const bool last = nout == 1;
    const int visible = p.start_pos == 0 ? (row + 1) / p.ratio : p.available;
    for (int i = threadIdx.x; i < len; i += 256) {
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
            v = A[i];
        }
        if (last) {
            const int key = (int)(uint32_t)(v & 0xffffffffull);
            p.out[(int64_t)row * p.out_stride + i] = key >= visible ? -1 : p.offset + key;
        } else {
            outc[((int64_t)row * nout + q) * len + i] = v;
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

size_t topk_workspace_bytes(int32_t rows, int32_t cols, int32_t selected) {
    auto a256 = [](size_t x) { return (x + 255) & ~size_t(255); };
    size_t bytes = a256(size_t(rows) * 4);
    if (cols > TOPK_SLICE) {
        const size_t slices = (size_t(cols) + TOPK_SLICE - 1) / TOPK_SLICE;
        bytes += a256(size_t(rows) * slices * 4);
        bytes += 2 * a256(size_t(rows) * slices * size_t(selected) * 8);
    }
    return bytes;
}

hipError_t launch_topk_select(const TopkParams& p0, void* workspace, int32_t* status, hipStream_t st) {
    TopkParams p = p0;
    p.slices = 1;
    // a single row's status comes from the kernel that flags its NaN (the
    // selection, or the last merge round), not from a launch of its own
    p.status_direct = p.rows == 1 ? status : nullptr;
    // keys per thread: the row's ranked keys in registers
    if (p.available <= 256 * 4) {
        hipLaunchKernelGGL((topk_select_kernel<256, 4>), dim3((unsigned)p.rows), dim3(256), 0, st, p);
    } else if (p.available <= 1024 * 16) {
        hipLaunchKernelGGL((topk_select_kernel<1024, 16>), dim3((unsigned)p.rows), dim3(1024), 0, st, p);
    } else if (p.available <= TOPK_SLICE) {
        hipLaunchKernelGGL((topk_select_kernel<1024, 32>), dim3((unsigned)p.rows), dim3(1024), 0, st, p);
    } else {
        // slices of 32768 keys in parallel, then pairwise merge rounds
        auto a256 = [](size_t x) { return (x + 255) & ~size_t(255); };
        char* ws = (char*)workspace + a256(size_t(p.rows) * 4);
        const int slices = (p.available + TOPK_SLICE - 1) / TOPK_SLICE;
        const int max_slices = (p.cols + TOPK_SLICE - 1) / TOPK_SLICE;
        p.slices = slices;
        p.slice_nan = (int32_t*)ws;
        ws += a256(size_t(p.rows) * max_slices * 4);
        unsigned long long* buf[2] = {(unsigned long long*)ws,
                                      (unsigned long long*)(ws + a256(size_t(p.rows) * max_slices * size_t(p.selected) * 8))};
        p.cand = buf[0];
        hipLaunchKernelGGL((topk_select_kernel<1024, 32>), dim3((unsigned)p.rows, (unsigned)slices), dim3(1024), 0, st, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        int lists = slices, cur = 0;
        while (lists > 1) {
            const int nout = (lists + 1) / 2;
            hipLaunchKernelGGL(topk_merge_kernel, dim3((unsigned)nout, (unsigned)p.rows), dim3(256), 0, st, p,
                               (const unsigned long long*)buf[cur], lists, buf[cur ^ 1]);
            if ((e = hipGetLastError()) != hipSuccess) return e;
            lists = nout;
            cur ^= 1;
        }
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && status && !p.status_direct) {
        hipLaunchKernelGGL(topk_status_kernel, dim3(1), dim3(256), 0, st, p.nan_flags, p.rows, status);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace mr
