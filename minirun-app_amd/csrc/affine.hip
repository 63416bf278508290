// MLX affine quantized weights on gfx950: dequantize and fused dequant-GEMV.
//
// Operand contract (MLXBridge/AffineWeights.swift:65-157): packed uint32
// [O, in*bits/32], element j of a word at bit offset bits*j (element 0 in the
// low bits, MXFP4Weights.swift:42-48); scales and biases [O, in/group] in
// bf16 / f16 / f32; w = scale * q + bias (AffineWeights.swift:320-342).
//
// GEMV fast path (bits 4, bf16 activations), per row o and group g:
//   y_o += s_og * sum_{i in g} x_i q_oi + b_og * sum_{i in g} x_i
// The inner sum runs on v_dot2c_f32_bf16: nibbles j and j+4 of a word become
// the bf16 pair (128 + q_j, 128 + q_j+4) with one shift and one and-or (the
// bf16 ulp at 128 is 1, so the pair is exact), dotted with the x pair
// (x_j, x_j+4) staged in LDS in that order; the 128 * sum(x) offset is folded
// into the bias term.  Products are exact in fp32, accumulation is fp32.
#include <algorithm>
#include <type_traits>

#include "capi_util.hpp"
#include "mr_kernels.hpp"

// Products and sums below round exactly as written: hipcc contracts a*b+c
// into one FMA by default, which changes dequantized weights whenever the
// product is inexact (f32 scales).  FMAs are spelled fmaf where intended.
#pragma clang fp contract(off)

namespace mr {

namespace {

template <int SDT>
__device__ __forceinline__ float load_scale(const void* p, int64_t i) {
    if (SDT == 0) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    if (SDT == 1) return f16_bits_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

__device__ __forceinline__ float load_act(const void* p, int x_f32, int64_t i) {
    return x_f32 ? ((const float*)p)[i] : bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

// ---------------------------------------------------------------- dequantize
// One thread per packed word; w = scale*q + bias as two float roundings.
template <int SDT>
__global__ void __launch_bounds__(256) affine_dequant_kernel(AffineDequantParams p) {
    const int per = 32 / p.bits;
    const uint32_t mask = p.bits == 32 ? 0xffffffffu : ((1u << p.bits) - 1u);
    const int64_t words_per_row = p.in_features / per;
    const int64_t total = p.out_features * words_per_row;
    const int64_t groups = p.in_features / p.group;
    for (int64_t wi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; wi < total; wi += (int64_t)gridDim.x * blockDim.x) {
        const int64_t o = wi / words_per_row;
        const int64_t k = wi - o * words_per_row;
        const uint32_t word = p.packed[wi];
        for (int j = 0; j < per; ++j) {
            const int64_t i = k * per + j;
            const int64_t gi = o * groups + i / p.group;
            const float s = load_scale<SDT>(p.scales, gi);
            const float b = load_scale<SDT>(p.biases, gi);
            const float q = (float)((word >> (p.bits * j)) & mask);
            const float v = add_rn(mul_rn(s, q), b);
            const int64_t oi = o * p.in_features + i;
            if (p.out_f32)
                ((float*)p.out)[oi] = v;
            else
                ((uint16_t*)p.out)[oi] = f32_to_bf16_bits(v);
        }
    }
}

// ---------------------------------------------------------------- GEMV, 4-bit fast path
// A workgroup owns a tile of tile_rows output rows of one activation vector
// (a tile never crosses a map_a boundary; output row j reads weight row
// (j / A) * B + C + (j % A) and activation vector j / A: a plain GEMV is
// A = O, B = 0, C = 0, the per-head W_UV product A = 128, B = 256, C = 128).
// It stages that vector once in LDS, one 16-byte chunk per thread and
// pass: the pair words (x_j | x_j+4 << 16) of every packed word and the
// per-group sums (eight chunk sums per group, combined by lane exchange).
// With norm_w set, the staged vector is bf16(w * (x * rsqrt(mean(x^2) +
// eps))), the RMSNorm stage's output.  tpr threads (a power of two <= 64)
// share an output row, each dotting groups lane, lane + tpr, ...; a step of
// the 256-thread workgroup covers 256 / tpr rows, and while one step is
// dotted the next two steps' weights are in flight.  Every load goes through
// a buffer descriptor, so rows past the tile and groups past the row take an
// out-of-buffer offset: they read zeros without a memory request or a branch.
// NT = 512 threads (two waves per SIMD on one staged vector, each thread
// dotting at most two groups of a row); a row of more than 64 threads sums
// its waves' parts through LDS.
constexpr int GEMV_NT = 512;
constexpr int GEMV_MAX_IN = 16384;  // activation length staged per vector
constexpr int GEMV_NPT_MAX = 2;  // groups per thread and row: tpr * GEMV_NPT >= G

template <int SDT, int GEMV_NPT, int NT>
__global__ void __launch_bounds__(NT)
    affine_gemv4_kernel(AffineGemvParams p0, uint32_t wbytes0, uint32_t sbytes0, AffineGemvParams p1, uint32_t wbytes1,
                        uint32_t sbytes1, int tiles0) {
    // two weights of one activation vector in one launch: workgroups from
    // tiles0 on take the second parameter set (tiles0 = gridDim.x: one set)
    const bool second = (int)blockIdx.x >= tiles0;
    const AffineGemvParams& p = second ? p1 : p0;
    const uint32_t wbytes = second ? wbytes1 : wbytes0, sbytes = second ? sbytes1 : sbytes0;
    // (x_j, x_j+4) pairs, 16 bytes per packed word; a group's 128 bytes are
    // followed by 16 bytes of padding, so lanes reading consecutive groups
    // start on different banks
    __shared__ __attribute__((aligned(16))) uint32_t xp[GEMV_MAX_IN / 2 + GEMV_MAX_IN / 16];
    __shared__ float xs[GEMV_MAX_IN / 64];                              // per-group sums of the staged x
    constexpr int GEMV_THREADS = NT;
    constexpr int GEMV_MAX_CH = GEMV_MAX_IN / 8 / NT;
    __shared__ float red[NT / 64];
    __shared__ float part[2][NT / 64];  // rows of more than one wave: the waves' sums, by step parity
    const int tile = (int)blockIdx.x - (second ? tiles0 : 0);
    const int xg = tile / p.tiles_per_vec;  // activation vector of this tile
    const int r0 = xg * p.map_a + (tile - xg * p.tiles_per_vec) * p.tile_rows;
    const int r_end = min(r0 + p.tile_rows, min((xg + 1) * p.map_a, p.out_rows));
    const int in = p.in_features;
    const int nch = in / 8;  // 16-byte chunks of x
    const int G = in / 64;
    const int t = threadIdx.x;
    const uint16_t* x = (const uint16_t*)p.x + (int64_t)(xg / p.x_div) * p.x_stride;

    // rows: tpr threads per row, steps of 256 / tpr rows; a thread dots at
    // most GEMV_NPT groups of a row (tpr * GEMV_NPT >= G)
    const int tpr = p.tpr;
    const int rps = GEMV_THREADS / tpr;
    const int tr = t / tpr, tl = t - tr * tpr;
    typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
    // weight, scale and bias rows through buffer descriptors: 32-bit offsets,
    // and a load whose offset is past the buffer returns 0 without a memory
    // request (rows past the tile and groups past the row point there)
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc((void*)p.packed, 0, (int)wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc((void*)p.scales, 0, (int)sbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc((void*)p.biases, 0, (int)sbytes, 0x00020000);
    constexpr uint32_t SB = SDT == 2 ? 4 : 2;
    constexpr uint32_t OOB = 0x80000000u;
    // a tile stays inside one activation vector, so output row j reads weight
    // row wbase + j
    // (routed: the expert's rows; an expert id out of range loads nothing)
    int64_t wfirst = xg * p.map_b + p.map_c;
    bool evalid = true;
    if (p.rhs_idx) {
        const int32_t e = p.rhs_idx[xg];
        evalid = e >= 0 && e < p.experts;
        wfirst = evalid ? (int64_t)e * p.map_a : 0;
    }
    const int wbase = (int)wfirst - xg * p.map_a;
    typedef typename std::conditional<SB == 2, uint16_t, uint32_t>::type SRaw;
    struct RowLoads {
        u32x4 w[GEMV_NPT][2];
        SRaw s[GEMV_NPT], b[GEMV_NPT];  // raw scale / bias words, converted at use
        uint32_t ok;  // bit q: group q of this thread is a real (row, group)
    };
    // byte offsets of this thread's groups inside a weight row / scale row
    uint32_t woq[GEMV_NPT], soq[GEMV_NPT];
    bool gq[GEMV_NPT];
#pragma unroll
    for (int q = 0; q < GEMV_NPT; ++q) {
        const int g = tl + tpr * q;
        gq[q] = g < G;
        woq[q] = 32u * (uint32_t)g;
        soq[q] = SB * (uint32_t)g;
    }
    const uint32_t wrow_bytes = (uint32_t)(in / 2), srow_bytes = (uint32_t)G * SB;
    auto load_row = [&](int j, RowLoads& L) {
        const bool rok = j < r_end && evalid;
        const uint32_t wr = (uint32_t)(wbase + j);  // < 2^24 (host check)
        const uint32_t wrow = __umul24(wr, wrow_bytes), srow = __umul24(wr, srow_bytes);
        L.ok = 0;
#pragma unroll
        for (int q = 0; q < GEMV_NPT; ++q) {
            const bool ok = rok && gq[q];
            L.ok |= ok ? (1u << q) : 0u;
            const uint32_t wo = ok ? wrow + woq[q] : OOB;
            const uint32_t so = ok ? srow + soq[q] : OOB;
            L.w[q][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, wo, 0, 0));
            L.w[q][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wres, wo + 16, 0, 0));
            if (SB == 2) {
                L.s[q] = __builtin_amdgcn_raw_buffer_load_b16(sres, so, 0, 0);
                L.b[q] = __builtin_amdgcn_raw_buffer_load_b16(bres, so, 0, 0);
            } else {
                L.s[q] = __builtin_amdgcn_raw_buffer_load_b32(sres, so, 0, 0);
                L.b[q] = __builtin_amdgcn_raw_buffer_load_b32(bres, so, 0, 0);
            }
        }
    };
    auto cvt = [&](SRaw raw) -> float {
        if (SDT == 0) return __uint_as_float((uint32_t)raw << 16);
        if (SDT == 1) return f16_bits_to_f32((uint16_t)raw);
        return __uint_as_float(raw);
    };
    // the first iteration's weights go out before x is staged: they do not
    // depend on it

    // ---- stage the activation vector (and the norm weights beside it)
    // every thread loads GEMV_MAX_CH chunks, clamped to the last real one
    // (no branch, so the loads overlap); chunks k >= nch are zeroed at use
    // chunk k of x (and of the norm weights) through buffer descriptors; a
    // chunk past the vector has an out-of-buffer offset and loads as zeros
    // with no memory request, so no select waits on the loads
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, in * 2, 0x00020000);
    u32x4 xc[GEMV_MAX_CH];
#pragma unroll
    for (int c = 0; c < GEMV_MAX_CH; ++c) {
        const int k = t + GEMV_THREADS * c;
        xc[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, k < nch ? 16u * k : OOB, 0, 0));
    }
    // norm weights of the same chunks (bf16: one 16-byte load, f32: two)
    u32x4 wn[GEMV_MAX_CH][2];
    if (p.norm_w) {
        const __amdgpu_buffer_rsrc_t nres =
            __builtin_amdgcn_make_buffer_rsrc((void*)p.norm_w, 0, in * (p.norm_w_f32 ? 4 : 2), 0x00020000);
#pragma unroll
        for (int c = 0; c < GEMV_MAX_CH; ++c) {
            const int k = t + GEMV_THREADS * c;
            if (p.norm_w_f32) {
                const uint32_t o = k < nch ? 32u * k : OOB;
                wn[c][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(nres, o, 0, 0));
                wn[c][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(nres, o + 16, 0, 0));
            } else {
                wn[c][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(nres, k < nch ? 16u * k : OOB, 0, 0));
            }
        }
    }
    // the first two row steps' weights go out behind x: a wait for x does
    // not wait for them
    RowLoads l0, l1, l2;
    load_row(r0 + tr, l0);
    load_row(r0 + rps + tr, l1);
    float inv = 1.f;
    if (p.norm_w) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < GEMV_MAX_CH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = __uint_as_float(xc[c][e] << 16), hi = __uint_as_float(xc[c][e] & 0xffff0000u);
                ss = fmaf(lo, lo, ss);
                ss = fmaf(hi, hi, ss);
            }
        ss = wave_sum(ss);
        if ((t & 63) == 0) red[t >> 6] = ss;
        __syncthreads();
        if (NT == 256) {
            ss = (red[0] + red[1]) + (red[2] + red[3]);
        } else {
            float r4[NT / 256];
#pragma unroll
            for (int i = 0; i < NT / 256; ++i) r4[i] = (red[4 * i] + red[4 * i + 1]) + (red[4 * i + 2] + red[4 * i + 3]);
            ss = 0.f;
#pragma unroll
            for (int i = 0; i < NT / 256; ++i) ss += r4[i];
        }
        inv = 1.f / sqrtf(ss / (float)in + p.norm_eps);
    }
#pragma unroll
    for (int c = 0; c < GEMV_MAX_CH; ++c) {
        if (GEMV_THREADS * c >= nch) break;  // uniform: no chunk of this pass exists
        const int k = t + GEMV_THREADS * c;
        float h[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            h[2 * e] = __uint_as_float(xc[c][e] << 16);
            h[2 * e + 1] = __uint_as_float(xc[c][e] & 0xffff0000u);
        }
        if (p.norm_w) {
            float w[8];
            if (p.norm_w_f32) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    w[i] = __uint_as_float(wn[c][0][i]);
                    w[4 + i] = __uint_as_float(wn[c][1][i]);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w[2 * e] = __uint_as_float(wn[c][0][e] << 16);
                    w[2 * e + 1] = __uint_as_float(wn[c][0][e] & 0xffff0000u);
                }
            }
            // chunks past the vector carry x = 0, so h stays 0
#pragma unroll
            for (int i = 0; i < 8; ++i) h[i] = bf16_bits_to_f32(f32_to_bf16_bits(w[i] * (h[i] * inv)));
        }
        if (k < nch) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xp[4 * (k + (k >> 3)) + j] = (__float_as_uint(h[j]) >> 16) | (__float_as_uint(h[j + 4]) & 0xffff0000u);
        }
        float cs = ((h[0] + h[1]) + (h[2] + h[3])) + ((h[4] + h[5]) + (h[6] + h[7]));
        cs = group_sum(cs, 8);
        if ((k & 7) == 0 && k < nch) xs[k >> 3] = cs;
    }
    __syncthreads();

    // and-or operands: a VOP3 takes no literal and reads one scalar at most,
    // so the mask sits in an SGPR and the bf16 pair 128|128 in a VGPR
    uint32_t nib_mask, bf_128;
    asm volatile("s_mov_b32 %0, 0x000f000f" : "=s"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(bf_128));
    auto dot_row = [&](const RowLoads& L) {
        float acc = 0.f, hist[GEMV_NPT + 1];
        hist[0] = 0.f;
#pragma unroll
        for (int q = 0; q < GEMV_NPT; ++q) {
            int g = min(tl + tpr * q, G - 1);
            // a group's x is read from LDS once the group two back is dotted:
            // two groups of x in registers at a time, none held across rows
            if (q >= 2) asm volatile("" : "+v"(g) : "v"(hist[q - 1]));
            else asm volatile("" : "+v"(g));
            float d4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t word = k < 4 ? L.w[q][0][k] : L.w[q][1][k - 4];
                const u32x4 xv = *(const u32x4*)(xp + 4 * (9 * g + k));
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const uint32_t sh = word >> (4 * jj);
                    uint32_t pr;
                    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(pr) : "v"(sh), "s"(nib_mask), "v"(bf_128));
                    const uint32_t xw = xv[jj];
                    d4[jj] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pr), __builtin_bit_cast(bf16x2v, xw),
                                                            d4[jj], false);
                }
            }
            const float d = (d4[0] + d4[1]) + (d4[2] + d4[3]);
            // sum x (128 + q) = d  ->  sum x q = d - 128 sum x
            const float sv = (L.ok >> q) & 1u ? cvt(L.s[q]) : 0.f;
            const float bv = (L.ok >> q) & 1u ? cvt(L.b[q]) : 0.f;
            acc = fmaf(sv, d, fmaf(bv - 128.f * sv, xs[g], acc));
            hist[q + 1] = acc;
        }
        return acc;
    };
    int fstep = 0;
    auto finish = [&](int j, float acc) {
        if (tpr <= 64) {
            acc = group_sum(acc, tpr);
        } else {
            // the row's waves: sums through LDS behind an LDS-only barrier
            // (the weights in flight are not waited for)
            acc = group_sum(acc, 64);
            float* pp = part[fstep & 1];
            if ((t & 63) == 0) pp[t >> 6] = acc;
            lds_barrier();
            const int w0 = (t - tl) >> 6;  // the row's first wave
            acc = 0.f;
            for (int i = 0; i < tpr / 64; ++i) acc += pp[w0 + i];
            ++fstep;
        }
        if (tl == 0 && j < r_end) {
            const int64_t o = (int64_t)j * p.y_stride_row;
            if (p.y_f32)
                ((float*)p.y)[o] = acc;
            else
                ((uint16_t*)p.y)[o] = f32_to_bf16_bits(acc);
        }
    };
    // three register sets rotate: while one row step is dotted the next two
    // are in flight, and no loaded value is copied before use.  Loads of
    // steps past the tile end are out-of-buffer offsets: no memory request.
    const int nsteps = (r_end - r0 + rps - 1) / rps;
    int rb = r0, i = 0;
    for (; i + 3 <= nsteps; i += 3) {
        load_row(rb + 2 * rps + tr, l2);
        finish(rb + tr, dot_row(l0));
        rb += rps;
        load_row(rb + 2 * rps + tr, l0);
        finish(rb + tr, dot_row(l1));
        rb += rps;
        load_row(rb + 2 * rps + tr, l1);
        finish(rb + tr, dot_row(l2));
        rb += rps;
    }
    if (i < nsteps) finish(rb + tr, dot_row(l0));
    if (i + 1 < nsteps) finish(rb + rps + tr, dot_row(l1));
}

// ---------------------------------------------------------------- GEMV, generic
// Any bits dividing 32, bf16 or f32 activations, M tokens: one wave per
// (token, output row), fp32 FMAs over dequantized weights.
template <int SDT>
__global__ void __launch_bounds__(256) affine_gemv_generic_kernel(AffineGemvParams p) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int l = threadIdx.x & 63;
    const int64_t total = (int64_t)p.m * p.out_rows;
    if (wave >= total) return;
    const int m = wave / p.out_rows;
    const int j = wave - m * p.out_rows;
    int64_t wr = (int64_t)(j / p.map_a) * p.map_b + p.map_c + (j % p.map_a);
    const int xrow = (m * (p.out_rows / p.map_a) + j / p.map_a) / p.x_div;
    if (p.rhs_idx) {  // routed: the expert's rows, zeros for an id out of range
        const int32_t e = p.rhs_idx[j / p.map_a];
        if (e < 0 || e >= p.experts) {
            if (l == 0) {
                const int64_t o = (int64_t)m * p.y_stride_token + (int64_t)j * p.y_stride_row;
                if (p.y_f32)
                    ((float*)p.y)[o] = 0.f;
                else
                    ((uint16_t*)p.y)[o] = 0;
            }
            return;
        }
        wr = (int64_t)e * p.map_a + (j % p.map_a);
    }
    const int per = 32 / p.bits;
    const uint32_t mask = p.bits == 32 ? 0xffffffffu : ((1u << p.bits) - 1u);
    const int64_t wpr = p.in_features / per;
    const int64_t groups = p.in_features / p.group;
    float acc = 0.f;
    for (int64_t i = l; i < p.in_features; i += 64) {
        const uint32_t word = p.packed[wr * wpr + i / per];
        const float q = (float)((word >> (p.bits * (i % per))) & mask);
        const float s = load_scale<SDT>(p.scales, wr * groups + i / p.group);
        const float b = load_scale<SDT>(p.biases, wr * groups + i / p.group);
        const float wv = add_rn(mul_rn(s, q), b);
        acc = fmaf(load_act(p.x, p.x_f32, (int64_t)xrow * p.x_stride + i), wv, acc);
    }
    acc = wave_sum(acc);
    if (l == 0) {
        const int64_t o = (int64_t)m * p.y_stride_token + (int64_t)j * p.y_stride_row;
        if (p.y_f32)
            ((float*)p.y)[o] = acc;
        else
            ((uint16_t*)p.y)[o] = f32_to_bf16_bits(acc);
    }
}

}  // namespace

hipError_t launch_affine_dequant(const AffineDequantParams& p, hipStream_t st) {
    const int64_t words = p.out_features * (p.in_features / (32 / p.bits));
    const int64_t blocks = std::min<int64_t>((words + 255) / 256, 65536);
    if (p.scale_dtype == 0)
        hipLaunchKernelGGL(affine_dequant_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, st, p);
    else if (p.scale_dtype == 1)
        hipLaunchKernelGGL(affine_dequant_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(affine_dequant_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, st, p);
    return hipGetLastError();
}

// Weight rows the fast path addresses: the last activation vector's rows end
// at (nvec - 1) * map_b + map_c + (its row count).
static int64_t gemv_weight_rows(const AffineGemvParams& p) {
    if (p.rhs_idx) return p.experts * p.map_a;
    const int64_t nvec = (p.out_rows + p.map_a - 1) / p.map_a;
    const int64_t last_rows = std::min<int64_t>(p.map_a, p.out_rows - (nvec - 1) * p.map_a);
    return (nvec - 1) * p.map_b + p.map_c + last_rows;
}

bool affine_gemv_fast_ok(const AffineGemvParams& p) {
    return !p.force_generic && p.bits == 4 && p.group == 64 && !p.x_f32 && p.m == 1 && p.in_features <= GEMV_MAX_IN &&
           p.in_features % 64 == 0 && ((uintptr_t)p.x & 15) == 0 && p.x_stride % 8 == 0 &&
           p.in_features <= 64 * GEMV_NPT_MAX * GEMV_NT && (!p.norm_w || ((uintptr_t)p.norm_w & 15) == 0) &&
           // 32-bit buffer offsets (24-bit row numbers) reach every weight and
           // scale byte, with 2^31 free above them for the out-of-buffer offset
           gemv_weight_rows(p) < (int64_t(1) << 24) &&
           gemv_weight_rows(p) * (p.in_features / 2) < (int64_t(1) << 31) &&
           gemv_weight_rows(p) * (p.in_features / 64) * (p.scale_dtype == 2 ? 4 : 2) < (int64_t(1) << 31);
}

// Launch geometry of the 4-bit fast path.
struct FastPlan {
    AffineGemvParams p;  // with tpr, tile_rows, tiles_per_vec set
    unsigned grid;
    int npt;
    int nt;  // threads per workgroup
    int64_t steps;  // row steps of the whole launch
    uint32_t wbytes, sbytes;
};

// Workgroups of the fast path one CU holds at once: the two-group instance
// takes 193 registers per lane (one 512-thread workgroup per CU), the
// one-group instance 95 (two).
static int64_t gemv_slots(int npt) { return (int64_t)mrc::cu_count() * (npt == 1 ? 2 : 1); }

// per_tile 0: tiles of ceil(steps / slots) row steps, so the launch runs in
// one round of workgroups (a second round repeats the whole staging chain)
static FastPlan plan_fast(const AffineGemvParams& q, int64_t per_tile_req = 0) {
    FastPlan f;
    AffineGemvParams& p = f.p;
    p = q;
    const int G = p.in_features / 64;
    const int nvec = (p.out_rows + p.map_a - 1) / p.map_a;
    const int per_vec = std::min(p.map_a, p.out_rows);
    const int nt = GEMV_NT;
    f.nt = nt;
    auto steps = [&](int t) { return (int64_t)nvec * ((per_vec + nt / t - 1) / (nt / t)); };
    // threads per row: at most two groups each (two waves per SIMD; a row of
    // more than 64 threads sums its waves through LDS), more while the grid
    // holds fewer row steps than the GPU has CUs; tiles of whole steps, at
    // least one per CU
    int tpr = 1;
    while (tpr < nt && tpr * 2 < G) tpr <<= 1;
    while (tpr < 64 && steps(tpr) < 256) tpr <<= 1;
    const int rps = nt / tpr;
    const int64_t total = steps(tpr);
    const int npt = (G + tpr - 1) / tpr;
    const int64_t slots = gemv_slots(npt);
    const int64_t per_tile = per_tile_req > 0 ? per_tile_req : std::max<int64_t>(1, (total + slots - 1) / slots);
    f.steps = total;
    p.tpr = tpr;
    p.tile_rows = (int)std::min<int64_t>(per_tile * rps, per_vec);
    p.tiles_per_vec = (per_vec + p.tile_rows - 1) / p.tile_rows;
    f.grid = (unsigned)(nvec * p.tiles_per_vec);
    f.npt = npt;  // 1 or 2
    const int64_t w_rows = gemv_weight_rows(p);
    f.wbytes = (uint32_t)(w_rows * (p.in_features / 2));
    f.sbytes = (uint32_t)(w_rows * G * (p.scale_dtype == 2 ? 4 : 2));
    return f;
}

// One launch of a (or of a and b, which share the template instance).
static hipError_t launch_fast(const FastPlan& a, const FastPlan* b, hipStream_t st) {
    const FastPlan& s = b ? *b : a;
    if (a.npt > 2 || (b && b->npt != a.npt)) return hipErrorInvalidValue;  // the instances hold 1 or 2 groups
    const dim3 grid(a.grid + (b ? b->grid : 0));
    const int tiles0 = (int)a.grid;
#define MR_GEMV4(SDT, NPT)                                                                                         \
    hipLaunchKernelGGL((affine_gemv4_kernel<SDT, NPT, GEMV_NT>), grid, dim3(GEMV_NT), 0, st, a.p, a.wbytes, a.sbytes, \
                       s.p, s.wbytes, s.sbytes, tiles0)
#define MR_GEMV4_NPT(SDT)     \
    do {                      \
        if (a.npt == 1)       \
            MR_GEMV4(SDT, 1); \
        else                  \
            MR_GEMV4(SDT, 2); \
    } while (0)
    if (a.p.scale_dtype == 0)
        MR_GEMV4_NPT(0);
    else if (a.p.scale_dtype == 1)
        MR_GEMV4_NPT(1);
    else
        MR_GEMV4_NPT(2);
#undef MR_GEMV4_NPT
#undef MR_GEMV4
    return hipGetLastError();
}

hipError_t launch_affine_gemv_pair(const AffineGemvParams& a, const AffineGemvParams& b, hipStream_t st) {
    if (affine_gemv_fast_ok(a) && affine_gemv_fast_ok(b) && a.scale_dtype == b.scale_dtype) {
        FastPlan fa = plan_fast(a), fb = plan_fast(b);
        if (fa.npt == fb.npt && fa.nt == fb.nt) {
            // one round of workgroups for the two together
            const int64_t slots = gemv_slots(fa.npt);
            if ((int64_t)fa.grid + fb.grid > slots) {
                const int64_t per_tile = (fa.steps + fb.steps + slots - 1) / slots;
                fa = plan_fast(a, per_tile);
                fb = plan_fast(b, per_tile);
            }
            return launch_fast(fa, &fb, st);
        }
    }
    const hipError_t e = launch_affine_gemv(a, st);
    return e != hipSuccess ? e : launch_affine_gemv(b, st);
}

hipError_t launch_affine_gemv(const AffineGemvParams& q, hipStream_t st) {
    if (affine_gemv_fast_ok(q)) return launch_fast(plan_fast(q), nullptr, st);
    const AffineGemvParams& p = q;
    const int64_t waves = (int64_t)p.m * p.out_rows;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    if (p.scale_dtype == 0)
        hipLaunchKernelGGL(affine_gemv_generic_kernel<0>, dim3(grid), dim3(256), 0, st, p);
    else if (p.scale_dtype == 1)
        hipLaunchKernelGGL(affine_gemv_generic_kernel<1>, dim3(grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(affine_gemv_generic_kernel<2>, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
