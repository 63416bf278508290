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
// Rows are processed in blocks of RB by one wave; lane l owns groups
// l, l+64, ... of those rows and reuses its staged x pairs for all RB rows.
// Output row j reads weight row (j / A) * B + C + (j % A) and activation
// vector (j / A) (a plain GEMV is A = O, B = 0, C = 0; the per-head W_UV
// product is A = 128, B = 256, C = 128).  One workgroup covers rows of a
// single activation vector, which it stages in LDS as pair words.
constexpr int GEMV_THREADS = 256;
constexpr int GEMV_MAX_IN = 16384;  // activation length staged per token

template <int SDT, int RB>
__global__ void __launch_bounds__(GEMV_THREADS) affine_gemv4_kernel(AffineGemvParams p) {
    __shared__ __attribute__((aligned(16))) uint32_t xp[GEMV_MAX_IN / 2];  // (x_j, x_j+4) pairs
    __shared__ float xs[GEMV_MAX_IN / 32];                              // per-group sums of x (group >= 32)
    const int rows_per_wg = (GEMV_THREADS / 64) * RB;
    const int j0 = blockIdx.x * rows_per_wg;
    if (j0 >= p.out_rows) return;
    const int xg = j0 / p.map_a;  // activation vector of this workgroup
    const int in = p.in_features;
    const int words = in / 8;
    const int groups = in / 64;
    const uint16_t* x = (const uint16_t*)p.x + (int64_t)xg * p.x_stride;

    // stage x as pair words: word k, pair j = (x[8k+j] | x[8k+j+4] << 16)
    for (int t = threadIdx.x; t < words * 4; t += GEMV_THREADS) {
        const int k = t >> 2, j = t & 3;
        xp[t] = (uint32_t)x[8 * k + j] | ((uint32_t)x[8 * k + j + 4] << 16);
    }
    for (int g = threadIdx.x; g < groups; g += GEMV_THREADS) {
        float s = 0.f;
        for (int i = 0; i < 64; ++i) s += bf16_bits_to_f32(x[64 * g + i]);
        xs[g] = s;
    }
    __syncthreads();

    const int w = threadIdx.x >> 6;
    const int l = threadIdx.x & 63;
    const int jw = j0 + w * RB;  // first output row of this wave
    float acc[RB];
    int64_t wrow[RB];
    bool rv[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        acc[r] = 0.f;
        const int j = jw + r;
        rv[r] = j < p.out_rows && j / p.map_a == xg;
        const int jj = rv[r] ? j : jw;
        wrow[r] = (int64_t)(jj / p.map_a) * p.map_b + p.map_c + (jj % p.map_a);
    }
    const int64_t wpr = words;  // packed words per weight row
    for (int g = l; g < groups; g += 64) {
        // x pairs of group g: 8 words x 4 pairs
        u32x4 xv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) xv[k] = *(const u32x4*)(xp + 4 * (8 * g + k));
        const float xsum = xs[g];
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            if (!rv[r]) continue;
            const uint32_t* wp = p.packed + wrow[r] * wpr + 8 * g;
            const u32x4 w0 = __builtin_nontemporal_load((const u32x4*)wp);
            const u32x4 w1 = __builtin_nontemporal_load((const u32x4*)wp + 1);
            const float s = load_scale<SDT>(p.scales, wrow[r] * groups + g);
            const float bb = load_scale<SDT>(p.biases, wrow[r] * groups + g);
            float d = 0.f;
            typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t word = k < 4 ? w0[k] : w1[k - 4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t pr = ((word >> (4 * j)) & 0x000F000Fu) | 0x43004300u;
                    const uint32_t xw = xv[k][j];  // bit_cast of a vector-element lvalue reads element 0
                    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, pr), __builtin_bit_cast(bf16x2v, xw),
                                                       d, false);
                }
            }
            // sum x (128 + q) = d  ->  sum x q = d - 128 sum x
            acc[r] = fmaf(s, d, fmaf(bb - 128.f * s, xsum, acc[r]));
        }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const float v = wave_sum(acc[r]);
        if (l == 0 && rv[r]) {
            const int64_t o = (int64_t)(jw + r) * p.y_stride_row;
            if (p.y_f32)
                ((float*)p.y)[o] = v;
            else
                ((uint16_t*)p.y)[o] = f32_to_bf16_bits(v);
        }
    }
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
    const int64_t wr = (int64_t)(j / p.map_a) * p.map_b + p.map_c + (j % p.map_a);
    const int xrow = m * (p.out_rows / p.map_a) + j / p.map_a;
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

bool affine_gemv_fast_ok(const AffineGemvParams& p) {
    return !p.force_generic && p.bits == 4 && p.group == 64 && !p.x_f32 && p.m == 1 && p.in_features <= GEMV_MAX_IN &&
           p.in_features % 64 == 0 && (p.map_a % 4 == 0 || p.map_a == p.out_rows);
}

hipError_t launch_affine_gemv(const AffineGemvParams& p, hipStream_t st) {
    if (affine_gemv_fast_ok(p)) {
        // rows per wave: enough waves to cover the GPU, RB rows to reuse x
        int rb = p.out_rows >= 8192 ? 4 : (p.out_rows >= 4096 ? 2 : 1);
        while (p.map_a != p.out_rows && p.map_a % (4 * rb) != 0) rb >>= 1;
        const int rows_per_wg = 4 * rb;  // divides map_a (a multiple of 4 ... 16) when grouped
        const unsigned grid = (unsigned)((p.out_rows + rows_per_wg - 1) / rows_per_wg);
#define MR_GEMV4(SDT, RB) hipLaunchKernelGGL((affine_gemv4_kernel<SDT, RB>), dim3(grid), dim3(GEMV_THREADS), 0, st, p)
        if (rb == 4) {
            if (p.scale_dtype == 0) MR_GEMV4(0, 4); else if (p.scale_dtype == 1) MR_GEMV4(1, 4); else MR_GEMV4(2, 4);
        } else if (rb == 2) {
            if (p.scale_dtype == 0) MR_GEMV4(0, 2); else if (p.scale_dtype == 1) MR_GEMV4(1, 2); else MR_GEMV4(2, 2);
        } else {
            if (p.scale_dtype == 0) MR_GEMV4(0, 1); else if (p.scale_dtype == 1) MR_GEMV4(1, 1); else MR_GEMV4(2, 1);
        }
#undef MR_GEMV4
        return hipGetLastError();
    }
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
