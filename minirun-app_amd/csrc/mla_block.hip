// Elementwise and small kernels of the MLA block on gfx950: RMSNorm, the
// adjacent-pair rotary embedding, the latent-cache append and the W_UK
// absorption of the query.
#include <algorithm>

#include "mr_kernels.hpp"

// Arithmetic rounds as written (no a*b+c contraction): the rotary and the
// normalisation follow the reference's separate fp32 operations.
#pragma clang fp contract(off)

namespace mr {

namespace {

__device__ __forceinline__ float ld(const void* p, int f32, int64_t i) {
    return f32 ? ((const float*)p)[i] : bf16_bits_to_f32(((const uint16_t*)p)[i]);
}
__device__ __forceinline__ void st(void* p, int f32, int64_t i, float v) {
    if (f32)
        ((float*)p)[i] = v;
    else
        ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
}

__device__ __forceinline__ float block_sum_256(float v, float* sh) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return t;
}

// K3Norm.rms (Normalization.swift:15-19): w * (x * rsqrt(mean(x^2) + eps)),
// eps inside the root, weight applied after.  One 256-thread block per row.
__global__ void __launch_bounds__(256) rmsnorm_kernel(RmsNormParams p) {
    __shared__ float sh[4];
    const int64_t row = blockIdx.x;
    float ss = 0.f;
    for (int i = threadIdx.x; i < p.dim; i += 256) {
        const float v = ld(p.x, p.x_f32, row * p.x_stride + i);
        ss = fmaf(v, v, ss);
    }
    ss = block_sum_256(ss, sh);
    const float inv = 1.f / sqrtf(ss / (float)p.dim + p.eps);
    for (int i = threadIdx.x; i < p.dim; i += 256) {
        const float v = ld(p.x, p.x_f32, row * p.x_stride + i);
        const float w = ld(p.weight, p.w_f32, i);
        st(p.out, p.out_f32, row * p.out_stride + i, w * (v * inv));
    }
}

// DeepSeekV4Rotary.apply (DeepSeekV4Attention.swift:151-163): pairs
// (2i, 2i+1) of columns [col0, col0+dim) of every row, fp32 arithmetic as
// written (two roundings per product sum), cast back to the storage dtype.
// Tables are [n_pos, dim/2] fp32, built on the host from fp64 angles.
__global__ void __launch_bounds__(256) rope_kernel(RopeParams p) {
    const int half = p.dim / 2;
    const int64_t total = p.n_pos * p.inner * half;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t pos = t / (p.inner * half);
        const int64_t rem = t - pos * (p.inner * half);
        const int64_t r = rem / half;
        const int i = (int)(rem - r * half);
        const int64_t base = (pos * p.inner + r) * p.row_stride + p.col0 + 2 * i;
        const float e = ld(p.x, p.x_f32, base);
        const float o = ld(p.x, p.x_f32, base + 1);
        const float c = p.cos_t[pos * half + i];
        const float s = p.sin_t[pos * half + i];
        const float re = sub_rn(mul_rn(e, c), mul_rn(o, s));
        const float im = add_rn(mul_rn(e, s), mul_rn(o, c));
        st(p.x, p.x_f32, base, re);
        st(p.x, p.x_f32, base + 1, im);
    }
}

// Latent-cache append (MLA.swift:142-157 with the rotary tail of
// DeepSeekV4CompressedAttention.swift:676-694): for token t, the kv_a row
// [kv_rank latent ++ rope_dim key] -> RMSNorm(latent) * w -> bf16 cache row
// (start + t)[0:kv_rank]; the key tail rotated at its position -> bf16
// [kv_rank : kv_rank + rope_dim].  One block per token.
__global__ void __launch_bounds__(256) cache_append_kernel(CacheAppendParams p) {
    __shared__ float sh[4];
    const int64_t t = blockIdx.x;
    float ss = 0.f;
    for (int i = threadIdx.x; i < p.kv_rank; i += 256) {
        const float v = ld(p.kv, p.kv_f32, t * p.kv_stride + i);
        ss = fmaf(v, v, ss);
    }
    ss = block_sum_256(ss, sh);
    const float inv = 1.f / sqrtf(ss / (float)p.kv_rank + p.eps);
    uint16_t* lat = p.latent + (p.start_row + t) * p.latent_stride;
    for (int i = threadIdx.x; i < p.kv_rank; i += 256) {
        const float v = ld(p.kv, p.kv_f32, t * p.kv_stride + i);
        lat[i] = f32_to_bf16_bits(ld(p.norm_w, p.w_f32, i) * (v * inv));
    }
    const int half = p.rope_dim / 2;
    uint16_t* rk = p.rope + (p.start_row + t) * p.rope_stride;
    for (int i = threadIdx.x; i < half; i += 256) {
        const float e = ld(p.kv, p.kv_f32, t * p.kv_stride + p.kv_rank + 2 * i);
        const float o = ld(p.kv, p.kv_f32, t * p.kv_stride + p.kv_rank + 2 * i + 1);
        const float c = p.cos_t[t * half + i];
        const float s = p.sin_t[t * half + i];
        rk[2 * i] = f32_to_bf16_bits(sub_rn(mul_rn(e, c), mul_rn(o, s)));
        rk[2 * i + 1] = f32_to_bf16_bits(add_rn(mul_rn(e, s), mul_rn(o, c)));
    }
}

// Query absorption (MLA.swift:180-188): q_lat[h][r] = sum_{d<dn} q_nope[h][d]
// * W_UK[h][d][r], with W_UK the rows h*(dn+dv) + d of the affine kv_b
// weight [H*(dn+dv), kv_rank] (4-bit, group 64).  One block per head:
// thread t owns packed word t%64 (8 columns) and rows d = t/64 (mod 4).
__global__ void __launch_bounds__(256) absorb_q_kernel(AbsorbParams p) {
    __shared__ float part[4][512];
    const int h = blockIdx.x;
    const int c = threadIdx.x & 63;  // word (8 columns of 512)
    const int ds = threadIdx.x >> 6;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    const int wpr = p.kv_rank / 8;
    const int gpr = p.kv_rank / 64;
    for (int d = ds; d < p.nope_dim; d += 4) {
        const int64_t row = (int64_t)h * (p.nope_dim + p.v_dim) + d;
        const uint32_t word = p.packed[row * wpr + c];
        const int64_t gi = row * gpr + c / 8;
        const float s = p.scale_dtype == 2 ? ((const float*)p.scales)[gi]
                        : (p.scale_dtype == 1 ? f16_bits_to_f32(((const uint16_t*)p.scales)[gi])
                                              : bf16_bits_to_f32(((const uint16_t*)p.scales)[gi]));
        const float b = p.scale_dtype == 2 ? ((const float*)p.biases)[gi]
                        : (p.scale_dtype == 1 ? f16_bits_to_f32(((const uint16_t*)p.biases)[gi])
                                              : bf16_bits_to_f32(((const uint16_t*)p.biases)[gi]));
        const float qn = bf16_bits_to_f32(p.q[(int64_t)h * p.q_head_stride + d]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float wv = add_rn(mul_rn(s, (float)((word >> (4 * j)) & 15u)), b);
            acc[j] = fmaf(qn, wv, acc[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) part[ds][8 * c + j] = acc[j];
    __syncthreads();
    for (int r = threadIdx.x; r < p.kv_rank; r += 256) {
        const float v = (part[0][r] + part[1][r]) + (part[2][r] + part[3][r]);
        p.q_lat[(int64_t)h * p.q_lat_head_stride + r] = f32_to_bf16_bits(v);
    }
}

}  // namespace

hipError_t launch_rmsnorm(const RmsNormParams& p, hipStream_t st) {
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)p.rows), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_rope(const RopeParams& p, hipStream_t st) {
    const int64_t total = p.n_pos * p.inner * (p.dim / 2);
    const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
    hipLaunchKernelGGL(rope_kernel, dim3(blocks > 0 ? blocks : 1), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_cache_append(const CacheAppendParams& p, hipStream_t st) {
    hipLaunchKernelGGL(cache_append_kernel, dim3((unsigned)p.tokens), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_absorb_q(const AbsorbParams& p, hipStream_t st) {
    hipLaunchKernelGGL(absorb_q_kernel, dim3((unsigned)p.heads), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
