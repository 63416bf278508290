// Elementwise and small kernels of the MLA block on gfx950: RMSNorm, the
// adjacent-pair rotary embedding, the latent-cache append and the W_UK
// absorption of the query.
#include <algorithm>

#include "cache_append.hpp"
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

// Latent-cache append: one block per token (cache_append_row).
__global__ void __launch_bounds__(256) cache_append_kernel(CacheAppendParams p) {
    __shared__ float sh[4];
    cache_append_row(p, blockIdx.x, sh);
}

// Query absorption (MLA.swift:180-188): q_lat[h][r] = sum_{d<dn} q_nope[h][d]
// * W_UK[h][d][r], with W_UK the rows h*(dn+dv) + d of the affine kv_b
// weight [H*(dn+dv), kv_rank] (4-bit, group 64).  One block per head:
// thread t owns packed word t%64 (8 columns) and rows d = t/64 (mod 4).
__global__ void __launch_bounds__(256) absorb_q_kernel(AbsorbParams p) {
    __shared__ float part[4][512];
    if (p.app_on && blockIdx.x == gridDim.x - 1) {  // the extra workgroup: the cache append
        cache_append_row(p.app, 0, &part[0][0]);
        return;
    }
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

// The same product, 256 columns of one head per workgroup (kv_rank 512,
// nope_dim 128): the head's query values, scales and biases are staged in
// LDS with one load per thread; lane (rs = l/8, quad wq = l%8) of wave w
// loads the 16-byte words of rows d = 32k + 8w + rs (k < 4) and columns
// 256 half + 32 wq .. +31, so a thread issues four weight loads.  Row sums
// meet by lane exchange (rs) and through LDS (waves).
template <int SDT>
__global__ void __launch_bounds__(256) absorb_q_fast_kernel(AbsorbParams p) {
    __shared__ float qs[128];
    __shared__ float sc[128][8], bi[128][8];
    __shared__ __attribute__((aligned(16))) float part[4][256];
    if (p.app_on && blockIdx.x == gridDim.x - 1) {  // the extra workgroup: the cache append
        cache_append_row(p.app, 0, qs);
        return;
    }
    const int h = blockIdx.x >> 1;
    const int half = blockIdx.x & 1;
    const int t = threadIdx.x;
    const int w = t >> 6, l = t & 63;
    const int rs = l >> 3, wq = l & 7;
    const int64_t row0 = (int64_t)h * (p.nope_dim + p.v_dim);
    if (p.rope_cos && half == 0 && t < p.rope_dim / 2) {
        // this head's rotary part, in place (the block reads only the nope
        // part): the arithmetic of rope_kernel at one position
        uint16_t* xr = (uint16_t*)p.q + (int64_t)h * p.q_head_stride + p.rope_col0 + 2 * t;
        const float e = bf16_bits_to_f32(xr[0]), o = bf16_bits_to_f32(xr[1]);
        const float c = p.rope_cos[t], sn = p.rope_sin[t];
        xr[0] = f32_to_bf16_bits(sub_rn(mul_rn(e, c), mul_rn(o, sn)));
        xr[1] = f32_to_bf16_bits(add_rn(mul_rn(e, sn), mul_rn(o, c)));
    }
    // weights first: they do not depend on the staging
    u32x4 wd[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int d = 32 * k + 8 * w + rs;
        wd[k] = *(const u32x4*)(p.packed + (row0 + d) * 64 + 32 * half + 4 * wq);
    }
    // scales and biases of the head's 128 nope rows (8 groups each) and q
    {
        const int64_t gi = row0 * 8 + 4 * t;  // four consecutive (row, group) entries
        float sv[4], bv[4];
        if (SDT == 2) {
            const f32x4 a = *(const f32x4*)((const float*)p.scales + gi);
            const f32x4 c = *(const f32x4*)((const float*)p.biases + gi);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sv[i] = a[i];
                bv[i] = c[i];
            }
        } else {
            const u32x2 a = *(const u32x2*)((const uint16_t*)p.scales + gi);
            const u32x2 c = *(const u32x2*)((const uint16_t*)p.biases + gi);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint16_t ua = (uint16_t)(a[i >> 1] >> (16 * (i & 1)));
                const uint16_t uc = (uint16_t)(c[i >> 1] >> (16 * (i & 1)));
                sv[i] = SDT == 1 ? f16_bits_to_f32(ua) : bf16_bits_to_f32(ua);
                bv[i] = SDT == 1 ? f16_bits_to_f32(uc) : bf16_bits_to_f32(uc);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[(4 * t + i) >> 3][(4 * t + i) & 7] = sv[i];
            bi[(4 * t + i) >> 3][(4 * t + i) & 7] = bv[i];
        }
        if (t < 128) qs[t] = bf16_bits_to_f32(p.q[(int64_t)h * p.q_head_stride + t]);
    }
    __syncthreads();
    const int grp = 4 * half + (wq >> 1);  // group of this lane's 32 columns
    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int d = 32 * k + 8 * w + rs;
        const float s = sc[d][grp], b = bi[d][grp], qd = qs[d];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                const float wv = add_rn(mul_rn(s, (float)((wd[k][j] >> (4 * n)) & 15u)), b);
                acc[8 * j + n] = fmaf(qd, wv, acc[8 * j + n]);
            }
    }
    // rows of the wave: lanes l, l^8, l^16, l^32 hold the same columns
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        acc[i] = xor8_sum(acc[i]);
        acc[i] = xor16_sum(acc[i]);
        acc[i] = xor32_sum(acc[i]);
    }
    if (rs == 0) {
#pragma unroll
        for (int i = 0; i < 32; i += 4)
            *(f32x4*)&part[w][32 * wq + i] = f32x4{acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
    }
    __syncthreads();
    const float v = (part[0][t] + part[1][t]) + (part[2][t] + part[3][t]);
    p.q_lat[(int64_t)h * p.q_lat_head_stride + 256 * half + t] = f32_to_bf16_bits(v);
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
    const int sz = p.scale_dtype == 2 ? 4 : 2;
    const bool fast = p.kv_rank == 512 && p.nope_dim == 128 && ((uintptr_t)p.packed & 15) == 0 &&
                      ((uintptr_t)p.scales & (2 * sz - 1)) == 0 && ((uintptr_t)p.biases & (2 * sz - 1)) == 0;
    if (p.rope_cos && (!fast || p.rope_dim > 512)) {  // the rotation as its own launch
        RopeParams r{};
        r.x = (void*)p.q;
        r.n_pos = 1;
        r.inner = p.heads;
        r.row_stride = p.q_head_stride;
        r.col0 = p.rope_col0;
        r.dim = p.rope_dim;
        r.cos_t = p.rope_cos;
        r.sin_t = p.rope_sin;
        const hipError_t e = launch_rope(r, st);
        if (e != hipSuccess) return e;
        AbsorbParams q = p;
        q.rope_cos = q.rope_sin = nullptr;
        return launch_absorb_q(q, st);
    }
    if (fast) {
        const dim3 grid((unsigned)p.heads * 2 + (p.app_on ? 1 : 0));
        if (p.scale_dtype == 0)
            hipLaunchKernelGGL(absorb_q_fast_kernel<0>, grid, dim3(256), 0, st, p);
        else if (p.scale_dtype == 1)
            hipLaunchKernelGGL(absorb_q_fast_kernel<1>, grid, dim3(256), 0, st, p);
        else
            hipLaunchKernelGGL(absorb_q_fast_kernel<2>, grid, dim3(256), 0, st, p);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(absorb_q_kernel, dim3((unsigned)p.heads + (p.app_on ? 1 : 0)), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
