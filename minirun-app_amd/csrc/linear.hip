// Dense projections for gfx950: k3Linear (Linear.swift:55-57), y = x . W^T
// with W output-major [out, in] in bf16 or f32, fp32 accumulation, and the
// two dense forms of the MLA decompression weight kv_b_proj that the
// absorbed decode uses (MLA.swift:180-197): query absorption through W_UK
// and value un-absorption through W_UV.
//
// dense_gemv_kernel (HBM-bound: every weight byte is read once per token
// tile):
//   - tpr lanes share an output row (a power of two, tpr * 4 >= the row's
//     16-byte chunks when it can, so a lane holds up to four loads of one
//     row); a wave covers 64 / tpr rows per step, a workgroup 4 waves.
//   - "staged" mode: the activation vectors of the token tile go to LDS as
//     fp32 once per workgroup, with the optional RMSNorm
//     (weight * (x * rsqrt(mean(x^2) + eps)), K3Norm.rms) or the optional
//     sigmoid gate (x * sigmoid(g), MLA.swift:209-211) applied there; bf16
//     inputs are rounded back to bf16 after that, as a separate norm or gate
//     stage would store them.
//   - "direct" mode (grouped rows, y[j] = x[j / map_a] . W[wrow(j)]): each
//     lane reads its x chunk from global memory next to the weight chunk
//     (the vectors are small and shared through L2).
//   - The lanes of a row meet by DPP / permlane butterflies (group_sum).
//
// dense_absorb_kernel: q_lat[h][:] = sum_d q[h][d] * W[h*(nope+v) + d][:]
// (the transposed product: each weight row is scaled by one query value),
// one workgroup per head, each lane owning 8 of the 512 columns, the four
// waves taking every fourth row and meeting in LDS; the head's rotary
// columns may be rotated in the same launch (one position, adjacent pairs).
#include "mr_kernels.hpp"

namespace mr {

namespace {

constexpr int LT = 256;  // threads per workgroup

__device__ __forceinline__ float load_act(const void* p, int f32, int64_t i) {
    return f32 ? ((const float*)p)[i] : bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// Dot of one 16-byte weight chunk with the matching activation values:
// bf16 weights and bf16 activations as four v_dot2_f32_bf16 on the pairs;
// otherwise fp32 multiply-adds (f32 weights: 4 values a chunk).
template <bool WF32, bool XF32>
__device__ __forceinline__ float chunk_dot(const u32x4& w, const void* x, float a) {
    if (WF32) {
        if (XF32) {
            const f32x4 xv = *(const f32x4*)x;
#pragma unroll
            for (int k = 0; k < 4; ++k) a = fmaf(__uint_as_float(w[k]), xv[k], a);
        } else {
            const u32x2 xv = *(const u32x2*)x;
            a = fmaf(__uint_as_float(w[0]), __uint_as_float(xv[0] << 16), a);
            a = fmaf(__uint_as_float(w[1]), __uint_as_float(xv[0] & 0xffff0000u), a);
            a = fmaf(__uint_as_float(w[2]), __uint_as_float(xv[1] << 16), a);
            a = fmaf(__uint_as_float(w[3]), __uint_as_float(xv[1] & 0xffff0000u), a);
        }
    } else if (!XF32) {
        const u32x4 xv = *(const u32x4*)x;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // bit_cast of a vector element reads element 0 with this compiler: copy to scalars first
            const uint32_t wk = w[k], xk = xv[k];
            a = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, wk), __builtin_bit_cast(bf16x2v, xk), a,
                                                false);
        }
    } else {
        const f32x4 x0 = *(const f32x4*)x, x1 = *((const f32x4*)x + 1);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            a = fmaf(__uint_as_float(w[k] << 16), x0[2 * k], a);
            a = fmaf(__uint_as_float(w[k] & 0xffff0000u), x0[2 * k + 1], a);
            a = fmaf(__uint_as_float(w[k + 2] << 16), x1[2 * k], a);
            a = fmaf(__uint_as_float(w[k + 2] & 0xffff0000u), x1[2 * k + 1], a);
        }
    }
    return a;
}

constexpr int GEMV_UNROLL = 8;  // weight chunks in flight per lane

template <bool WF32, bool XF32, bool STAGED>
__global__ void __launch_bounds__(LT) dense_gemv_kernel(DenseGemvParams p) {
    constexpr int VPC = WF32 ? 4 : 8;  // values per 16-byte weight chunk
    constexpr int XE = XF32 ? 4 : 2;   // bytes per activation value
    extern __shared__ __attribute__((aligned(16))) char xs[];  // staged: [mt][in] activations
    __shared__ float red[LT / 64];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.y * p.mt;
    const int mt = min(p.mt, p.m - t0);
    if (STAGED) {
        for (int t = 0; t < mt; ++t) {
            const int64_t xo = (int64_t)(t0 + t) * p.x_stride;
            float r = 1.f;
            if (p.norm_w) {  // sum of squares over the whole vector
                float ss = 0.f;
                for (int i = tid; i < p.in; i += LT) {
                    const float v = load_act(p.x, p.x_f32, xo + i);
                    ss = fmaf(v, v, ss);
                }
                ss = wave_sum(ss);
                if ((tid & 63) == 0) red[tid >> 6] = ss;
                __syncthreads();
                float tot = 0.f;
#pragma unroll
                for (int w = 0; w < LT / 64; ++w) tot += red[w];
                r = rsqrtf(tot / (float)p.in + p.norm_eps);
                __syncthreads();
            }
            for (int i = tid; i < p.in; i += LT) {
                float v = load_act(p.x, p.x_f32, xo + i);
                if (p.norm_w) v = load_act(p.norm_w, p.norm_w_f32, i) * (v * r);
                if (p.gate) {
                    const float g = load_act(p.gate, p.gate_f32, (int64_t)(t0 + t) * p.gate_stride + i);
                    v = v * (1.f / (1.f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f)));
                }
                if (XF32)
                    ((float*)xs)[t * p.in + i] = v;
                else  // bf16 inputs stay bf16, as a separate norm or gate stage would store them
                    ((uint16_t*)xs)[t * p.in + i] = f32_to_bf16_bits(v);
            }
        }
        __syncthreads();
    }
    const int tpr = p.tpr;
    const int lane = tid & 63;
    const int sub = lane / tpr;      // row of this lane within the wave's step
    const int li = lane - sub * tpr;  // lane within the row
    const int rows_per_wave = 64 / tpr;
    const int chunks = p.in / VPC;
    const int wave = tid >> 6;
    const int64_t step0 = (int64_t)blockIdx.x * p.steps_per_wg;
    for (int s = 0; s < p.steps_per_wg; ++s) {
        const int64_t j = ((step0 + s) * (LT / 64) + wave) * rows_per_wave + sub;
        const bool live = j < p.out_rows;
        const int64_t jj = live ? j : 0;
        const int64_t g = jj / p.map_a;
        const int64_t wrow = g * p.map_b + p.map_c + (jj - g * p.map_a);
        const char* wr = (const char*)p.w + wrow * p.w_rs * (WF32 ? 4 : 2);
        // direct mode: this row's activation vector in global memory
        const char* xd = (const char*)p.x + ((int64_t)t0 * p.x_stride + g * p.x_vec_stride) * XE;
        float acc[MAX_GEMV_TOKENS];
#pragma unroll
        for (int t = 0; t < MAX_GEMV_TOKENS; ++t) acc[t] = 0.f;
        auto use = [&](const u32x4& wv, int c) {
            const int i0 = c * VPC;
            if (STAGED) {
#pragma unroll
                for (int t = 0; t < MAX_GEMV_TOKENS; ++t)
                    if (t < mt) acc[t] = chunk_dot<WF32, XF32>(wv, xs + ((int64_t)t * p.in + i0) * XE, acc[t]);
            } else {
                acc[0] = chunk_dot<WF32, XF32>(wv, xd + (int64_t)i0 * XE, acc[0]);
            }
        };
        int c = li;
        // GEMV_UNROLL chunks of the row in flight per lane, then the remainder
        for (; c + (GEMV_UNROLL - 1) * tpr < chunks; c += GEMV_UNROLL * tpr) {
            u32x4 wv[GEMV_UNROLL];
#pragma unroll
            for (int u = 0; u < GEMV_UNROLL; ++u)
                wv[u] = __builtin_nontemporal_load((const u32x4*)(wr + 16 * (int64_t)(c + u * tpr)));
#pragma unroll
            for (int u = 0; u < GEMV_UNROLL; ++u) use(wv[u], c + u * tpr);
        }
        for (; c < chunks; c += tpr) use(__builtin_nontemporal_load((const u32x4*)(wr + 16 * (int64_t)c)), c);
        const int nt = STAGED ? mt : 1;
#pragma unroll
        for (int t = 0; t < MAX_GEMV_TOKENS; ++t) {
            if (t >= nt) break;
            const float v = group_sum(acc[t], tpr);
            if (live && li == 0) {
                const int64_t yo = (int64_t)(t0 + t) * p.y_stride_token + j * p.y_stride_row;
                if (p.y_f32)
                    ((float*)p.y)[yo] = v;
                else
                    ((uint16_t*)p.y)[yo] = f32_to_bf16_bits(v);
            }
        }
    }
}

template <bool WF32>
__global__ void __launch_bounds__(LT) dense_absorb_kernel(DenseAbsorbParams p) {
    constexpr int VPC = WF32 ? 4 : 8;
    constexpr int CPL = 8 / VPC;  // 16-byte chunks per lane (a lane owns 8 columns)
    __shared__ float qs[1024];
    __shared__ __attribute__((aligned(16))) float part[LT / 64][512];
    const int h = blockIdx.x;
    const int tid = threadIdx.x;
    uint16_t* qh = (uint16_t*)p.q + (int64_t)h * p.q_head_stride;
    for (int d = tid; d < p.nope_dim; d += LT) qs[d] = bf16_bits_to_f32(qh[d]);
    if (p.rope_cos) {  // the head's rotary columns, in place (they are not read below)
        for (int i = tid; i < p.rope_dim / 2; i += LT) {
            const float a = bf16_bits_to_f32(qh[p.rope_col0 + 2 * i]);
            const float b = bf16_bits_to_f32(qh[p.rope_col0 + 2 * i + 1]);
            const float c = p.rope_cos[i], s = p.rope_sin[i];
            qh[p.rope_col0 + 2 * i] = f32_to_bf16_bits(sub_rn(mul_rn(a, c), mul_rn(b, s)));
            qh[p.rope_col0 + 2 * i + 1] = f32_to_bf16_bits(add_rn(mul_rn(a, s), mul_rn(b, c)));
        }
    }
    __syncthreads();
    const int wave = tid >> 6, lane = tid & 63;
    float acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = 0.f;
    const int64_t row0 = (int64_t)h * (p.nope_dim + p.v_dim);
    const int esz = WF32 ? 4 : 2;
#pragma unroll 4
    for (int d = wave; d < p.nope_dim; d += LT / 64) {
        const char* wr = (const char*)p.w + (row0 + d) * p.w_rs * esz + 16 * lane * CPL;
        const float qd = qs[d];
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const u32x4 wv = __builtin_nontemporal_load((const u32x4*)(wr + 16 * u));
#pragma unroll
            for (int k = 0; k < VPC; ++k) {
                const float wk = WF32 ? __uint_as_float(wv[k]) : __uint_as_float(k & 1 ? wv[k >> 1] & 0xffff0000u : wv[k >> 1] << 16);
                acc[u * VPC + k] = fmaf(qd, wk, acc[u * VPC + k]);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) part[wave][8 * lane + k] = acc[k];
    __syncthreads();
    uint16_t* out = p.q_lat + (int64_t)h * p.q_lat_head_stride;
    for (int c = tid; c < 512; c += LT) {
        const float v = (part[0][c] + part[1][c]) + (part[2][c] + part[3][c]);
        out[c] = f32_to_bf16_bits(v);
    }
}

// out[i] = bf16(x[i] * sigmoid(g[i])), MLA.swift:209-211 as its own stage
__global__ void __launch_bounds__(LT) gate_mul_kernel(const uint16_t* x, const uint16_t* g, int64_t n, uint16_t* out) {
    for (int64_t i = (int64_t)blockIdx.x * LT + threadIdx.x; i < n; i += (int64_t)gridDim.x * LT) {
        const float gv = bf16_bits_to_f32(g[i]);
        out[i] = f32_to_bf16_bits(bf16_bits_to_f32(x[i]) * (1.f / (1.f + __builtin_amdgcn_exp2f(-gv * 1.4426950408889634f))));
    }
}

}  // namespace

hipError_t launch_gate_mul(const uint16_t* x, const uint16_t* g, int64_t n, uint16_t* out, hipStream_t st) {
    const int64_t blocks = (n + LT - 1) / LT;
    hipLaunchKernelGGL(gate_mul_kernel, dim3((unsigned)(blocks < 1024 ? (blocks > 0 ? blocks : 1) : 1024)), dim3(LT), 0,
                       st, x, g, n, out);
    return hipGetLastError();
}

int dense_gemv_tokens_per_tile(int in, int m, bool x_f32) {
    const int cap = DENSE_STAGE_BYTES / (in * (x_f32 ? 4 : 2));
    return max(1, min(min(m, cap > 0 ? cap : 1), MAX_GEMV_TOKENS));
}

template <bool WF32, bool XF32>
static hipError_t launch_gemv(const DenseGemvParams& p, bool staged, dim3 grid, size_t lds, hipStream_t st) {
    if (staged) {
        if (lds > 65536) {
            const hipError_t e = hipFuncSetAttribute((const void*)dense_gemv_kernel<WF32, XF32, true>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL((dense_gemv_kernel<WF32, XF32, true>), grid, dim3(LT), lds, st, p);
    } else {
        hipLaunchKernelGGL((dense_gemv_kernel<WF32, XF32, false>), grid, dim3(LT), 0, st, p);
    }
    return hipGetLastError();
}

hipError_t launch_dense_gemv(DenseGemvParams p, bool staged, int cus, hipStream_t st) {
    const int vpc = p.w_f32 ? 4 : 8;
    const int chunks = p.in / vpc;
    int tpr = 64;
    while (tpr > 1 && tpr * 4 > chunks) tpr >>= 1;
    p.tpr = tpr;
    const int rows_per_step = (LT / 64) * (64 / tpr);
    const int64_t steps = (p.out_rows + rows_per_step - 1) / rows_per_step;
    const int64_t max_wg = 2 * (int64_t)cus;
    const int64_t wg = steps < max_wg ? steps : max_wg;
    p.steps_per_wg = (int)((steps + wg - 1) / wg);
    const int64_t grid_x = (steps + p.steps_per_wg - 1) / p.steps_per_wg;
    p.mt = staged ? dense_gemv_tokens_per_tile(p.in, p.m, p.x_f32) : 1;
    const int grid_y = (p.m + p.mt - 1) / p.mt;
    const size_t lds = staged ? (size_t)p.mt * p.in * (p.x_f32 ? 4 : 2) : 0;
    const dim3 grid((unsigned)grid_x, (unsigned)grid_y);
    if (p.w_f32)
        return p.x_f32 ? launch_gemv<true, true>(p, staged, grid, lds, st) : launch_gemv<true, false>(p, staged, grid, lds, st);
    return p.x_f32 ? launch_gemv<false, true>(p, staged, grid, lds, st) : launch_gemv<false, false>(p, staged, grid, lds, st);
}

hipError_t launch_dense_absorb(const DenseAbsorbParams& p, hipStream_t st) {
    if (p.w_f32)
        hipLaunchKernelGGL(dense_absorb_kernel<true>, dim3(p.heads), dim3(LT), 0, st, p);
    else
        hipLaunchKernelGGL(dense_absorb_kernel<false>, dim3(p.heads), dim3(LT), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
