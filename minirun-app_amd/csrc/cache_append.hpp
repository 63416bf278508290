// Latent-cache append of one token as a device function, shared by the
// append kernel and the launches that carry the append as one extra
// workgroup (MLA.swift:142-157 with the rotary tail of
// DeepSeekV4CompressedAttention.swift:676-694): the kv_a row
// [kv_rank latent ++ rope_dim key] -> RMSNorm(latent) * w -> bf16 cache row
// (start_row + t)[0:kv_rank]; the key tail rotated at its position (or kept
// as it is for NoPE) -> bf16 [kv_rank : kv_rank + rope_dim].
#pragma once

#include "mr_kernels.hpp"

namespace mr {

// All 256 threads of the workgroup call it; sh holds 4 floats.
__device__ inline void cache_append_row(const CacheAppendParams& p, int64_t t, float* sh) {
#pragma clang fp contract(off)  // the rotary and the norm round as written
    auto ld = [](const void* q, int f32, int64_t i) {
        return f32 ? ((const float*)q)[i] : bf16_bits_to_f32(((const uint16_t*)q)[i]);
    };
    float ss = 0.f;
    for (int i = threadIdx.x; i < p.kv_rank; i += 256) {
        const float v = ld(p.kv, p.kv_f32, t * p.kv_stride + i);
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
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
        if (!p.cos_t) {  // NoPE (MLA.swift:5-13): the shared key slice is kept as it is
            rk[2 * i] = f32_to_bf16_bits(e);
            rk[2 * i + 1] = f32_to_bf16_bits(o);
            continue;
        }
        const float c = p.cos_t[t * half + i];
        const float s = p.sin_t[t * half + i];
        rk[2 * i] = f32_to_bf16_bits(sub_rn(mul_rn(e, c), mul_rn(o, s)));
        rk[2 * i + 1] = f32_to_bf16_bits(add_rn(mul_rn(e, s), mul_rn(o, c)));
    }
}

}  // namespace mr
