// Lightning-index scores on gfx950 (DeepSeekV4LightningIndexer.scores,
// DeepSeekV4Attention.swift:530-549):
//   scores[s][t] = sum_h w[s][h] * max(q[s][h] . k[t], 0)
// perHead is the GEMM Q . K^T (heads x keys per query token), then a ReLU
// and a weighted sum over heads.  The keys dominate the bytes (T x D), so
// the kernel streams them once; Q (H x D per token) and the weights are
// small and sit in registers.
//
// MFMA kernel (bf16 q and keys, D = 128, H = 16..64 in steps of 16): one
// 256-thread workgroup per (128 keys, token s); each wave takes 32 keys as
// two 16-key tiles.  v_mfma_f32_16x16x32_bf16 with A = Q (row = head, lane
// l holds head 16ht + l%16, dims 32ks + 8(l/16)..+7) and B = K^T (column =
// key, the same dims), so D[head][key] leaves each lane with key l%16 and
// heads 4(l/16)+0..3 of every 16-head tile: the ReLU and the head weights
// apply in the lane, and the sum over heads ends with two permlane swaps.
// Keys load through a buffer descriptor: a key past T reads zeros and is
// not written.  fp32 accumulation; the head order of the sum differs from
// the reference's, so scores match it to rounding, not bits.
//
// Generic kernel (any D, H, f32 or bf16 inputs): one thread per (s, t),
// the dot summed over d in order and the heads in order.
#include "mr_kernels.hpp"

namespace mr {

namespace {

__device__ __forceinline__ float ix_ld(const void* p, int f32, int64_t i) {
    return f32 ? ((const float*)p)[i] : bf16_bits_to_f32(((const uint16_t*)p)[i]);
}

// max(x, 0) with NaN kept (MLX maximum propagates NaN; the selection that
// consumes the scores reports it)
__device__ __forceinline__ float relu_nan(float x) { return x > 0.f ? x : (x != x ? x : 0.f); }

constexpr int IX_KEYS = 128;  // keys per workgroup
constexpr int IX_KS = 4;      // 32-dim MFMA steps: D = 128

template <int HT>
__global__ void __launch_bounds__(256) indexer_scores_mfma(IndexerParams p) {
    const int s = blockIdx.y;
    const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int key0 = blockIdx.x * IX_KEYS + 32 * w;
    // Q rows of this token: A operands for every (head tile, k step)
    const uint16_t* q = (const uint16_t*)p.q + (int64_t)s * p.q_ss;
    bf16x8 qa[HT][IX_KS];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
        for (int ks = 0; ks < IX_KS; ++ks)
            qa[ht][ks] = *(const bf16x8*)(q + (int64_t)(16 * ht + (l & 15)) * p.q_hs + 32 * ks + 8 * (l >> 4));
    // head weights of the D rows this lane holds: head 16ht + 4(l/16) + i
    float wv[HT][4];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht)
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[ht][i] = ix_ld(p.w, p.w_f32, (int64_t)s * p.w_ss + 16 * ht + 4 * (l >> 4) + i);
    // keys: B operands of both 16-key tiles
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc((void*)p.k, 0, (int)p.k_bytes, 0x00020000);
    bf16x8 kb[2][IX_KS];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        const int key = key0 + 16 * kt + (l & 15);
        const uint32_t base = key < p.T ? (uint32_t)key * (uint32_t)(p.k_rs * 2) + 16u * (l >> 4) : 0x80000000u;
#pragma unroll
        for (int ks = 0; ks < IX_KS; ++ks)
            kb[kt][ks] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(kres, base + 64u * ks, 0, 0));
    }
    f32x4 acc[2][HT];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) acc[kt][ht] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < IX_KS; ++ks)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int ht = 0; ht < HT; ++ht) acc[kt][ht] = mfma16(qa[ht][ks], kb[kt][ks], acc[kt][ht]);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        float sc = 0.f;
#pragma unroll
        for (int ht = 0; ht < HT; ++ht)
#pragma unroll
            for (int i = 0; i < 4; ++i) sc = fmaf(wv[ht][i], relu_nan(acc[kt][ht][i]), sc);
        sc = xor32_sum(xor16_sum(sc));  // the four lane groups hold the other heads
        const int key = key0 + 16 * kt + l;
        if (l < 16 && key < p.T) p.out[(int64_t)s * p.out_ss + key] = sc;
    }
}

__global__ void __launch_bounds__(256) indexer_scores_generic(IndexerParams p) {
    const int64_t st = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (st >= (int64_t)p.S * p.T) return;
    const int64_t s = st / p.T, t = st - s * p.T;
    float acc = 0.f;
    for (int h = 0; h < p.H; ++h) {
        float d = 0.f;
        for (int i = 0; i < p.D; ++i)
            d = fmaf(ix_ld(p.q, p.q_f32, s * p.q_ss + (int64_t)h * p.q_hs + i), ix_ld(p.k, p.k_f32, t * p.k_rs + i), d);
        acc = fmaf(relu_nan(d), ix_ld(p.w, p.w_f32, s * p.w_ss + h), acc);
    }
    p.out[s * p.out_ss + t] = acc;
}

}  // namespace

bool indexer_mfma_ok(const IndexerParams& p) {
    return !p.q_f32 && !p.k_f32 && p.D == 128 && p.H % 16 == 0 && p.H <= 64 && p.q_hs % 8 == 0 && p.q_ss % 8 == 0 &&
           p.k_rs % 8 == 0 && ((uintptr_t)p.q & 15) == 0 && ((uintptr_t)p.k & 15) == 0 &&
           (int64_t)p.T * p.k_rs * 2 < (int64_t(1) << 31);
}

hipError_t launch_indexer_scores(const IndexerParams& q, hipStream_t st) {
    if (q.T == 0) return hipSuccess;
    IndexerParams p = q;
    if (indexer_mfma_ok(p)) {
        p.k_bytes = (uint32_t)((int64_t)(p.T - 1) * p.k_rs * 2 + 256);  // through the last key's 128 dims
        const dim3 grid((unsigned)((p.T + IX_KEYS - 1) / IX_KEYS), (unsigned)p.S);
        switch (p.H / 16) {
            case 1: hipLaunchKernelGGL(indexer_scores_mfma<1>, grid, dim3(256), 0, st, p); break;
            case 2: hipLaunchKernelGGL(indexer_scores_mfma<2>, grid, dim3(256), 0, st, p); break;
            case 3: hipLaunchKernelGGL(indexer_scores_mfma<3>, grid, dim3(256), 0, st, p); break;
            default: hipLaunchKernelGGL(indexer_scores_mfma<4>, grid, dim3(256), 0, st, p); break;
        }
        return hipGetLastError();
    }
    const int64_t n = (int64_t)p.S * p.T;
    hipLaunchKernelGGL(indexer_scores_generic, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
