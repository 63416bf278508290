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
    // the token's queries (16 HT rows of 128 dims, rows padded by 16 bytes so
    // the fragment reads spread over the banks) and head weights, staged
    // once per workgroup: every wave needs all of them
    __shared__ __attribute__((aligned(16))) uint16_t qs[16 * HT][128 + 8];
    __shared__ float hw[16 * HT];
    const int s = blockIdx.y;
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const int key0 = blockIdx.x * IX_KEYS + 32 * w;
    // queries first, then the keys: the staging waits for the queries only
    // (loads complete in order), the keys stay in flight across the barrier
    const uint16_t* q = (const uint16_t*)p.q + (int64_t)s * p.q_ss;
    static_assert(16 * HT * 16 <= 4 * 256, "query chunks per thread");
    bf16x8 qc[HT];
#pragma unroll
    for (int i = 0; i < HT; ++i) {
        const int c = t + 256 * i, r = c >> 4, k = c & 15;  // 16-byte chunk k of query row r
        qc[i] = *(const bf16x8*)(q + (int64_t)r * p.q_hs + 8 * k);
    }
    // the head weight of thread t < 16 HT: one unconditional dword load (the
    // dword holding a bf16 weight, through a descriptor that bounds the row
    // set), its half picked once the keys are issued
    const uint32_t esz = p.w_f32 ? 4u : 2u;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.w, 0, (int)(((int64_t)(p.S - 1) * p.w_ss + p.H) * esz), 0x00020000);
    const uint32_t wa = (uint32_t)(((int64_t)s * p.w_ss + min(t, 16 * HT - 1)) * esz);
    const uint32_t wraw = __builtin_amdgcn_raw_buffer_load_b32(wres, wa & ~3u, 0, 0);
    asm volatile("" ::: "memory");  // the key loads issue after the query and weight loads
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
#pragma unroll
    for (int i = 0; i < HT; ++i) {
        const int c = t + 256 * i;
        *(bf16x8*)&qs[c >> 4][8 * (c & 15)] = qc[i];
    }
    if (t < 16 * HT)
        hw[t] = p.w_f32 ? __uint_as_float(wraw) : __uint_as_float((wa & 2u) ? wraw & 0xffff0000u : wraw << 16);
    lds_barrier();
    // A operands for every (head tile, k step), and the head weights of the
    // D rows this lane holds: head 16ht + 4(l/16) + i
    bf16x8 qa[HT][IX_KS];
    float wv[HT][4];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
#pragma unroll
        for (int ks = 0; ks < IX_KS; ++ks) qa[ht][ks] = *(const bf16x8*)&qs[16 * ht + (l & 15)][32 * ks + 8 * (l >> 4)];
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[ht][i] = hw[16 * ht + 4 * (l >> 4) + i];
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
