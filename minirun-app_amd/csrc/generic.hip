// MLA attention at any widths, for the model configurations the fixed-width
// kernels do not take (decode.hip: kv_rank 512, rope 64 or 0; prefill.hip:
// qk_nope 128, qk_rope 64, v_head 128, kv_rank 512), such as the reference's
// synthetic K3 artifact (kv_lora 16, nope 8, rope 4, v 8).  The same
// computations, in fp32 throughout (no bf16 rounding of P or of the
// up-projected keys and values):
//   decode  (K3MLA.forward absorbed branch, MLA.swift:174-197; sparse form
//           DeepSeekV4SparseAttention.expressingBatched,
//           DeepSeekV4Attention.swift:861-920, sinks :908-913): per (batch,
//           head), s_n = (q_lat . c_n[0:R] + q_rope . k_n) * scale over the
//           selected rows, out = softmax(s) . c[0:R], the sink in the max and
//           the denominator only, an empty selection giving zeros.
//   prefill (K3MLA.forward eager branch, MLA.swift:159-168,198-206, expand
//           :231-245, causal mask :257-275): K_h[p] = [latent[p] . W_UK_h^T
//           ++ rope_keys[p]], V_h[p] = latent[p] . W_UV_h^T, query i sees keys
//           0 .. P - T + i.
// One workgroup per (batch or token, head) runs a flash loop over chunks of
// 256 keys: thread t scores key t of the chunk, the chunk's max and sum
// meet in LDS, and each thread then accumulates its output columns over
// the chunk's keys (a key's row is read by consecutive threads, so the
// reads of one key are coalesced).  Correctness path for small and unusual
// widths: every element is a 2-byte load, no alignment beyond the element's.
#include "mr_kernels.hpp"

namespace mr {

namespace {

constexpr int AN_T = 256;  // threads per workgroup, keys per chunk
constexpr float NEG_INF_ANY = -__builtin_huge_valf();
constexpr int AN_ACC = 8;  // output columns per thread: widths up to 2048
static_assert(AN_T * AN_ACC >= ANY_MAX_RANK, "output columns per thread");

__device__ __forceinline__ float bfv(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }

// block-wide max / sum of one value per thread (every thread gets the result)
__device__ __forceinline__ float an_block_max(float v, float* red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float an_block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Flash loop state of one (query, head): running max m (base 2), sum l and
// the thread's output columns d = threadIdx.x + AN_T * j.
struct AnState {
    float m, l;
    float acc[AN_ACC];
};

// One chunk: s = this thread's scaled score (-inf for no key), key = its
// key id (-1 for none); val(key, d) reads value column d of a key.
template <typename Val>
__device__ __forceinline__ void an_chunk(AnState& st, float s, int key, int ncols, float* p_s, int* k_s, float* red,
                                         Val val) {
    const float cm = an_block_max(s, red);
    const float m_new = fmaxf(st.m, cm);
    if (m_new == NEG_INF_ANY) return;  // no key so far (uniform: cm is block-wide)
    const float alpha = exp2f(st.m - m_new);  // 0 while st.m is -inf (st.l and acc are 0 then)
    const float pv = key >= 0 ? exp2f(s - m_new) : 0.f;
    p_s[threadIdx.x] = pv;
    k_s[threadIdx.x] = key;
    const float ls = an_block_sum(pv, red);  // its barriers also publish p_s, k_s
    st.l = st.l * alpha + ls;
    st.m = m_new;
#pragma unroll
    for (int j = 0; j < AN_ACC; ++j) {
        const int d = threadIdx.x + AN_T * j;
        if (d >= ncols) break;
        float a = st.acc[j] * alpha;
        for (int t = 0; t < AN_T; ++t) {
            const int k = k_s[t];
            if (k >= 0) a = fmaf(p_s[t], val(k, d), a);
        }
        st.acc[j] = a;
    }
    __syncthreads();  // p_s, k_s are rewritten by the next chunk
}

// out column d of the state, with the optional sink (base 2) in the max and
// the denominator; an empty selection gives zeros
__device__ __forceinline__ void an_store(const AnState& st, bool has_sink, float sink2, int ncols, void* out,
                                         int out_f32) {
    float num = 1.f, den = st.l;
    if (st.m == NEG_INF_ANY) {
        num = 0.f;
        den = 1.f;
    } else if (has_sink) {
        const float M = fmaxf(st.m, sink2);
        num = exp2f(st.m - M);
        den = st.l * num + exp2f(sink2 - M);
    }
    const float sc = num / den;
#pragma unroll
    for (int j = 0; j < AN_ACC; ++j) {
        const int d = threadIdx.x + AN_T * j;
        if (d >= ncols) break;
        const float v = st.acc[j] * sc;
        if (out_f32)
            ((float*)out)[d] = v;
        else
            ((uint16_t*)out)[d] = f32_to_bf16_bits(v);
    }
}

__global__ void __launch_bounds__(AN_T) mla_decode_any_kernel(AnyDecodeParams p) {
    __shared__ float q_s[ANY_MAX_RANK + ANY_MAX_ROPE];
    __shared__ float p_s[AN_T];
    __shared__ int k_s[AN_T];
    __shared__ float red[AN_T / 64];
    const int b = blockIdx.x / p.heads, h = blockIdx.x - b * p.heads;
    const uint16_t* ql = p.q_lat + (int64_t)b * p.q_lat_bs + (int64_t)h * p.q_lat_hs;
    for (int d = threadIdx.x; d < p.R; d += AN_T) q_s[d] = bfv(ql, d);
    if (p.DR) {
        const uint16_t* qr = p.q_rope + (int64_t)b * p.q_rope_bs + (int64_t)h * p.q_rope_hs;
        for (int d = threadIdx.x; d < p.DR; d += AN_T) q_s[p.R + d] = bfv(qr, d);
    }
    __syncthreads();
    const uint16_t* lat = p.latent + (int64_t)b * p.lat_bs;
    const uint16_t* rop = p.DR ? p.rope + (int64_t)b * p.rope_bs : nullptr;
    const int32_t* ind = p.indices ? p.indices + (int64_t)b * p.n_idx : nullptr;
    const int n = ind ? p.n_idx : p.n_ctx;
    AnState st;
    st.m = NEG_INF_ANY;
    st.l = 0.f;
#pragma unroll
    for (int j = 0; j < AN_ACC; ++j) st.acc[j] = 0.f;
    for (int c0 = 0; c0 < n; c0 += AN_T) {
        const int i = c0 + threadIdx.x;
        int key = -1;
        if (i < n) {
            key = ind ? ind[i] : i;
            if (key < 0 || key >= p.n_ctx) key = -1;  // -1 entries (and, unchecked, bad ones) are skipped
        }
        float s = NEG_INF_ANY;
        if (key >= 0) {
            const uint16_t* cl = lat + (int64_t)key * p.lat_rs;
            float a = 0.f;
            for (int d = 0; d < p.R; ++d) a = fmaf(q_s[d], bfv(cl, d), a);
            if (p.DR) {
                const uint16_t* cr = rop + (int64_t)key * p.rope_rs;
                for (int d = 0; d < p.DR; ++d) a = fmaf(q_s[p.R + d], bfv(cr, d), a);
            }
            s = a * p.scale_log2;
        }
        an_chunk(st, s, key, p.R, p_s, k_s, red,
                 [&](int k, int d) { return bfv(lat, (int64_t)k * p.lat_rs + d); });
    }
    char* out = (char*)p.out + ((int64_t)b * p.out_bs + (int64_t)h * p.out_hs) * (p.out_f32 ? 4 : 2);
    an_store(st, p.sinks != nullptr, p.sinks ? p.sinks[h] * 1.4426950408889634f : 0.f, p.R, out, p.out_f32);
}

// kv[h][pos][e] = latent[pos] . kv_b[h * (nope + v) + e] (fp32), one
// workgroup per (pos, head), the latent row staged in LDS
__global__ void __launch_bounds__(AN_T) upproj_any_kernel(AnyPrefillParams p) {
    __shared__ float l_s[ANY_MAX_RANK];
    const int pos = blockIdx.x / p.H, h = blockIdx.x - pos * p.H;
    const uint16_t* lr = p.latent + (int64_t)pos * p.lat_rs;
    for (int c = threadIdx.x; c < p.R; c += AN_T) l_s[c] = bfv(lr, c);
    __syncthreads();
    const int W = p.NOPE + p.V;
    float* dst = p.kv + ((int64_t)h * p.P + pos) * W;
    for (int e = threadIdx.x; e < W; e += AN_T) {
        const uint16_t* wr = p.kv_b + ((int64_t)h * W + e) * p.kvb_rs;
        float a = 0.f;
        for (int c = 0; c < p.R; ++c) a = fmaf(l_s[c], bfv(wr, c), a);
        dst[e] = a;
    }
}

// one workgroup per (query token, head): keys 0 .. P - T + t
__global__ void __launch_bounds__(AN_T) prefill_any_kernel(AnyPrefillParams p) {
    __shared__ float q_s[ANY_MAX_NOPE + ANY_MAX_ROPE];
    __shared__ float p_s[AN_T];
    __shared__ int k_s[AN_T];
    __shared__ float red[AN_T / 64];
    const int t = blockIdx.x / p.H, h = blockIdx.x - t * p.H;
    const uint16_t* qp = p.q + (int64_t)t * p.q_ts + (int64_t)h * p.q_hs;
    for (int d = threadIdx.x; d < p.NOPE + p.DR; d += AN_T) q_s[d] = bfv(qp, d);
    __syncthreads();
    const int W = p.NOPE + p.V;
    const float* kvh = p.kv + (int64_t)h * p.P * W;
    const int n = p.P - p.T + t + 1;  // visible keys
    AnState st;
    st.m = NEG_INF_ANY;
    st.l = 0.f;
#pragma unroll
    for (int j = 0; j < AN_ACC; ++j) st.acc[j] = 0.f;
    for (int c0 = 0; c0 < n; c0 += AN_T) {
        const int key = c0 + threadIdx.x < n ? c0 + threadIdx.x : -1;
        float s = NEG_INF_ANY;
        if (key >= 0) {
            const float* kr = kvh + (int64_t)key * W;
            float a = 0.f;
            for (int d = 0; d < p.NOPE; ++d) a = fmaf(q_s[d], kr[d], a);
            const uint16_t* rr = p.rope + (int64_t)key * p.rope_rs;
            for (int d = 0; d < p.DR; ++d) a = fmaf(q_s[p.NOPE + d], bfv(rr, d), a);
            s = a * p.scale_log2;
        }
        an_chunk(st, s, key, p.V, p_s, k_s, red,
                 [&](int k, int d) { return kvh[(int64_t)k * W + p.NOPE + d]; });
    }
    char* out = (char*)p.out + ((int64_t)t * p.out_ts + (int64_t)h * p.out_hs) * (p.out_f32 ? 4 : 2);
    an_store(st, false, 0.f, p.V, out, p.out_f32);
}

}  // namespace

hipError_t launch_mla_decode_any(const AnyDecodeParams& p, hipStream_t st) {
    hipLaunchKernelGGL(mla_decode_any_kernel, dim3((unsigned)(p.batch * p.heads)), dim3(AN_T), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_mla_prefill_any(const AnyPrefillParams& p, hipEvent_t const* events, hipStream_t st) {
    hipError_t e;
    if (events && (e = hipEventRecord(events[0], st)) != hipSuccess) return e;
    hipLaunchKernelGGL(upproj_any_kernel, dim3((unsigned)(p.P * p.H)), dim3(AN_T), 0, st, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[1], st)) != hipSuccess) return e;
    hipLaunchKernelGGL(prefill_any_kernel, dim3((unsigned)(p.T * p.H)), dim3(AN_T), 0, st, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return events ? hipEventRecord(events[2], st) : hipSuccess;
}

}  // namespace mr
