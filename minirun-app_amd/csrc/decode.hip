// Absorbed-latent MLA decode and index-driven sparse decode for gfx950.
//
// Computes, per (batch b, head h), over the selected cache rows c_n:
//   s_n   = (q_lat[h] . c_n[0:R] + q_rope[h] . c_n[R:R+dr]) * scale
//   out_h = sum_n softmax(s)_n * c_n[0:R]              (R = 512)
// which is the absorbed branch of K3MLA.forward (MLA.swift:188-196) and, with
// an index list and optional sinks, DeepSeekV4SparseAttention.expressingBatched
// (DeepSeekV4Attention.swift:861-920) with K = row[0:R+dr], V = row[0:R].
//
// Decomposition (one workgroup per CU, 4 waves):
//   grid unit   = (batch, context split) x head group of 32 heads
//   blockIdx    -> XCD-aware: the head groups of one unit share blockIdx % 8,
//                  so they run on one XCD and read the same rows through its L2
//   sub-chunk   = 64 cache rows, staged global -> VGPR -> LDS, double buffered,
//                 LDS rows padded to DK*2+16 bytes (conflict-free MFMA reads)
//   QK          = 16x16x32 bf16 MFMA, A = cache rows (LDS), B = Q (VGPRs);
//                 wave w scores 16 rows x 32 heads
//   softmax     = online, base-2, the running max shared by the 4 waves
//   PV          = 16x16x32 bf16 MFMA, A = P (LDS, bf16), B = cache rows read
//                 transposed with ds_read_b64_tr_b16; wave w owns 128 of the
//                 512 output columns for all 32 heads
//   epilogue    = unnormalised O, running max m and sum l per (unit, head)
//                 into the workspace; mla_combine merges the splits (and the
//                 sink term) and writes bf16/f32.
#include "mr_kernels.hpp"

namespace mr {

namespace {

constexpr int R = 512;
constexpr int ROWS = 64;      // rows per sub-chunk
constexpr int HG = 32;        // heads per workgroup
constexpr int THREADS = 256;  // 4 waves
constexpr int PSTR = 144;     // bytes per head row of P (64 bf16 + 16 pad)
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LOG2E = 1.4426950408889634f;

template <int DR>
struct Geo {
    static constexpr int DK = R + DR;
    static constexpr int KS = DK / 32;             // MFMA k-steps for QK
    static constexpr int CPR = DK / 8;             // 16-byte chunks per row
    static constexpr int LROW = DK * 2 + 16;       // padded LDS row, bytes
    static constexpr int BUF = ROWS * LROW;        // one sub-chunk buffer
    static constexpr int NCH = ROWS * CPR / THREADS;  // chunks per thread
    static_assert(ROWS * CPR % THREADS == 0, "chunking");
};

// row of the 64-row sub-chunk that MFMA A-row `a` (0..15) of wave w scores:
// rows 16w + {0,2,4,6}, {1,3,5,7}, {8,..14}, {9,..15} for a/4 = 0..3.  The
// order makes the P write contiguous and the transposed PV reads
// bank-conflict free (see rho() below).
__device__ __forceinline__ int sigma_row(int w, int a) {
    int g = a >> 2;
    return 16 * w + 8 * (g >> 1) + (g & 1) + 2 * (a & 3);
}

template <int DR, bool GATHER, bool TR>
__global__ void __launch_bounds__(THREADS, 1) mla_decode_split(DecodeParams p) {
    using G = Geo<DR>;
    __shared__ __attribute__((aligned(16))) char cbuf[2 * G::BUF];
    __shared__ __attribute__((aligned(16))) char pbuf[HG * PSTR];
    __shared__ float red[4][HG];
    __shared__ __attribute__((aligned(16))) float alpha_s[HG];
    __shared__ int32_t idx_s[GATHER ? MAX_GATHER_ROWS : 1];

    const int bid = blockIdx.x;
    const int xcd = bid & 7;
    const int qb = bid >> 3;
    const int hg = qb % p.head_groups;
    const int unit = (qb / p.head_groups) * 8 + xcd;
    if (unit >= p.batch * p.splits) return;
    const int b = unit / p.splits;
    const int split = unit % p.splits;
    const int row_begin = split * p.rows_per_split;
    const int row_end = min(row_begin + p.rows_per_split, p.n_rows);
    const int nrows = max(row_end - row_begin, 0);
    const int nsub = (nrows + ROWS - 1) / ROWS;

    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int l = tid & 63;
    const int lg = l >> 4;
    const int lc = l & 15;

    const uint16_t* lat = p.latent + (int64_t)b * p.lat_bs;
    const uint16_t* rop = DR ? p.rope + (int64_t)b * p.rope_bs : nullptr;

    if (GATHER) {
        const int32_t* ind = p.indices + (int64_t)b * p.n_idx;
        for (int i = tid; i < nrows; i += THREADS) {
            int32_t v = ind[row_begin + i];
            bool ok = v >= 0 && v < p.n_ctx;
            if (!ok && v != -1 && p.err_flag) atomicOr(p.err_flag, 1);
            idx_s[i] = ok ? v : -1;
        }
        __syncthreads();
    }

    // ---- Q for this head group, B-operand layout: head 16T+lc, k = 32ks+8lg..+7
    bf16x8 qreg[G::KS][2];
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        const int h = hg * HG + 16 * T + lc;
        const bool hv = h < p.heads;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            const int d = 32 * ks + 8 * lg;
            u32x4 v = {0u, 0u, 0u, 0u};
            if (hv) {
                const uint16_t* src = d < R ? p.q_lat + (int64_t)b * p.q_lat_bs + (int64_t)h * p.q_lat_hs + d
                                            : p.q_rope + (int64_t)b * p.q_rope_bs + (int64_t)h * p.q_rope_hs + (d - R);
                v = *(const u32x4*)src;
            }
            qreg[ks][T] = __builtin_bit_cast(bf16x8, v);
        }
    }

    // ---- staging of one sub-chunk: global -> registers
    u32x4 stage[G::NCH];
    auto load_sub = [&](int s) {
        const int rbase = row_begin + s * ROWS;
#pragma unroll
        for (int k = 0; k < G::NCH; ++k) {
            const int c = tid + THREADS * k;
            const int row = c / G::CPR;
            const int cc = c - row * G::CPR;
            const int r = rbase + row;
            int src_row = r;
            bool ok = r < row_end;
            if (GATHER) {
                src_row = ok ? idx_s[r - row_begin] : -1;
                ok = src_row >= 0;
            }
            u32x4 v = {0u, 0u, 0u, 0u};
            if (ok) {
                const uint16_t* src = cc < R / 8 ? lat + (int64_t)src_row * p.lat_rs + cc * 8
                                                 : rop + (int64_t)src_row * p.rope_rs + (cc - R / 8) * 8;
                v = __builtin_nontemporal_load((const u32x4*)src);
            }
            stage[k] = v;
        }
    };
    auto store_sub = [&](int buf) {
        char* base = cbuf + buf * G::BUF;
#pragma unroll
        for (int k = 0; k < G::NCH; ++k) {
            const int c = tid + THREADS * k;
            const int row = c / G::CPR;
            const int cc = c - row * G::CPR;
            *(u32x4*)(base + row * G::LROW + cc * 16) = stage[k];
        }
    };
    auto row_valid = [&](int s, int r_local) -> bool {
        const int r = row_begin + s * ROWS + r_local;
        if (r >= row_end) return false;
        if (GATHER) return idx_s[r - row_begin] >= 0;
        return true;
    };

    f32x4 oacc[2][8];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int J = 0; J < 8; ++J) oacc[T][J] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {NEG_INF, NEG_INF};
    float l_run[2] = {0.f, 0.f};

    if (nsub > 0) {
        load_sub(0);
        store_sub(0);
        if (nsub > 1) load_sub(1);
    }

    const int arow = sigma_row(w, lc);
    const int lbase = 8 * (lg >> 1) + (lg & 1);  // sigma base of this lane group

    for (int s = 0; s < nsub; ++s) {
        const int cb = s & 1;
        const char* cur = cbuf + cb * G::BUF;
        __syncthreads();  // sub-chunk s in LDS; every wave is done with s-1

        // ---- QK: S[16 rows][32 heads]
        f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        const char* arow_p = cur + arow * G::LROW + 16 * lg;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            const bf16x8 a = *(const bf16x8*)(arow_p + 64 * ks);
            sacc[0] = mfma16(a, qreg[ks][0], sacc[0]);
            sacc[1] = mfma16(a, qreg[ks][1], sacc[1]);
        }

        float sv[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ok = row_valid(s, 16 * w + lbase + 2 * i);
#pragma unroll
            for (int T = 0; T < 2; ++T) sv[T][i] = ok ? sacc[T][i] * p.scale_log2 : NEG_INF;
        }
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            float mx = fmaxf(fmaxf(sv[T][0], sv[T][1]), fmaxf(sv[T][2], sv[T][3]));
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            if (lg == 0) red[w][16 * T + lc] = mx;
        }
        __syncthreads();

        // ---- running max, P, l
        const int kso = w >> 1;  // k-step of the PV product this wave's rows fall in
        const int kap = 8 * (2 * (w & 1) + (lg >> 1)) + 4 * (lg & 1);
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const int hh = 16 * T + lc;
            const float cm = fmaxf(fmaxf(red[0][hh], red[1][hh]), fmaxf(red[2][hh], red[3][hh]));
            const float m_new = fmaxf(m_run[T], cm);
            const float alpha = (m_run[T] == NEG_INF) ? 0.f : exp2f(m_run[T] - m_new);
            m_run[T] = m_new;
            float pv[4];
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pv[i] = (m_new == NEG_INF) ? 0.f : exp2f(sv[T][i] - m_new);
                psum += pv[i];
            }
            l_run[T] = l_run[T] * alpha + psum;
            u32x2 pk = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
            *(u32x2*)(pbuf + hh * PSTR + (32 * kso + kap) * 2) = pk;
            if (w == 0 && lg == 0) alpha_s[hh] = alpha;
        }
        __syncthreads();

        // ---- PV: O[32 heads][128w .. 128w+127] += P[32][64] . C[64][...]
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const f32x4 a4 = *(const f32x4*)(alpha_s + 16 * T + 4 * lg);
#pragma unroll
            for (int J = 0; J < 8; ++J) oacc[T][J] *= a4;
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bf16x8 pa[2];
#pragma unroll
            for (int T = 0; T < 2; ++T)
                pa[T] = *(const bf16x8*)(pbuf + (16 * T + lc) * PSTR + (32 * ks + 8 * lg) * 2);
            // rho(g, t, e) = 16(g/2) + 8(g%2) + 2e + t  (row inside the k-step)
            const int rrow = 32 * ks + 16 * (lg >> 1) + 8 * (lg & 1);
#pragma unroll
            for (int J = 0; J < 8; ++J) {
                const int v0 = 128 * w + 16 * J;
                bf16x8 bb;
                if (TR) {
                    const char* bp = cur + (rrow + 2 * (lc >> 2)) * G::LROW + (v0 + 4 * (lc & 3)) * 2;
                    const bf16x4 b0 = ds_read_tr16(bp);
                    const bf16x4 b1 = ds_read_tr16(bp + G::LROW);
                    bb = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
                } else {
                    uint16_t e[8];
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int q = 0; q < 4; ++q)
                            e[4 * t + q] = *(const uint16_t*)(cur + (rrow + 2 * q + t) * G::LROW + (v0 + lc) * 2);
                    u32x4 u;
#pragma unroll
                    for (int j = 0; j < 4; ++j) u[j] = e[2 * j] | ((uint32_t)e[2 * j + 1] << 16);
                    bb = __builtin_bit_cast(bf16x8, u);
                }
#pragma unroll
                for (int T = 0; T < 2; ++T) oacc[T][J] = mfma16(pa[T], bb, oacc[T][J]);
            }
        }

        // ---- next sub-chunk into the other buffer, prefetch the one after
        if (s + 1 < nsub) {
            store_sub(cb ^ 1);
            if (s + 2 < nsub) load_sub(s + 2);
        }
    }

    // ---- epilogue: l over lane groups and waves, then the partial record
#pragma unroll
    for (int T = 0; T < 2; ++T) {
        l_run[T] += __shfl_xor(l_run[T], 16);
        l_run[T] += __shfl_xor(l_run[T], 32);
    }
    __syncthreads();
#pragma unroll
    for (int T = 0; T < 2; ++T)
        if (lg == 0) red[w][16 * T + lc] = l_run[T];
    __syncthreads();

    const int64_t rec = (int64_t)unit * p.h_pad + hg * HG;
    if (w == 0 && lg == 0) {
#pragma unroll
        for (int T = 0; T < 2; ++T) {
            const int hh = 16 * T + lc;
            const float lt = red[0][hh] + red[1][hh] + red[2][hh] + red[3][hh];
            p.ws_ml[(rec + hh) * 2 + 0] = m_run[T];
            p.ws_ml[(rec + hh) * 2 + 1] = lt;
        }
    }
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float* dst = p.ws_o + (rec + 16 * T + 4 * lg + i) * R + 128 * w + lc;
#pragma unroll
            for (int J = 0; J < 8; ++J) dst[16 * J] = oacc[T][J][i];
        }
}

// Merge the split partials of one (batch, head): 256 threads, 2 blocks per
// head cover the 512 output columns.
__global__ void __launch_bounds__(256) mla_combine(CombineParams p) {
    const int bh = blockIdx.x;
    const int b = bh / p.heads;
    const int h = bh % p.heads;
    const int v = blockIdx.y * 256 + threadIdx.x;
    float M = NEG_INF;
    for (int s = 0; s < p.splits; ++s) M = fmaxf(M, p.ws_ml[(((int64_t)(b * p.splits + s)) * p.h_pad + h) * 2]);
    const bool any = M != NEG_INF;
    float sink2 = NEG_INF;
    if (p.sinks) {
        sink2 = p.sinks[h] * LOG2E;
        M = fmaxf(M, sink2);
    }
    float L = 0.f, acc = 0.f;
    for (int s = 0; s < p.splits; ++s) {
        const int64_t rec = ((int64_t)(b * p.splits + s)) * p.h_pad + h;
        const float ms = p.ws_ml[rec * 2];
        if (ms == NEG_INF) continue;
        const float wgt = exp2f(ms - M);
        L += p.ws_ml[rec * 2 + 1] * wgt;
        acc += wgt * p.ws_o[rec * R + v];
    }
    if (p.sinks) L += exp2f(sink2 - M);
    const float r = any ? acc / L : 0.f;
    const int64_t o = (int64_t)b * p.out_bs + (int64_t)h * p.out_hs + v;
    if (p.out_f32)
        ((float*)p.out)[o] = r;
    else
        ((uint16_t*)p.out)[o] = f32_to_bf16_bits(r);
}

template <int DR, bool GATHER, bool TR>
hipError_t launch_split(const DecodeParams& p, int grid, hipStream_t st) {
    hipLaunchKernelGGL((mla_decode_split<DR, GATHER, TR>), dim3(grid), dim3(THREADS), 0, st, p);
    return hipGetLastError();
}

// One workgroup per token b.  Range errors: smallest offending position.
// Duplicates: keys (value << 32 | position) sorted in LDS; every entry of an
// equal-value run after its first is a repeat; the smallest such position is
// the one the reference's in-order scan stops at.
__global__ void __launch_bounds__(256) validate_indices_kernel(const int32_t* indices, int32_t n_idx,
                                                               int32_t n_rows, int32_t npad,
                                                               int32_t* result) {
    extern __shared__ uint64_t keys[];
    __shared__ int32_t range_pos, dup_pos;
    const int b = blockIdx.x;
    const int32_t* ind = indices + (int64_t)b * n_idx;
    if (threadIdx.x == 0) {
        range_pos = 0x7fffffff;
        dup_pos = 0x7fffffff;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < npad; i += blockDim.x) {
        uint64_t k = ~0ull;
        if (i < n_idx) {
            const int32_t v = ind[i];
            if (v != -1) {
                if (v < 0 || v >= n_rows)
                    atomicMin(&range_pos, i);
                else
                    k = ((uint64_t)(uint32_t)v << 32) | (uint32_t)i;
            }
        }
        keys[i] = k;
    }
    __syncthreads();
    for (int size = 2; size <= npad; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < npad; i += blockDim.x) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    const uint64_t a = keys[i], c = keys[j];
                    if ((a > c) == up) {
                        keys[i] = c;
                        keys[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int i = threadIdx.x + 1; i < npad; i += blockDim.x) {
        const uint64_t k = keys[i];
        if (k != ~0ull && (k >> 32) == (keys[i - 1] >> 32)) atomicMin(&dup_pos, (int32_t)(k & 0xffffffffu));
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        result[2 * b] = range_pos;
        result[2 * b + 1] = dup_pos;
    }
}

}  // namespace

hipError_t launch_validate_indices(const int32_t* indices, int32_t batch, int32_t n_idx, int32_t n_rows,
                                   int32_t* result, hipStream_t st) {
    int npad = 1;
    while (npad < n_idx) npad <<= 1;
    hipLaunchKernelGGL(validate_indices_kernel, dim3(batch), dim3(256), npad * sizeof(uint64_t), st, indices,
                       n_idx, n_rows, npad, result);
    return hipGetLastError();
}

int decode_head_groups(int heads) { return (heads + HG - 1) / HG; }

hipError_t launch_mla_decode(const DecodeParams& p, const CombineParams& cp, bool transpose_reads,
                             hipEvent_t const* events, hipStream_t st) {
    const int units = p.batch * p.splits;
    const int grid = 8 * p.head_groups * ((units + 7) / 8);
    hipError_t e;
    if (events && (e = hipEventRecord(events[0], st)) != hipSuccess) return e;
    const bool g = p.indices != nullptr;
    if (p.rope_dim == 64) {
        if (g)
            e = transpose_reads ? launch_split<64, true, true>(p, grid, st) : launch_split<64, true, false>(p, grid, st);
        else
            e = transpose_reads ? launch_split<64, false, true>(p, grid, st) : launch_split<64, false, false>(p, grid, st);
    } else {
        if (g)
            e = transpose_reads ? launch_split<0, true, true>(p, grid, st) : launch_split<0, true, false>(p, grid, st);
        else
            e = transpose_reads ? launch_split<0, false, true>(p, grid, st) : launch_split<0, false, false>(p, grid, st);
    }
    if (e != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[1], st)) != hipSuccess) return e;
    hipLaunchKernelGGL(mla_combine, dim3(p.batch * p.heads, R / 256), dim3(256), 0, st, cp);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[2], st)) != hipSuccess) return e;
    return hipSuccess;
}

}  // namespace mr
