// Dense projections for gfx950: k3Linear (Linear.swift:55-57), y = x . W^T
// with W output-major [out, in] in bf16 or f32, fp32 accumulation, and the
// two dense forms of the MLA decompression weight kv_b_proj that the
// absorbed decode uses (MLA.swift:180-197): query absorption through W_UK
// and value un-absorption through W_UV.
//
// dense_gemv_kernel (HBM-bound: every weight byte is read once per token
// tile):
//   - tpr lanes share an output row (a power of two, tpr * 4 <= the row's
//     16-byte chunks when it can); a wave covers 64 / tpr rows, a "unit".
//   - Each wave walks a flat list of items (unit, batch of GEMV_BATCH chunks
//     per lane) with two batches of loads in flight: batch k + 1 streams in
//     while batch k is multiplied, and the next load is issued as soon as a
//     batch's registers are free (past its last item a wave loads from the
//     activation vector instead, an L2 hit, so every load is unconditional).  A row's tail batch clamps its chunk index
//     (re-reading the last chunk, a cache hit) and masks the product, so no
//     lane runs a serial remainder loop.  The first two batches are issued
//     before the activations are staged.
//   - The grid holds up to GEMV_WG_PER_CU workgroups per CU and the waves
//     stride over the units, which spreads the activation staging over many
//     rows.
//   - "staged" mode: the activation vectors of the token tile go to LDS
//     once per workgroup (bf16 activations stay bf16 pairs for
//     v_dot2_f32_bf16; 16-byte loads when aligned), with the optional RMSNorm
//     (weight * (x * rsqrt(mean(x^2) + eps)), K3Norm.rms) or the optional
//     sigmoid gate (x * sigmoid(g), MLA.swift:209-211) applied there; bf16
//     inputs are rounded back to bf16 after that, as a separate norm or gate
//     stage would store them.
//   - "direct" mode (grouped rows, y[j] = x[j / map_a] . W[wrow(j)]): each
//     lane reads its x chunk from global memory next to the weight chunk
//     (the vectors are small and shared through L2); with bf16 weights and
//     activations the x chunks are loaded with the weight batch.
//   - The lanes of a row meet by DPP / permlane butterflies (group_sum).
//   - A staged launch may stack up to three weights of the same width along
//     its output rows (projections of one activation vector in one launch).
//
// dense_absorb_kernel: q_lat[h][:] = sum_d q[h][d] * W[h*(nope+v) + d][:]
// (the transposed product: each weight row is scaled by one query value),
// four workgroups per head, each taking 128 of the 512 columns: a lane owns
// one 16-byte chunk of the slice, the row groups step over the nope rows
// with ABS_UNROLL rows in flight per lane and meet in LDS; the head's rotary
// columns may be rotated in the same launch (one position, adjacent pairs),
// and one extra workgroup may append the token's cache row.
#include <algorithm>

#include "cache_append.hpp"
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

// Eight consecutive activations at element offset o as floats; the address
// is 16-byte aligned (bf16: one 16-byte load, f32: two).
__device__ __forceinline__ void load8(const void* p, bool f32, int64_t o, float (&v)[8]) {
    if (f32) {
        const f32x4 a = *(const f32x4*)((const float*)p + o), b = *(const f32x4*)((const float*)p + o + 4);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[k] = a[k];
            v[k + 4] = b[k];
        }
    } else {
        const u32x4 a = *(const u32x4*)((const uint16_t*)p + o);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = __uint_as_float(a[k] << 16);
            v[2 * k + 1] = __uint_as_float(a[k] & 0xffff0000u);
        }
    }
}

__device__ __forceinline__ float sigmoid_gate(float e, float g) { return e * sigmoid_f32(g); }

// sum over the workgroup of one value per thread
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < LT / 64; ++w) tot += red[w];
    __syncthreads();
    return tot;
}

// Stage token t's effective activations (optional RMSNorm or gate applied)
// into xs[t][in], eight values per 16-byte load, SG groups of eight per
// thread with all loads of a round issued before the first use.
template <bool XF32>
__device__ void stage_vec8(const DenseGemvParams& p, int t, char* xs, float* red) {
    constexpr int SG = 2;
    const int tid = threadIdx.x;
    const int groups = p.in / 8;
    const int tt = blockIdx.y * p.mt + t;
    const int64_t xo = (int64_t)tt * p.x_stride, go = (int64_t)tt * p.gate_stride;
    float r = 1.f;
    if (p.norm_w) {
        float ss = 0.f;
        for (int base = 0; base < groups; base += LT * SG) {
            float v[SG][8];
#pragma unroll
            for (int u = 0; u < SG; ++u) load8(p.x, XF32, xo + 8 * (int64_t)min(base + u * LT + tid, groups - 1), v[u]);
#pragma unroll
            for (int u = 0; u < SG; ++u) {
                float s8 = 0.f;
#pragma unroll
                for (int k = 0; k < 8; ++k) s8 = fmaf(v[u][k], v[u][k], s8);
                ss += base + u * LT + tid < groups ? s8 : 0.f;
            }
        }
        r = rsqrtf(block_sum(ss, red) / (float)p.in + p.norm_eps);
    }
    for (int base = 0; base < groups; base += LT * SG) {
        float v[SG][8], a[SG][8];
#pragma unroll
        for (int u = 0; u < SG; ++u) {
            const int gi = min(base + u * LT + tid, groups - 1);
            load8(p.x, XF32, xo + 8 * (int64_t)gi, v[u]);
            if (p.norm_w)
                load8(p.norm_w, p.norm_w_f32, 8 * (int64_t)gi, a[u]);
            else if (p.gate)
                load8(p.gate, p.gate_f32, go + 8 * (int64_t)gi, a[u]);
        }
#pragma unroll
        for (int u = 0; u < SG; ++u) {
            const int gi = base + u * LT + tid;
            float e[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                e[k] = v[u][k];
                if (p.norm_w) e[k] = a[u][k] * (e[k] * r);
                else if (p.gate) e[k] = sigmoid_gate(e[k], a[u][k]);
            }
            if (gi < groups) {
                if (XF32) {
                    f32x4* d = (f32x4*)(xs + 4 * ((int64_t)t * p.in + 8 * gi));
                    d[0] = f32x4{e[0], e[1], e[2], e[3]};
                    d[1] = f32x4{e[4], e[5], e[6], e[7]};
                } else {  // bf16 inputs stay bf16, as a separate norm or gate stage would store them
                    u32x4 w;
#pragma unroll
                    for (int k = 0; k < 4; ++k) w[k] = f32_to_bf16_bits(e[2 * k]) | ((uint32_t)f32_to_bf16_bits(e[2 * k + 1]) << 16);
                    *(u32x4*)(xs + 2 * ((int64_t)t * p.in + 8 * gi)) = w;
                }
            }
        }
    }
}

// The same for activations without 16-byte alignment: element loads, SR per
// thread per round.
template <bool XF32>
__device__ void stage_scalar(const DenseGemvParams& p, int t, char* xs, float* red) {
    constexpr int SR = 8;
    const int tid = threadIdx.x;
    const int tt = blockIdx.y * p.mt + t;
    const int64_t xo = (int64_t)tt * p.x_stride, go = (int64_t)tt * p.gate_stride;
    float r = 1.f;
    if (p.norm_w) {
        float ss = 0.f;
        for (int base = 0; base < p.in; base += LT * SR) {
            float v[SR];
#pragma unroll
            for (int u = 0; u < SR; ++u) v[u] = load_act(p.x, XF32, xo + min(base + u * LT + tid, p.in - 1));
#pragma unroll
            for (int u = 0; u < SR; ++u) ss = base + u * LT + tid < p.in ? fmaf(v[u], v[u], ss) : ss;
        }
        r = rsqrtf(block_sum(ss, red) / (float)p.in + p.norm_eps);
    }
    for (int base = 0; base < p.in; base += LT * SR) {
        float v[SR], a[SR];
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int i = min(base + u * LT + tid, p.in - 1);
            v[u] = load_act(p.x, XF32, xo + i);
            if (p.norm_w)
                a[u] = load_act(p.norm_w, p.norm_w_f32, i);
            else if (p.gate)
                a[u] = load_act(p.gate, p.gate_f32, go + i);
        }
#pragma unroll
        for (int u = 0; u < SR; ++u) {
            const int i = base + u * LT + tid;
            float e = v[u];
            if (p.norm_w) e = a[u] * (e * r);
            else if (p.gate) e = sigmoid_gate(e, a[u]);
            if (i < p.in) {
                if (XF32)
                    ((float*)xs)[t * p.in + i] = e;
                else
                    ((uint16_t*)xs)[t * p.in + i] = f32_to_bf16_bits(e);
            }
        }
    }
}

constexpr int GEMV_BATCH = 8;      // 16-byte weight chunks per lane per batch
constexpr int GEMV_WG_PER_CU = 4;  // resident workgroups per CU the grid aims for

template <bool WF32, bool XF32, bool STAGED, int MT>
__global__ void __launch_bounds__(LT) dense_gemv_kernel(DenseGemvParams p) {
    constexpr int VPC = WF32 ? 4 : 8;  // values per 16-byte weight chunk
    constexpr int XE = XF32 ? 4 : 2;   // bytes per activation value
    constexpr int B = GEMV_BATCH;
    extern __shared__ __attribute__((aligned(16))) char xs[];  // staged: [mt][in] activations
    __shared__ float red[LT / 64];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.y * p.mt;
    const int mt = min(p.mt, p.m - t0);
    const int tpr = p.tpr;
    const int lane = tid & 63;
    const int sub = lane / tpr;       // row of this lane within its unit
    const int li = lane - sub * tpr;  // lane within the row
    const int rpw = 64 / tpr;
    const int chunks = p.in / VPC;
    const int nb = p.batches;  // batches per unit
    const int64_t gw = (int64_t)blockIdx.x * (LT / 64) + (tid >> 6);
    const int64_t tw = (int64_t)gridDim.x * (LT / 64);
    const int64_t my_units = gw < p.units ? (p.units - 1 - gw) / tw + 1 : 0;
    const int nitems = (int)my_units * nb;

    // item k: unit gw + (k / nb) * tw, chunks li + (b * B + u) * tpr of its rows
    auto row_of = [&](int ui) -> int64_t { return (gw + (int64_t)ui * tw) * rpw + sub; };
    auto wrow_of = [&](int64_t j, int64_t& g) -> int64_t {
        const int64_t jj = j < p.out_rows ? j : 0;
        if (STAGED) {
            g = 0;
            return jj + p.map_c;
        }
        g = (int64_t)((uint32_t)jj / (uint32_t)p.map_a);
        return g * p.map_b + p.map_c + (jj - g * p.map_a);
    };
    // stacked weights (staged only): segment of row j and its first row
    auto seg_of = [&](int64_t j, int& sg, int64_t& first) {
        sg = (j >= p.seg_end[0]) + (p.nseg > 2 && j >= p.seg_end[1]);
        first = sg == 0 ? 0 : (sg == 1 ? p.seg_end[0] : p.seg_end[1]);
    };
    // direct mode with bf16 activations: the activation chunks ride with the
    // weight chunks (same 8 values when the weights are bf16)
    constexpr bool XPRE = !STAGED && !XF32 && !WF32;
    const int xch = max(1, p.in * XE / 16);  // 16-byte chunks of one activation vector
    auto load = [&](int k, u32x4(&w)[B], u32x4(&xv)[B]) {
        // past its last item a wave still loads (unconditional loads keep the
        // compiler's count of loads in flight exact across the loop), from
        // the activation vector, which every workgroup has just read (L2)
        const bool past = k >= nitems;
        k = min(k, nitems - 1);
        const int ui = k / nb, b = k - ui * nb;
        int64_t g;
        const int64_t wrow = wrow_of(row_of(ui), g);
        const char* wr = (const char*)p.w + wrow * p.w_rs * (WF32 ? 4 : 2);
        if (STAGED && p.nseg) {
            int sg;
            int64_t first;
            seg_of(wrow, sg, first);
            const void* sw = sg == 0 ? p.seg_w[0] : (sg == 1 ? p.seg_w[1] : p.seg_w[2]);
            const int64_t rs = sg == 0 ? p.seg_w_rs[0] : (sg == 1 ? p.seg_w_rs[1] : p.seg_w_rs[2]);
            wr = (const char*)sw + (wrow - first) * rs * (WF32 ? 4 : 2);
        }
        const char* xd = (const char*)p.x + ((int64_t)t0 * p.x_stride + g * p.x_vec_stride) * XE;
        if (past) wr = (const char*)p.x;
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int cl = li + (b * B + u) * tpr;
            const int c = min(cl, past ? xch - 1 : chunks - 1);
            w[u] = __builtin_nontemporal_load((const u32x4*)(wr + 16 * (int64_t)c));
            if (XPRE) xv[u] = *(const u32x4*)(xd + 16 * (int64_t)c);
        }
    };
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.f;
    auto consume = [&](int k, const u32x4(&w)[B], const u32x4(&xv)[B]) {
        const int ui = k / nb, b = k - ui * nb;
        const int64_t j = row_of(ui);
        int64_t g;
        (void)wrow_of(j, g);
        const char* xd = (const char*)p.x + ((int64_t)t0 * p.x_stride + g * p.x_vec_stride) * XE;
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int cr = li + (b * B + u) * tpr;
            const bool ok = cr < chunks;
            const int i0 = min(cr, chunks - 1) * VPC;
            if (STAGED) {
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    if (t < mt) {
                        const float a = chunk_dot<WF32, XF32>(w[u], xs + ((int64_t)t * p.in + i0) * XE, acc[t]);
                        acc[t] = ok ? a : acc[t];
                    }
                }
            } else if (XPRE) {
                const float a = chunk_dot<WF32, XF32>(w[u], &xv[u], acc[0]);
                acc[0] = ok ? a : acc[0];
            } else {
                const float a = chunk_dot<WF32, XF32>(w[u], xd + (int64_t)i0 * XE, acc[0]);
                acc[0] = ok ? a : acc[0];
            }
        }
        if (b == nb - 1) {  // the unit's last batch: reduce its rows and store
            const bool live = j < p.out_rows;
            const int nt = STAGED ? mt : 1;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if (t >= nt) break;
                const float v = group_sum(acc[t], tpr);
                acc[t] = 0.f;
                if (live && li == 0) {
                    void* y = p.y;
                    int64_t yo = (int64_t)(t0 + t) * p.y_stride_token + j * p.y_stride_row;
                    if (STAGED && p.nseg) {
                        int sg;
                        int64_t first;
                        seg_of(j, sg, first);
                        y = sg == 0 ? p.seg_y[0] : (sg == 1 ? p.seg_y[1] : p.seg_y[2]);
                        const int64_t ts = sg == 0 ? p.seg_y_ts[0] : (sg == 1 ? p.seg_y_ts[1] : p.seg_y_ts[2]);
                        yo = (int64_t)(t0 + t) * ts + (j - first) * p.y_stride_row;
                    }
                    if (p.y_f32)
                        ((float*)y)[yo] = v;
                    else
                        ((uint16_t*)y)[yo] = f32_to_bf16_bits(v);
                }
            }
        }
    };

    u32x4 wa[B], wb[B];
    u32x4 xa[B], xb[B];  // used only with XPRE
    if (nitems > 0) {
        load(0, wa, xa);
        load(1, wb, xb);
    }
    if (STAGED) {
        for (int t = 0; t < mt; ++t) {
            if (p.stage_vec)
                stage_vec8<XF32>(p, t, xs, red);
            else
                stage_scalar<XF32>(p, t, xs, red);
        }
        __syncthreads();
    }
    for (int k = 0; k < nitems; k += 2) {
        consume(k, wa, xa);
        load(k + 2, wa, xa);
        if (k + 1 >= nitems) break;
        consume(k + 1, wb, xb);
        load(k + 3, wb, xb);
    }
}

constexpr int ABS_CW = 128;  // q_lat columns per absorb workgroup
constexpr int ABS_UNROLL = 8;  // row steps in flight per lane

template <bool WF32>
__global__ void __launch_bounds__(LT) dense_absorb_kernel(DenseAbsorbParams p) {
    constexpr int VPC = WF32 ? 4 : 8;      // columns per 16-byte chunk
    constexpr int LPR = ABS_CW / VPC;      // lanes per weight row slice
    constexpr int RPS = LT / LPR;          // rows per step
    __shared__ __attribute__((aligned(16))) float part[RPS][ABS_CW];
    if (p.app_on && blockIdx.x == gridDim.x - 1) {  // the extra workgroup: the cache append
        cache_append_row(p.app, 0, &part[0][0]);
        return;
    }
    const int h = blockIdx.x / (512 / ABS_CW);
    const int cs = blockIdx.x - h * (512 / ABS_CW);
    const int tid = threadIdx.x;
    uint16_t* qh = (uint16_t*)p.q + (int64_t)h * p.q_head_stride;
    if (cs == 0 && p.rope_cos) {  // the head's rotary columns, in place (they are not read below)
        for (int i = tid; i < p.rope_dim / 2; i += LT) {
            const float a = bf16_bits_to_f32(qh[p.rope_col0 + 2 * i]);
            const float b = bf16_bits_to_f32(qh[p.rope_col0 + 2 * i + 1]);
            const float c = p.rope_cos[i], s = p.rope_sin[i];
            qh[p.rope_col0 + 2 * i] = f32_to_bf16_bits(sub_rn(mul_rn(a, c), mul_rn(b, s)));
            qh[p.rope_col0 + 2 * i + 1] = f32_to_bf16_bits(add_rn(mul_rn(a, s), mul_rn(b, c)));
        }
    }
    const int rg = tid / LPR, li = tid - rg * LPR;  // row group, chunk of the slice
    const int64_t row0 = (int64_t)h * (p.nope_dim + p.v_dim);
    const int esz = WF32 ? 4 : 2;
    const char* wc = (const char*)p.w + (int64_t)(cs * ABS_CW + li * VPC) * esz;
    float acc[VPC];
#pragma unroll
    for (int k = 0; k < VPC; ++k) acc[k] = 0.f;
    for (int d0 = rg; d0 < p.nope_dim; d0 += RPS * ABS_UNROLL) {
        u32x4 wv[ABS_UNROLL];
        float qd[ABS_UNROLL];
#pragma unroll
        for (int u = 0; u < ABS_UNROLL; ++u) {  // rows past nope_dim re-read the last one, weighted 0
            const int d = d0 + u * RPS;
            const int dc = min(d, p.nope_dim - 1);
            wv[u] = __builtin_nontemporal_load((const u32x4*)(wc + (row0 + dc) * p.w_rs * esz));
            qd[u] = d < p.nope_dim ? bf16_bits_to_f32(qh[dc]) : 0.f;
        }
#pragma unroll
        for (int u = 0; u < ABS_UNROLL; ++u)
#pragma unroll
            for (int k = 0; k < VPC; ++k) {
                const float wk =
                    WF32 ? __uint_as_float(wv[u][k]) : __uint_as_float(k & 1 ? wv[u][k >> 1] & 0xffff0000u : wv[u][k >> 1] << 16);
                acc[k] = fmaf(qd[u], wk, acc[k]);
            }
    }
#pragma unroll
    for (int k = 0; k < VPC; ++k) part[rg][li * VPC + k] = acc[k];
    __syncthreads();
    uint16_t* out = p.q_lat + (int64_t)h * p.q_lat_head_stride + cs * ABS_CW;
    for (int c = tid; c < ABS_CW; c += LT) {
        float v = 0.f;
#pragma unroll
        for (int g = 0; g < RPS; ++g) v += part[g][c];
        out[c] = f32_to_bf16_bits(v);
    }
}

// out[i] = bf16(x[i] * sigmoid(g[i])), MLA.swift:209-211 as its own stage:
// 8 elements (16 bytes) per step over the first n8 * 8, one by one after
__global__ void __launch_bounds__(LT) gate_mul_kernel(const uint16_t* x, const uint16_t* g, int64_t n, int64_t n8,
                                                      uint16_t* out) {
    const int64_t stride = (int64_t)gridDim.x * LT;
    for (int64_t i = (int64_t)blockIdx.x * LT + threadIdx.x; i < n8; i += stride) {
        u32x4 a = *(const u32x4*)(x + 8 * i);
        const u32x4 b = *(const u32x4*)(g + 8 * i);
#pragma unroll
        for (int k = 0; k < 4; ++k) a[k] = gated_bf16x2(a[k], b[k]);
        *(u32x4*)(out + 8 * i) = a;
    }
    for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * LT + threadIdx.x; i < n; i += stride)
        out[i] = (uint16_t)gated_bf16x2(x[i], g[i]);
}

}  // namespace

hipError_t launch_gate_mul(const uint16_t* x, const uint16_t* g, int64_t n, uint16_t* out, hipStream_t st) {
    const bool vec = (((uintptr_t)x | (uintptr_t)g | (uintptr_t)out) & 15) == 0;
    const int64_t n8 = vec ? n / 8 : 0;
    const int64_t blocks = (std::max<int64_t>(n8, n - 8 * n8) + LT - 1) / LT;
    hipLaunchKernelGGL(gate_mul_kernel, dim3((unsigned)std::min<int64_t>(std::max<int64_t>(blocks, 1), 2048)), dim3(LT),
                       0, st, x, g, n, n8, out);
    return hipGetLastError();
}

int dense_gemv_tokens_per_tile(int in, int m, bool x_f32) {
    const int cap = DENSE_STAGE_BYTES / (in * (x_f32 ? 4 : 2));
    return max(1, min(min(m, cap > 0 ? cap : 1), MAX_GEMV_TOKENS));
}

template <bool WF32, bool XF32, bool STAGED, int MT>
static hipError_t launch_gemv_mt(const DenseGemvParams& p, dim3 grid, size_t lds, hipStream_t st) {
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void*)dense_gemv_kernel<WF32, XF32, STAGED, MT>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((dense_gemv_kernel<WF32, XF32, STAGED, MT>), grid, dim3(LT), lds, st, p);
    return hipGetLastError();
}

template <bool WF32, bool XF32>
static hipError_t launch_gemv(const DenseGemvParams& p, bool staged, dim3 grid, size_t lds, hipStream_t st) {
    if (!staged) return launch_gemv_mt<WF32, XF32, false, 1>(p, grid, 0, st);
    if (p.mt == 1) return launch_gemv_mt<WF32, XF32, true, 1>(p, grid, lds, st);
    if (p.mt <= 4) return launch_gemv_mt<WF32, XF32, true, 4>(p, grid, lds, st);
    return launch_gemv_mt<WF32, XF32, true, MAX_GEMV_TOKENS>(p, grid, lds, st);
}

hipError_t launch_dense_gemv(DenseGemvParams p, bool staged, int cus, hipStream_t st) {
    const int vpc = p.w_f32 ? 4 : 8;
    const int chunks = p.in / vpc;
    int tpr = 64;
    while (tpr > 1 && tpr * 4 > chunks) tpr >>= 1;
    p.tpr = tpr;
    const int rpw = 64 / tpr;
    p.units = (p.out_rows + rpw - 1) / rpw;
    const int per_lane = (chunks + tpr - 1) / tpr;
    p.batches = (per_lane + GEMV_BATCH - 1) / GEMV_BATCH;
    const int64_t waves = (int64_t)GEMV_WG_PER_CU * cus * (LT / 64);
    const int64_t wave_need = p.units < waves ? p.units : waves;
    const int64_t grid_x = (wave_need + LT / 64 - 1) / (LT / 64);
    p.mt = staged ? dense_gemv_tokens_per_tile(p.in, p.m, p.x_f32) : 1;
    const int grid_y = (p.m + p.mt - 1) / p.mt;
    const size_t lds = staged ? (size_t)p.mt * p.in * (p.x_f32 ? 4 : 2) : 0;
    auto al16 = [](const void* q, int64_t stride_bytes) { return ((uintptr_t)q & 15) == 0 && stride_bytes % 16 == 0; };
    p.stage_vec = staged && p.in % 8 == 0 && al16(p.x, p.x_stride * (p.x_f32 ? 4 : 2)) &&
                  (!p.norm_w || al16(p.norm_w, 0)) && (!p.gate || al16(p.gate, p.gate_stride * (p.gate_f32 ? 4 : 2)));
    const dim3 grid((unsigned)grid_x, (unsigned)grid_y);
    if (p.w_f32)
        return p.x_f32 ? launch_gemv<true, true>(p, staged, grid, lds, st) : launch_gemv<true, false>(p, staged, grid, lds, st);
    return p.x_f32 ? launch_gemv<false, true>(p, staged, grid, lds, st) : launch_gemv<false, false>(p, staged, grid, lds, st);
}

hipError_t launch_dense_absorb(const DenseAbsorbParams& p, hipStream_t st) {
    const dim3 grid((unsigned)(p.heads * (512 / ABS_CW) + (p.app_on ? 1 : 0)));
    if (p.w_f32)
        hipLaunchKernelGGL(dense_absorb_kernel<true>, grid, dim3(LT), 0, st, p);
    else
        hipLaunchKernelGGL(dense_absorb_kernel<false>, grid, dim3(LT), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
