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
//   sub-chunk   = 32 cache rows, global -> LDS by DMA (global_load_lds_dwordx4),
//                 4 buffers so 3 sub-chunks are in flight while one is used;
//                 rows unpadded, 16-byte chunks XOR-swizzled (bank-conflict
//                 free MFMA and transposed reads); LDS-only barriers keep the
//                 DMA in flight across them
//   QK          = 16x16x32 bf16 MFMA, A = cache rows (LDS), B = Q (VGPRs);
//                 wave w scores one 16-row x 16-head tile
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
constexpr int ROWS = 32;      // rows per sub-chunk
constexpr int NBUF = 4;       // LDS sub-chunk buffers (3 in flight while one is consumed)
constexpr int HG = 32;        // heads per workgroup
constexpr int THREADS = 256;  // 4 waves
constexpr int PSTR = 80;      // bytes per head row of P (32 bf16 + 16 pad)
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LOG2E = 1.4426950408889634f;

template <int DR>
struct Geo {
    static constexpr int DK = R + DR;
    static constexpr int KS = DK / 32;        // MFMA k-steps of QK
    static constexpr int CPR = DK / 8;        // 16-byte chunks per row
    static constexpr int ROWB = DK * 2;       // bytes per LDS row (unpadded, swizzled)
    static constexpr int BUF = ROWS * ROWB;   // one sub-chunk
    static constexpr int NLD = BUF / 1024 / 4;  // 1 KB DMA loads per wave per sub-chunk
    static_assert(BUF % 4096 == 0, "sub-chunk must split into 4 waves x 1 KB loads");
};

// Physical 16-byte slot of logical chunk c in LDS row r.  The XOR keeps the
// QK A-operand reads (16 rows, one chunk column) and the transposed PV reads
// (8 rows of one parity, one chunk pair) on distinct banks.  The rope chunks
// (c >= 64) swizzle inside their own 8-chunk group.  The map is an involution.
__device__ __forceinline__ int swz(int c, int r) {
    return c < 64 ? (c ^ (r & 15)) : (64 + ((c - 64) ^ (r & 7)));
}

// Row of the 32-row sub-chunk that MFMA A-row `a` of row tile `rt` scores:
// rows 16rt + {0,2,4,6}, {1,3,5,7}, {8..14 even}, {9..15 odd} for a/4 = 0..3.
// This makes each lane's four P values contiguous in the PV k order below.
__device__ __forceinline__ int sigma_row(int rt, int a) {
    const int g = a >> 2;
    return 16 * rt + 8 * (g >> 1) + (g & 1) + 2 * (a & 3);
}

// LDS-only barrier: waits for this wave's LDS traffic, not for its global
// (DMA) loads, so prefetches stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// All global -> LDS traffic of the split kernel is issued with this
// instruction from inline asm, so the compiler neither knows of it nor
// inserts its conservative vmcnt(0) before LDS reads; the kernel waits for
// it explicitly with wait_vmcnt.  The kernel issues no other vector-memory
// load after the first DMA, which keeps those counts exact.  (Extra loads
// the compiler does not see can only make its own waits stricter.)
__device__ __forceinline__ void dma16(const void* src, const void* lds_dst_wave_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_dst_wave_base;  // LDS offset (low 32 bits)
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// Same DMA with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane
// byte offset: one VGPR per load instead of two.
__device__ __forceinline__ void dma16_off(const void* sbase, uint32_t voff, const void* lds_dst_wave_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_dst_wave_base;
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

constexpr float TAU = 8.f;  // log2 headroom before the running max is raised

template <int DR, bool GATHER, bool TR, bool PACKED>
__global__ void __launch_bounds__(THREADS, 1) mla_decode_split(DecodeParams p) {
    using G = Geo<DR>;
    __shared__ __attribute__((aligned(1024))) char cbuf[NBUF * G::BUF];
    __shared__ __attribute__((aligned(16))) char pbuf[HG * PSTR];
    __shared__ float red[4][16];
    __shared__ __attribute__((aligned(16))) float red4[4][16][4];  // [wave][head col][lane group] partial maxes
    __shared__ __attribute__((aligned(16))) float alpha_s[HG];
    __shared__ int flag_s[2];
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
    const int rt = w >> 1;  // QK row tile of this wave
    const int ht = w & 1;   // QK head tile of this wave

    const uint16_t* lat = p.latent + (int64_t)b * p.lat_bs;
    const uint16_t* rop = DR ? p.rope + (int64_t)b * p.rope_bs : nullptr;

    if (GATHER) {
        const int32_t* ind = p.indices + (int64_t)b * p.n_idx;
        for (int i = tid; i < nrows; i += THREADS) {
            const int32_t v = ind[row_begin + i];
            idx_s[i] = (v >= 0 && v < p.n_ctx) ? v : -1;
        }
        __syncthreads();
    }

    // ---- DMA geometry, loop invariant: load k of this lane fills slot
    // 64(w+4k)+l, i.e. chunk dma_c[k] of row dma_row[k] of a sub-chunk.
    int dma_row[G::NLD], dma_c16[G::NLD];
#pragma unroll
    for (int k = 0; k < G::NLD; ++k) {
        const int slot = 64 * (w + 4 * k) + l;
        dma_row[k] = slot / G::CPR;
        dma_c16[k] = 16 * swz(slot - dma_row[k] * G::CPR, dma_row[k]);
    }
    const uint32_t rs_b = (uint32_t)(p.lat_rs * 2);
    // Every lane always loads: a row past the split reads the split's last
    // row (dense) or row 0 (gather) and is masked to P = 0, so each wave issues
    // exactly NLD loads per sub-chunk and the vmcnt waits are exact.
    auto issue_one = [&](int s, char* base, int k) {
        const int rbase = row_begin + s * ROWS;
        int rr = dma_row[k];  // row relative to rbase
        int src_row;
        if (GATHER) {
            const int v = (rbase + rr < row_end) ? idx_s[rbase + rr - row_begin] : -1;
            src_row = v >= 0 ? v : 0;
        } else {
            if (rbase + ROWS > row_end) rr = min(rr, row_end - 1 - rbase);
            src_row = rbase + rr;
        }
        if (PACKED) {
            if (GATHER)
                dma16_off(lat, (uint32_t)src_row * rs_b + (uint32_t)dma_c16[k], base + 1024 * (w + 4 * k));
            else
                dma16_off((const char*)lat + (int64_t)rbase * rs_b, (uint32_t)rr * rs_b + (uint32_t)dma_c16[k],
                          base + 1024 * (w + 4 * k));
        } else {
            const int c = dma_c16[k] >> 4;
            const uint16_t* src = c < R / 8 ? lat + (int64_t)src_row * p.lat_rs + c * 8
                                            : rop + (int64_t)src_row * p.rope_rs + (c - R / 8) * 8;
            dma16(src, base + 1024 * (w + 4 * k));
        }
    };
    auto issue = [&](int s, char* base) {
#pragma unroll
        for (int k = 0; k < G::NLD; ++k) issue_one(s, base, k);
    };

    // ---- Q of the head group, staged through the last buffer: "row" h of the
    // buffer is head hg*32+h (q_lat ++ q_rope, the shape and swizzle of a cache
    // row).  Heads past p.heads read head 0 (their outputs are discarded).
    {
        char* base = cbuf + (NBUF - 1) * G::BUF;
#pragma unroll
        for (int k = 0; k < G::NLD; ++k) {
            const int row = dma_row[k];
            const int c = dma_c16[k] >> 4;
            const int h0 = hg * HG + row;
            const int h = h0 < p.heads ? h0 : 0;
            const uint16_t* src = c < R / 8 ? p.q_lat + (int64_t)b * p.q_lat_bs + (int64_t)h * p.q_lat_hs + c * 8
                                            : p.q_rope + (int64_t)b * p.q_rope_bs + (int64_t)h * p.q_rope_hs + (c - R / 8) * 8;
            dma16(src, base + 1024 * (w + 4 * k));
        }
    }
    for (int s = 0; s < NBUF - 1 && s < nsub; ++s) issue(s, cbuf + s * G::BUF);
    const int pro = min(nsub, NBUF - 1);  // sub-chunks issued after Q
    if (pro >= 3)
        wait_vmcnt<3 * G::NLD>();
    else if (pro == 2)
        wait_vmcnt<2 * G::NLD>();
    else if (pro == 1)
        wait_vmcnt<G::NLD>();
    else
        wait_vmcnt<0>();
    lds_barrier();
    bf16x8 qreg[G::KS];  // B operand: head 16ht+lc, k = 32ks+8lg..+7
    {
        const int qrow = 16 * ht + lc;
        const char* qp = cbuf + (NBUF - 1) * G::BUF + qrow * G::ROWB;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) qreg[ks] = *(const bf16x8*)(qp + 16 * swz(4 * ks + lg, qrow));
    }
    // (the first loop barrier orders these reads before buffer NBUF-1 refills)

    f32x4 oacc[2][8];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int J = 0; J < 8; ++J) oacc[T][J] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = NEG_INF;  // reference max (base 2) of head 16ht+lc; scores may exceed it by < TAU
    float l_run = 0.f;      // this lane's share of that head's sum

    // QK A operand: chunk 4ks+lg of row `arow` is at
    // 16*((4ks+lg) ^ (arow&15)) = qk_off[ks%4] + 256*(ks/4) (latent) and qk_rope[ks-16].
    const int arow = sigma_row(rt, lc);
    const int lbase = 8 * (lg >> 1) + (lg & 1);
    int qk_off[4], qk_rope[2];
    {
        const int x = arow & 15, y = x >> 2, z0 = (lg ^ x) & 3;
#pragma unroll
        for (int u = 0; u < 4; ++u) qk_off[u] = arow * G::ROWB + 16 * z0 + 64 * (u ^ y);
#pragma unroll
        for (int u = 0; u < 2; ++u) qk_rope[u] = arow * G::ROWB + 1024 + 16 * z0 + 64 * (u ^ (y & 1));
    }
    // PV transposed reads: chunk (16w + 2J + h) of rows r0 / r0+1 (r0 even) is
    // at 256w + 32(J ^ z) + 16h (+16 flipped on the odd row)
    int tr0[8], tr1[8];
    {
        const int r0 = 16 * (lg >> 1) + 8 * (lg & 1) + 2 * (lc >> 2);
        const int z32 = 32 * ((r0 & 15) >> 1);
        const int h = (lc & 3) >> 1;
        const int b0 = r0 * G::ROWB + 256 * w + 16 * h + 8 * (lc & 1);
        const int b1 = (r0 + 1) * G::ROWB + 256 * w + 16 * (h ^ 1) + 8 * (lc & 1);
#pragma unroll
        for (int J = 0; J < 8; ++J) {
            tr0[J] = b0 + ((32 * J) ^ z32);
            tr1[J] = b1 + ((32 * J) ^ z32);
        }
    }
    const int kap = 8 * (2 * rt + (lg >> 1)) + 4 * (lg & 1);  // P k-slot of this lane's 4 rows
    const float scale2 = p.scale_log2;

    auto step = [&](int s, const char* cur) {
        // ---- wait for sub-chunk s, then refill the buffer freed by s-1
        const int later = min(nsub - 1 - s, NBUF - 2);  // sub-chunks issued after s
        if (later >= 2)
            wait_vmcnt<2 * G::NLD>();
        else if (later == 1)
            wait_vmcnt<G::NLD>();
        else
            wait_vmcnt<0>();
        lds_barrier();  // s landed for every wave; PV(s-1) done everywhere
        // refill the buffer freed by s-1 with sub-chunk s+3; the DMA is issued
        // between the QK MFMAs so the address unit drains while they run
        const bool refill = s + NBUF - 1 < nsub;
        const int sn = s + NBUF - 1;
        char* nbuf = cbuf + (sn & (NBUF - 1)) * G::BUF;

        // ---- QK: S[16 rows][16 heads]
        f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
        {
            bf16x8 a[G::KS];
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) a[ks] = *(const bf16x8*)(cur + qk_off[ks & 3] + 256 * (ks >> 2));
#pragma unroll
            for (int ks = 16; ks < G::KS; ++ks) a[ks] = *(const bf16x8*)(cur + qk_rope[ks - 16]);
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks) {
                sacc = mfma16(a[ks], qreg[ks], sacc);
                if ((ks & 1) && (ks >> 1) < G::NLD) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (refill) issue_one(sn, nbuf, ks >> 1);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        float sv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[i] = sacc[i] * scale2;
        const int rbase = row_begin + s * ROWS;
        if (GATHER || rbase + ROWS > row_end) {  // mask rows past the split / -1 entries
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = rbase + 16 * rt + lbase + 2 * i;
                bool ok = r < row_end;
                if (GATHER) ok = ok && idx_s[r - row_begin] >= 0;
                if (!ok) sv[i] = NEG_INF;
            }
        }
        // partial max over this lane's 4 rows; the 8 partials of a head (4 lane
        // groups x 2 row tiles) are combined after the barrier, no shuffles
        red4[w][lc][lg] = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
        lds_barrier();

        // ---- reference max: raised only when a score passes it by TAU (or
        // on the first valid rows), so O is rarely rescaled; P <= 2^TAU.
        const f32x4 pm0 = *(const f32x4*)red4[w][lc];
        const f32x4 pm1 = *(const f32x4*)red4[w ^ 2][lc];
        const float cm = fmaxf(fmaxf(fmaxf(pm0[0], pm0[1]), fmaxf(pm0[2], pm0[3])),
                               fmaxf(fmaxf(pm1[0], pm1[1]), fmaxf(pm1[2], pm1[3])));
        const bool raise = cm > m_run + TAU;  // false while cm is -inf
        const float m_new = raise ? cm : m_run;
        const float alpha = raise ? exp2f(m_run - m_new) : 1.f;  // 0 when m_run was -inf
        m_run = m_new;
        float pv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) pv[i] = (m_new == NEG_INF) ? 0.f : __builtin_amdgcn_exp2f(sv[i] - m_new);
        l_run = l_run * alpha + ((pv[0] + pv[1]) + (pv[2] + pv[3]));
        {
            typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
            const bf16x2v lo = {(__bf16)pv[0], (__bf16)pv[1]};
            const bf16x2v hi = {(__bf16)pv[2], (__bf16)pv[3]};
            const int hh = 16 * ht + lc;
            *(u32x2*)(pbuf + hh * PSTR + kap * 2) =
                u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
            if (rt == 0) {
                if (lg == 0) alpha_s[hh] = alpha;
                const bool any = __builtin_amdgcn_ballot_w64(raise) != 0;
                if (l == 0) flag_s[ht] = any;
            }
        }
        lds_barrier();

        // ---- PV: O[32 heads][128w .. 128w+127] += P[32][32] . C[32][...]
        if (flag_s[0] | flag_s[1]) {  // some head's reference max moved: rescale
#pragma unroll
            for (int T = 0; T < 2; ++T) {
                const f32x4 a4 = *(const f32x4*)(alpha_s + 16 * T + 4 * lg);
#pragma unroll
                for (int J = 0; J < 8; ++J) oacc[T][J] *= a4;
            }
        }
        bf16x8 pa[2];
#pragma unroll
        for (int T = 0; T < 2; ++T) pa[T] = *(const bf16x8*)(pbuf + (16 * T + lc) * PSTR + 16 * lg);
        // k index 8lg + 4t + e of the product <-> row 16(lg/2) + 8(lg%2) + 2e + t
        if (TR) {
            bf16x4 b0[8], b1[8];
#pragma unroll
            for (int J = 0; J < 8; ++J) {
                b0[J] = ds_read_tr16(cur + tr0[J]);
                b1[J] = ds_read_tr16(cur + tr1[J]);
            }
#pragma unroll
            for (int J = 0; J < 8; ++J) {
                const bf16x8 bb = __builtin_shufflevector(b0[J], b1[J], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int T = 0; T < 2; ++T) oacc[T][J] = mfma16(pa[T], bb, oacc[T][J]);
            }
        } else {
#pragma unroll
            for (int J = 0; J < 8; ++J) {
                const int v0 = 128 * w + 16 * J;
                uint16_t e[8];
                const int c = (v0 + lc) >> 3;
                const int sub = 2 * ((v0 + lc) & 7);
                const int rr = 16 * (lg >> 1) + 8 * (lg & 1);
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int row = rr + 2 * q + t;
                        e[4 * t + q] = *(const uint16_t*)(cur + row * G::ROWB + 16 * swz(c, row) + sub);
                    }
                u32x4 u;
#pragma unroll
                for (int j = 0; j < 4; ++j) u[j] = e[2 * j] | ((uint32_t)e[2 * j + 1] << 16);
                const bf16x8 bb = __builtin_bit_cast(bf16x8, u);
#pragma unroll
                for (int T = 0; T < 2; ++T) oacc[T][J] = mfma16(pa[T], bb, oacc[T][J]);
            }
        }
    };

    // four copies of the step, one per buffer, so buffer offsets are constants
    for (int s0 = 0; s0 < nsub; s0 += NBUF) {
        step(s0, cbuf);
        if (s0 + 1 < nsub) step(s0 + 1, cbuf + G::BUF);
        if (s0 + 2 < nsub) step(s0 + 2, cbuf + 2 * G::BUF);
        if (s0 + 3 < nsub) step(s0 + 3, cbuf + 3 * G::BUF);
    }

    // ---- epilogue: l over lane groups and the two row tiles
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    lds_barrier();  // every wave is past its last LDS read of the buffers
    if (lg == 0) red[w][lc] = l_run;
    // O through LDS (the sub-chunk buffers are free): [32 heads][512] fp32,
    // then 16-byte coalesced stores of the partial record
    float* ostage = (float*)cbuf;
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int J = 0; J < 8; ++J) ostage[(16 * T + 4 * lg + i) * R + 128 * w + 16 * J + lc] = oacc[T][J][i];
    lds_barrier();

    const int64_t rec = (int64_t)unit * p.h_pad + hg * HG;
    if (rt == 0 && lg == 0) {
        const int hh = 16 * ht + lc;
        p.ws_ml[(rec + hh) * 2 + 0] = m_run;
        p.ws_ml[(rec + hh) * 2 + 1] = red[w][lc] + red[w ^ 2][lc];
    }
    float* dst = p.ws_o + rec * R;
#pragma unroll
    for (int k = 0; k < HG * R / 4 / THREADS; ++k) {
        const int e4 = tid + THREADS * k;
        *(f32x4*)(dst + 4 * e4) = *(const f32x4*)(ostage + 4 * e4);
    }
}

// Merge the split partials: one 256-thread block per (batch, head, 256-column
// half).  Split weights are computed once into LDS; wave q then streams the
// splits q, q+4, ... with independent 16-byte loads (four columns per lane)
// and the four waves' sums are added through LDS.
__global__ void __launch_bounds__(256) mla_combine(CombineParams p) {
    __shared__ float wgt[MAX_COMBINE_SPLITS];
    __shared__ float red_w[4];
    __shared__ f32x4 part[3][64];
    const int bh = blockIdx.x;
    const int b = bh / p.heads;
    const int h = bh % p.heads;
    const int tid = threadIdx.x;
    const int q = tid >> 6;
    const int l = tid & 63;
    const int64_t rec0 = (int64_t)b * p.splits * p.h_pad + h;
    float M = NEG_INF;
    for (int s = tid; s < p.splits; s += 256) M = fmaxf(M, p.ws_ml[(rec0 + (int64_t)s * p.h_pad) * 2]);
    M = wave_max(M);
    if (l == 0) red_w[q] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red_w[0], red_w[1]), fmaxf(red_w[2], red_w[3]));
    const bool any = M != NEG_INF;
    const float sink2 = p.sinks ? p.sinks[h] * LOG2E : NEG_INF;
    M = fmaxf(M, sink2);
    float L = 0.f;
    for (int s = tid; s < p.splits; s += 256) {
        const int64_t rec = rec0 + (int64_t)s * p.h_pad;
        const float ms = p.ws_ml[rec * 2];
        const float wv = ms == NEG_INF ? 0.f : exp2f(ms - M);
        wgt[s] = wv;
        L += wv * p.ws_ml[rec * 2 + 1];
    }
    L = wave_sum(L);
    __syncthreads();
    if (l == 0) red_w[q] = L;
    __syncthreads();
    L = (red_w[0] + red_w[1]) + (red_w[2] + red_w[3]);
    if (p.sinks) L += exp2f(sink2 - M);
    const int v = blockIdx.y * 256 + 4 * l;
    const float* src = p.ws_o + rec0 * R + v;
    const int64_t step = (int64_t)p.h_pad * R;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    int s = q;
    // a split with no valid row has weight 0 and may hold non-finite
    // scratch: select, never multiply it in
    for (; s + 12 < p.splits; s += 16) {
        const f32x4 x0 = *(const f32x4*)(src + (s + 0) * step);
        const f32x4 x1 = *(const f32x4*)(src + (s + 4) * step);
        const f32x4 x2 = *(const f32x4*)(src + (s + 8) * step);
        const f32x4 x3 = *(const f32x4*)(src + (s + 12) * step);
        acc += wgt[s] != 0.f ? wgt[s] * x0 : zero;
        acc += wgt[s + 4] != 0.f ? wgt[s + 4] * x1 : zero;
        acc += wgt[s + 8] != 0.f ? wgt[s + 8] * x2 : zero;
        acc += wgt[s + 12] != 0.f ? wgt[s + 12] * x3 : zero;
    }
    for (; s < p.splits; s += 4) {
        const f32x4 x = *(const f32x4*)(src + s * step);
        acc += wgt[s] != 0.f ? wgt[s] * x : zero;
    }
    if (q > 0) part[q - 1][l] = acc;
    __syncthreads();
    if (q != 0) return;
    acc += part[0][l];
    acc += part[1][l];
    acc += part[2][l];
    acc *= any ? 1.f / L : 0.f;
    const int64_t o = (int64_t)b * p.out_bs + (int64_t)h * p.out_hs + v;
    if (p.out_f32) {
        *(f32x4*)((float*)p.out + o) = acc;
    } else {
        *(u32x2*)((uint16_t*)p.out + o) = u32x2{pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3])};
    }
}

template <int DR, bool GATHER, bool TR>
hipError_t launch_split(const DecodeParams& p, int grid, hipStream_t st) {
    const bool packed = DR == 0 || (p.rope == p.latent + R && p.rope_rs == p.lat_rs && p.rope_bs == p.lat_bs);
    if (packed)
        hipLaunchKernelGGL((mla_decode_split<DR, GATHER, TR, true>), dim3(grid), dim3(THREADS), 0, st, p);
    else
        hipLaunchKernelGGL((mla_decode_split<DR, GATHER, TR, false>), dim3(grid), dim3(THREADS), 0, st, p);
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
