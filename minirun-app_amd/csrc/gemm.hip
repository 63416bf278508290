// Token-tiled projections on MFMA: y[T][N] = x[T][K] . W[N][K]^T for the
// prefill-sized (many-token) calls of k3Linear (Linear.swift:55-57) and
// affineMM (AffineWeights.swift:239-254).  x is bf16; W is dense bf16 rows
// or MLX 4-bit affine rows (packed uint32 nibbles, element j of a word in
// bits 4j..4j+3, one scale and bias per `group` inputs).  fp32 accumulation;
// y bf16 or f32.
//
// Affine weights are dequantized per k-tile into LDS, w = fp32(scale * q +
// bias) (exact product, one rounding: the affineDequantize value), and
// carried as two bf16 operands hi = bf16(w), lo = bf16(w - hi): x is bf16,
// so x . hi + x . lo on two MFMAs misses x . w by at most 2^-18 |w| per
// product, where a single bf16 weight (2^-9 |w|) would put outputs of the
// 4-bit projections outside a 1e-2 + 2e-2 |y| bar.
//
// One workgroup of 4 waves computes a TM x 256 tile of y (TM = 256 or 128),
// each wave a (TM/2) x 128 block of 32x32x16 bf16 MFMA tiles.  K streams in
// k-tiles of BK = 32 through NS LDS stages (4 dense, 2 affine); a stage holds
// the x tile [TM][32] and the W tile(s) [256][32] in rows of 4 16-byte
// chunks, chunk c of row r in slot c ^ ((r >> 2) & 3), so the 16 lanes of a
// ds_read_b128 phase (16 consecutive rows, one chunk) hit 16 distinct bank
// groups.
//
// Pipeline, iteration kt (stage kt % NS is complete when it starts):
//   - x (and dense W) k-tile kt + NS - 1 goes to the stage read in the
//     previous iteration by global -> LDS DMA (issued by every wave, 1 KB
//     per instruction): dense tiles keep up to NS - 1 k-tiles (96 KB per
//     workgroup) in flight and issue each k-tile's DMA a k-step's share at
//     a time between that k-step's MFMAs; affine ones issue k-tile kt + 1
//     at the top of the iteration;
//   - affine W: the packed words, scales and biases of k-tile kt + 2 go to
//     an LDS slot by DMA too, and those of k-tile kt + 1 (fetched one
//     iteration earlier) are dequantized into the other stage.  Thread t
//     owns W row t of the tile, and the 64 rows of a wave are fetched by
//     that wave's own DMA, so its vmcnt wait alone makes them visible to it;
//   - the k-steps' MFMAs on stage kt % NS, fragments read one step ahead;
//   - one barrier, after this wave's DMA of kt + 1 has landed.
// Past the last k-tile the issues repeat the last one (into a stage or slot
// that is never read again), so every iteration issues the same loads and
// the vmcnt waits are constants.  Every global load is a DMA issued from
// inline asm and waited for explicitly (the compiler neither sees them nor
// adds waits of its own); the only compiler-visible global accesses are the
// output stores.
//
// Rows past T (x) or N (W) repeat the last row; their outputs are not stored.
//
// One launch can stack up to three projections of the same tokens (e.g.
// q_a, kv_a and g_proj of one activation): their N tiles follow each other
// in the grid, and a workgroup takes its projection's weight, output and
// shape from the stack entry its tile falls in.
#include <algorithm>

#include "mr_kernels.hpp"

namespace mr {

namespace {

constexpr int PG_TN = 256, PG_THREADS = 256;

template <int CPR>
__device__ __forceinline__ int pg_slot(int r, int c) {
    static_assert(CPR == 4, "rows of four 16-byte chunks");
    return r * 4 + (c ^ ((r >> 2) & 3));
}

// DMA of 4 bytes per lane (lane i lands at lds_dst_wave_base + 4 i); the
// same wait rules as dma16_off
__device__ __forceinline__ void dma4_off(const void* sbase, uint32_t voff, const void* lds_dst_wave_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_dst_wave_base;
    asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

__device__ __forceinline__ float scale_value(uint32_t bits, int dtype) {
    return dtype == 0 ? __uint_as_float(bits << 16) : (dtype == 1 ? f16_bits_to_f32((uint16_t)bits) : __uint_as_float(bits));
}

// affine k-tile slot in LDS (k-tiles of 32): packed [256 rows][16 bytes],
// then one dword per row of scales and of biases (the dword that holds the
// row's scale for this k-tile)
constexpr int PG_PSLOT = 256 * 16 + 2 * 256 * 4;  // bytes

template <int TM, bool AFFINE>
struct PgShape {
    static constexpr int BK = 32;
    static constexpr int NS = AFFINE ? 2 : 4;             // LDS stages (k-tiles)
    static constexpr int CPR = BK / 8;                    // 16-byte chunks per row
    static constexpr int KS = BK / 16;                    // 16-deep MFMA steps per k-tile
    static constexpr int A_EL = TM * BK;                  // x tile elements
    static constexpr int B_EL = PG_TN * BK;               // one W tile's elements
    static constexpr int STAGE = A_EL + (AFFINE ? 2 : 1) * B_EL;
    static constexpr int RING = NS * STAGE * 2;           // bytes of the stages
    static constexpr size_t LDS_BF16 = std::max<size_t>(RING + (AFFINE ? 2 * PG_PSLOT : 0), (size_t)TM * PG_TN * 2);
    static constexpr size_t LDS_F32 = std::max<size_t>(RING + (AFFINE ? 2 * PG_PSLOT : 0), (size_t)TM / 2 * PG_TN * 4);
};

template <int TM, bool AFFINE, bool YF32>
__global__ void __launch_bounds__(PG_THREADS, 1) proj_gemm_kernel(ProjGemmStack ps) {
    using S = PgShape<TM, AFFINE>;
    constexpr int BK = S::BK, NS = S::NS, CPR = S::CPR, KS = S::KS, A_EL = S::A_EL, B_EL = S::B_EL, STAGE = S::STAGE;
    constexpr int WM = TM / 2;                 // rows per wave
    constexpr int MI = WM / 32;                // 32-row MFMA tiles per wave
    constexpr int RPI = 64 / CPR;              // rows per DMA instruction
    constexpr int DA = TM / RPI / 4;           // x DMA instructions per wave per k-tile
    constexpr int DB = AFFINE ? 0 : PG_TN / RPI / 4;  // dense W DMA instructions per wave per k-tile
    constexpr int DP = AFFINE ? 3 : 0;         // affine DMA instructions per wave per k-tile
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;

    // the stacked projections share x and M; their N tiles follow each other
    const int m_tiles = (ps.seg[0].M + TM - 1) / TM, n_tiles = ps.tile_end[ps.nseg - 1];
    const int total = m_tiles * n_tiles;
    // XCD-aware order: consecutive workgroups go to the 8 XCDs in turn, so
    // XCD x gets tile ids x * total / 8 ..; ids run over groups of 4 M
    // tiles, N tiles outer, M tiles inner, so one XCD's resident workgroups
    // share x rows and W rows in its L2
    int bid = blockIdx.x;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
    constexpr int GM = 4;
    const int group = bid / (GM * n_tiles), first_m = group * GM;
    const int gsize = min(m_tiles - first_m, GM);
    const int mt = first_m + (bid % (GM * n_tiles)) % gsize;
    const int nt_all = (bid % (GM * n_tiles)) / gsize;
    const int seg = (nt_all >= ps.tile_end[0]) + (nt_all >= ps.tile_end[1]);
    const ProjGemmParams p = ps.seg[seg];
    const int nt = nt_all - (seg ? ps.tile_end[seg - 1] : 0);
    const int m0 = mt * TM, n0 = nt * PG_TN;
    const int KT = p.K / BK;

    // DMA instruction i of a tile: rows RPI i ..; lane l fills slot 64 i + l
    // = row RPI i + l / CPR, slot chunk l % CPR, which holds global chunk
    // (l % CPR) ^ f(row).  Byte offsets from the tile's first row.
    const uint16_t* abase = p.x + (int64_t)m0 * p.ldx;
    const uint16_t* bbase = AFFINE ? nullptr : p.w + (int64_t)n0 * p.ldw;
    auto chunk_of = [](int row, int sc) { return sc ^ ((row >> 2) & 3); };
    uint32_t aoff[DA], boff[DB > 0 ? DB : 1];
#pragma unroll
    for (int q = 0; q < DA; ++q) {
        const int row = RPI * (DA * w + q) + l / CPR;
        aoff[q] = (uint32_t)(((int64_t)min(row, p.M - 1 - m0) * p.ldx + 8 * chunk_of(row, l % CPR)) * 2);
    }
    if constexpr (!AFFINE) {
#pragma unroll
        for (int q = 0; q < DB; ++q) {
            const int row = RPI * (DB * w + q) + l / CPR;
            boff[q] = (uint32_t)(((int64_t)min(row, p.N - 1 - n0) * p.ldw + 8 * chunk_of(row, l % CPR)) * 2);
        }
    }
    const int wu = __builtin_amdgcn_readfirstlane(w);
    auto issue_dma = [&](int kt) {  // k-tile min(kt, KT - 1) into stage kt % NS
        uint16_t* st = lds + (kt & (NS - 1)) * STAGE;
        const uint32_t ko = (uint32_t)min(kt, KT - 1) * BK * 2;
#pragma unroll
        for (int q = 0; q < DA; ++q) dma16_off(abase, aoff[q] + ko, st + 512 * (DA * wu + q));
        if constexpr (!AFFINE) {
#pragma unroll
            for (int q = 0; q < DB; ++q) dma16_off(bbase, boff[q] + ko, st + A_EL + 512 * (DB * wu + q));
        }
    };

    // affine: wave w fetches W rows 64w .. 64w + 63 of the tile (lane l: row
    // 64w + l): one 16-byte packed instruction, one dword instruction each
    // for the scales and the biases
    const char* pslots = (const char*)lds + S::RING;
    uint32_t poff = 0, soff = 0;  // soff: byte offset of the row's first scale
    if constexpr (AFFINE) {
        const int row = min(n0 + tid, p.N - 1);
        poff = (uint32_t)((int64_t)row * (p.K / 2));
        soff = (uint32_t)((int64_t)row * (p.K / p.group) * (p.scale_dtype == 2 ? 4 : 2));
    }
    auto scale_byte = [&](int kt) -> uint32_t {  // k-tile kt's scale in the row
        const uint32_t e = (uint32_t)(kt * BK / p.group);
        return soff + (p.scale_dtype == 2 ? 4 * e : 2 * e);
    };
    auto issue_w = [&](int kt) {  // k-tile min(kt, KT - 1) into slot kt % 2
        const char* slot = pslots + (kt & 1) * PG_PSLOT;
        kt = min(kt, KT - 1);
        dma16_off(p.packed, poff + 16 * kt, slot + 1024 * wu);
        const uint32_t so = scale_byte(kt) & ~3u;  // the dword that holds it
        dma4_off(p.scales, so, slot + 4096 + 256 * wu);
        dma4_off(p.biases, so, slot + 5120 + 256 * wu);
    };
    // slot kt % 2 (landed) -> hi and lo bf16 rows of stage kt % 2
    auto dequant_w = [&](int kt) {
        const char* slot = pslots + (kt & 1) * PG_PSLOT;
        uint16_t* sh = lds + (kt & (NS - 1)) * STAGE + A_EL;
        uint16_t* sl = sh + B_EL;
        kt = min(kt, KT - 1);
        const u32x4 q = *(const u32x4*)(slot + 16 * tid);
        uint32_t sw = *(const uint32_t*)(slot + 4096 + 4 * tid), bw = *(const uint32_t*)(slot + 5120 + 4 * tid);
        if (p.scale_dtype != 2 && ((scale_byte(kt) >> 1) & 1)) {  // the high half of the dword
            sw >>= 16;
            bw >>= 16;
        }
        const float s = scale_value(p.scale_dtype == 2 ? sw : sw & 0xffffu, p.scale_dtype);
        const float b = scale_value(p.scale_dtype == 2 ? bw : bw & 0xffffu, p.scale_dtype);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint32_t word = q[c];
            const uint32_t lo4 = word & 0x0F0F0F0Fu, hi4 = (word >> 4) & 0x0F0F0F0Fu;  // nibbles 0,2,4,6 / 1,3,5,7
            u32x4 vh, vl;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float w0 = fmaf(s, (float)((lo4 >> (8 * k)) & 0xffu), b);
                const float w1 = fmaf(s, (float)((hi4 >> (8 * k)) & 0xffu), b);
                vh[k] = pack_bf16x2_hw(w0, w1);
                // w - hi is exact in fp32
                vl[k] = pack_bf16x2_hw(w0 - __uint_as_float(vh[k] << 16), w1 - __uint_as_float(vh[k] & 0xffff0000u));
            }
            *(u32x4*)(sh + 8 * pg_slot<CPR>(tid, c)) = vh;
            *(u32x4*)(sl + 8 * pg_slot<CPR>(tid, c)) = vl;
        }
    };

    const int wm = w >> 1, wn = w & 1;
    constexpr int NB = AFFINE ? 2 : 1;  // W operands per k-step (hi, lo)
    f32x16 acc[MI][4];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
    auto read = [&](int kt, int ks, bf16x8(&a)[MI], bf16x8(&b)[NB][4]) {
        const uint16_t* sa = lds + (kt & (NS - 1)) * STAGE;
        const int ch = 2 * ks + (l >> 5);
#pragma unroll
        for (int i = 0; i < MI; ++i) a[i] = *(const bf16x8*)(sa + 8 * pg_slot<CPR>(wm * WM + i * 32 + (l & 31), ch));
#pragma unroll
        for (int u = 0; u < NB; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                b[u][j] = *(const bf16x8*)(sa + A_EL + u * B_EL + 8 * pg_slot<CPR>(wn * 128 + j * 32 + (l & 31), ch));
    };
    auto mma = [&](const bf16x8(&a)[MI], const bf16x8(&b)[NB][4]) {
#pragma unroll
        for (int u = 0; u < NB; ++u)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(b[u][j], a[i], acc[i][j]);
    };
    // dense: DMA instruction q (of DA + DB) of k-tile kt, and one k-step's
    // MFMAs with the k-step's share of a k-tile's DMA spread among them, so
    // the MFMA pipe stays busy while the address unit takes the loads
    constexpr int NQ = DA + DB, QS = NQ / KS;
    static_assert(AFFINE || NQ % KS == 0, "DMA instructions split evenly over the k-steps");
    auto dma_one = [&](int kt, int q) {
        uint16_t* st = lds + (kt & (NS - 1)) * STAGE;
        const uint32_t ko = (uint32_t)min(kt, KT - 1) * BK * 2;
        if (q < DA)
            dma16_off(abase, aoff[q] + ko, st + 512 * (DA * wu + q));
        else
            dma16_off(bbase, boff[q - DA] + ko, st + A_EL + 512 * (DB * wu + q - DA));
    };
    auto mma_dma = [&](const bf16x8(&a)[MI], const bf16x8(&b)[NB][4], int kt_dma, int ks) {
        constexpr int NM = MI * 4;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            acc[m / 4][m % 4] = mfma32(b[0][m % 4], a[m / 4], acc[m / 4][m % 4]);
#pragma unroll
            for (int r = 0; r < QS; ++r)
                if (m == (r + 1) * NM / QS - 1) {
                    dma_one(kt_dma, ks * QS + r);
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
    };

    // prologue: stage 0 complete, k-tiles 1 .. NS - 2 (and the affine slot
    // of k-tile 1) in flight
#pragma unroll
    for (int k = 0; k < NS - 1; ++k) issue_dma(k);
    constexpr int LATER = (NS - 2) * (DA + DB);  // DMA of the k-tiles after the next one
    if constexpr (AFFINE) {
        issue_w(0);
        issue_w(1);
        wait_vmcnt<LATER + DP>();
        dequant_w(0);
    } else {
        wait_vmcnt<LATER>();
    }
    lds_barrier();
    bf16x8 fa[2][MI], fb[2][NB][4];
    read(0, 0, fa[0], fb[0]);
    if constexpr (!AFFINE) {
        // k-tile kt + NS - 1 is issued a k-step's share at a time; the wait
        // before the last k-step's MFMAs leaves k-tiles kt + 2 .. kt + NS - 2
        // and the shares of kt + NS - 1 issued so far in flight
        static_assert(NS >= 3, "the interleaved DMA needs a stage beyond the next");
        constexpr int WAIT = (NS - 3) * NQ + (NQ - QS);
#pragma unroll 1
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int nx = (ks + 1) & 1;
                if (ks + 1 < KS) {
                    read(kt, ks + 1, fa[nx], fb[nx]);
                } else {
                    wait_vmcnt<WAIT>();  // this wave's DMA of k-tile kt + 1 landed
                    lds_barrier();       // every wave's; every wave done with stage kt
                    read(kt + 1, 0, fa[nx], fb[nx]);  // past the last k-tile: a stage never used, in bounds
                }
                mma_dma(fa[ks & 1], fb[ks & 1], kt + NS - 1, ks);
            }
        }
    }
#pragma unroll 1
    for (int kt = 0; AFFINE && kt < KT; ++kt) {
        issue_dma(kt + NS - 1);
        if constexpr (AFFINE) {
            issue_w(kt + 2);
            wait_vmcnt<DA + DP>();  // this wave's slot of k-tile kt + 1
            dequant_w(kt + 1);
        }
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int nx = (ks + 1) & 1;
            if (ks + 1 < KS) {
                read(kt, ks + 1, fa[nx], fb[nx]);
            } else {
                wait_vmcnt<LATER + DP>();  // this wave's DMA of k-tile kt + 1 landed
                lds_barrier();     // every wave's; every wave done with stage kt
                read(kt + 1, 0, fa[nx], fb[nx]);  // past the last k-tile: a stage never used, in bounds
            }
            mma(fa[ks & 1], fb[ks & 1]);
        }
    }
    wait_vmcnt<0>();
    lds_barrier();  // the ring is free

    // acc[i][j][4g + e]: y row wm*WM + i*32 + l%32, column
    // wn*128 + j*32 + 8g + 4(l/32) + e of the tile
    if constexpr (YF32) {
        // half a tile at a time through LDS (the rows of the waves with
        // wm = h; 16-byte chunk q of row r at q ^ (r & 15)), then
        // row-contiguous 16-byte stores
        float* ly = (float*)lds;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (wm == h) {
#pragma unroll
                for (int i = 0; i < MI; ++i) {
                    const int row = i * 32 + (l & 31);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
#pragma unroll
                        for (int g = 0; g < 4; ++g) {
                            const int q = (wn * 128 + j * 32 + 8 * g + 4 * (l >> 5)) >> 2;
                            *(f32x4*)(ly + row * PG_TN + 4 * (q ^ (row & 15))) =
                                f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                        }
                }
            }
            __syncthreads();
            float* yf = (float*)p.y + (int64_t)(m0 + h * WM) * p.ldy + n0;
            constexpr int PER = WM * PG_TN / 4 / PG_THREADS;
#pragma unroll
            for (int it = 0; it < PER; ++it) {
                const int idx = tid + PG_THREADS * it, row = idx >> 6, q = idx & 63;
                const f32x4 v = *(const f32x4*)(ly + row * PG_TN + 4 * (q ^ (row & 15)));
                if (m0 + h * WM + row < p.M && n0 + 4 * q < p.N) *(f32x4*)(yf + (int64_t)row * p.ldy + 4 * q) = v;
            }
            __syncthreads();
        }
    } else {
        // the bf16 tile through LDS (16-byte chunk q of row r at q ^ (r & 31)),
        // then row-contiguous 16-byte stores
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int row = wm * WM + i * 32 + (l & 31);
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int col = wn * 128 + j * 32 + 8 * g + 4 * (l >> 5);
                    const int q = (col >> 3) ^ (row & 31);
                    u32x2 v;
                    v[0] = pack_bf16x2_hw(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
                    v[1] = pack_bf16x2_hw(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                    *(u32x2*)(lds + row * PG_TN + 8 * q + (col & 7)) = v;
                }
        }
        __syncthreads();
        uint16_t* yb = (uint16_t*)p.y + (int64_t)m0 * p.ldy + n0;
        constexpr int PER = TM * PG_TN / 8 / PG_THREADS;
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int idx = tid + PG_THREADS * it, row = idx >> 5, q = idx & 31;
            const u32x4 v = *(const u32x4*)(lds + row * PG_TN + 8 * (q ^ (row & 31)));
            if (m0 + row < p.M && n0 + 8 * q < p.N) *(u32x4*)(yb + (int64_t)row * p.ldy + 8 * q) = v;
        }
    }
}

template <int TM, bool AFFINE, bool YF32>
hipError_t launch_tm(const ProjGemmStack& ps, hipStream_t st) {
    using S = PgShape<TM, AFFINE>;
    const int m_tiles = (ps.seg[0].M + TM - 1) / TM, n_tiles = ps.tile_end[ps.nseg - 1];
    const size_t lds = YF32 ? S::LDS_F32 : S::LDS_BF16;
    const auto kern = proj_gemm_kernel<TM, AFFINE, YF32>;
    const hipError_t attr = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(kern, dim3((unsigned)(m_tiles * n_tiles)), dim3(PG_THREADS), lds, st, ps);
    return hipGetLastError();
}

template <int TM, bool AFFINE>
hipError_t launch_y(const ProjGemmStack& ps, hipStream_t st) {
    return ps.seg[0].y_f32 ? launch_tm<TM, AFFINE, true>(ps, st) : launch_tm<TM, AFFINE, false>(ps, st);
}

}  // namespace

bool proj_gemm_ok(const ProjGemmParams& p) {
    const int bk = 32;
    if (p.M <= 0 || p.N <= 0 || p.N % 8 || p.K % bk || p.K < bk) return false;
    if (((uintptr_t)p.x & 15) || p.ldx % 8 || p.ldx < p.K || ((uintptr_t)p.y & 15) || p.ldy % (p.y_f32 ? 4 : 8) ||
        p.ldy < p.N)
        return false;
    // one tile's x rows within 32-bit byte offsets
    if ((int64_t)256 * p.ldx * 2 >= (1ll << 31)) return false;
    if (p.packed) {
        // 4 bits, a group that is a multiple of the 32-deep k-tile, 16-byte
        // aligned packed rows, 4-byte aligned scales and biases
        if (p.bits != 4 || p.group % 32 || p.K % p.group || ((uintptr_t)p.packed & 15)) return false;
        if (!p.scales || !p.biases || (((uintptr_t)p.scales | (uintptr_t)p.biases) & 3)) return false;
        if ((int64_t)p.N * (p.K / 2) >= (1ll << 32)) return false;  // packed byte offsets
        // 2-byte scales are fetched by the dword that holds them: an even
        // count keeps the last one's dword inside the buffer
        if (p.scale_dtype != 2 && ((int64_t)p.N * (p.K / p.group)) % 2) return false;
    } else {
        if (!p.w || ((uintptr_t)p.w & 15) || p.ldw % 8 || p.ldw < p.K || (int64_t)PG_TN * p.ldw * 2 >= (1ll << 31))
            return false;
    }
    return true;
}

hipError_t launch_proj_gemm_stack(const ProjGemmParams* segs, int n, int cu_count, hipStream_t st) {
    if (n < 1 || n > 3) return hipErrorInvalidValue;
    ProjGemmStack ps{};
    ps.nseg = n;
    int tiles = 0;
    for (int i = 0; i < 3; ++i) {
        if (i < n) {
            const ProjGemmParams& q = segs[i];
            if (!proj_gemm_ok(q) || q.M != segs[0].M || !q.packed != !segs[0].packed || q.y_f32 != segs[0].y_f32)
                return hipErrorInvalidValue;
            ps.seg[i] = q;
            tiles += (q.N + PG_TN - 1) / PG_TN;
            ps.tile_end[i] = tiles;
        } else {
            ps.tile_end[i] = INT32_MAX;
        }
    }
    // 256-row tiles when they alone fill the GPU, else 128
    const bool big = (int64_t)((segs[0].M + 255) / 256) * tiles >= cu_count;
    if (segs[0].packed) return big ? launch_y<256, true>(ps, st) : launch_y<128, true>(ps, st);
    return big ? launch_y<256, false>(ps, st) : launch_y<128, false>(ps, st);
}

hipError_t launch_proj_gemm(const ProjGemmParams& p, int cu_count, hipStream_t st) {
    return launch_proj_gemm_stack(&p, 1, cu_count, st);
}

}  // namespace mr
