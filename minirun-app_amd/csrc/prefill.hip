// Causal MLA prefill on gfx950 (K3MLA.forward eager branch, MLA.swift:159-168,
// 198-206; expand :231-245; causal mask :257-275).
//
// Two kernels:
//   upproj_kernel       kv[h][p][e] = latent[p] . kv_b[h*256 + e]: the
//                       per-head keys (e < 128, W_UK rows) and values (e >= 128,
//                       W_UV rows) of every cached position, one NT GEMM on
//                       32x32x16 bf16 MFMA (256 x 256 tiles, DMA-fed LDS
//                       ring), fp32 accumulation, bf16 out.
//   prefill_attn_kernel flash attention over those keys/values plus the
//                       shared rotary key, fp32 online softmax, bf16 P.
//
// The attention computes S^T = K . Q^T and O^T = V^T . P^T, so a lane owns
// one query: its row max, row sum and rescale never leave the lane except
// for one exchange between the two 32-lane halves that hold different keys.
// P goes from the S^T accumulators into the B operand of the PV product
// without a shuffle; V^T comes from row-major V tiles through
// ds_read_b64_tr_b16.
#include <algorithm>
#include <math.h>

#include <type_traits>

#include "mr_kernels.hpp"

namespace mr {

namespace {

// ---------------------------------------------------------------- up-projection
// C [M][N] = A [M][K] . B [N][K]^T, K = 512, with C stored in blocks of 256
// columns (one head's keys and values): column n of row m at
// c + (n / 256) * c_hs + m * ldc + n % 256, so a workgroup's 256 x 256 tile
// is one contiguous 128 KB block when ldc = 256.
//
// A 256 x 256 tile per workgroup of 4 waves, each wave a 128 x 128 block of
// 4 x 4 32x32x16 MFMA tiles (256 accumulators per lane, in AGPRs), so a
// 16-deep k-step reads 8 KB of operands per wave for 16 MFMAs.  The wave
// computes C^T blocks (B rows as the MFMA's first operand), so each lane
// ends with four runs of four consecutive N columns of one C row.
//
// K streams through two LDS stages (UG_STAGES) of UG_BK = 64 columns (A 32 KB
// + B 32 KB each, 128 KB in all) filled by global -> LDS DMA one stage
// ahead; a stage is 128-byte rows of eight 16-byte chunks, chunk c of row r
// in slot c ^ ((r >> 1) & 7) (ug_slot), so the 16 lanes of one ds_read_b128
// phase (16 consecutive rows, one chunk) hit 16 distinct bank groups.  The DMA writes
// slots in lane order, so lane l of a 1 KB instruction fetches the global
// chunk that belongs in slot l.  The operand fragments are read one 16-deep
// step ahead of the MFMAs that use them, and the one barrier per stage sits
// after 16 MFMAs, by when the reads it waits for have landed.
//
// Epilogue: bf16 C tile through LDS (128 KB of the ring), 16-byte
// chunk q of row r at q ^ (r & 31), then 16-byte row-contiguous stores.
constexpr int UG_TM = 256, UG_TN = 256, UG_BK = 64, UG_STAGES = 2;
constexpr int UG_THREADS = 256;
constexpr int UG_GROUP_M = 4;  // M tiles that share an L2 walk
constexpr int UG_STAGE_HALF = UG_TM * UG_BK;  // bf16 elements of A (or B) in one stage
constexpr int UG_CPR = UG_BK / 8;             // 16-byte chunks per stage row
constexpr int UG_KS = UG_BK / 16;             // 16-deep MFMA steps per stage
constexpr int UG_DPW = 2 * UG_CPR;            // DMA instructions per wave per stage
static_assert((UG_CPR == 4 || UG_CPR == 8) && UG_KS % 2 == 0, "stage shape");

// chunk c of stage row r: 16 consecutive rows read at one chunk land in 16
// distinct 16-byte bank groups
__device__ __forceinline__ int ug_slot(int r, int c) {
    return UG_CPR == 4 ? r * 4 + (c ^ ((r >> 2) & 3)) : r * 8 + (c ^ ((r >> 1) & 7));
}

// lds_barrier with its lgkmcnt(0) also issued as the builtin (gfx9 encoding:
// vmcnt 63, expcnt 7, lgkmcnt 0), so the compiler knows every earlier LDS
// read has landed and adds no waits for them after the barrier
__device__ __forceinline__ void lds_barrier_seen() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    lds_barrier();
}

__global__ void __launch_bounds__(UG_THREADS, 1) upproj_kernel(UpProjParams p) {
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[];  // UG_STAGES x (A, B), 160 KB
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int m_tiles = (p.M + UG_TM - 1) / UG_TM, n_tiles = p.N / UG_TN;
    const int total = m_tiles * n_tiles;
    // XCD-aware order: consecutive workgroups land on the 8 XCDs in turn, so
    // each XCD gets a contiguous range of tile ids; ids run over groups of
    // UG_GROUP_M M tiles, and within a group over the N tiles with the M
    // tiles fastest.  One XCD's 32 resident workgroups then cover 4 M x 8 N
    // tiles (1 MB of latent rows, 2 MB of kv_b rows), and its next rounds
    // keep the same latent rows in its L2.
    int bid = blockIdx.x;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
    const int group = bid / (UG_GROUP_M * n_tiles), first_m = group * UG_GROUP_M;
    const int gsize = min(m_tiles - first_m, UG_GROUP_M);
    const int mt = first_m + (bid % (UG_GROUP_M * n_tiles)) % gsize;
    const int nt = (bid % (UG_GROUP_M * n_tiles)) / gsize;
    const int m0 = mt * UG_TM, n0 = nt * UG_TN;
    const int KT = p.K / UG_BK;

    // DMA: a stage is 32 instructions of 64 lanes x 16 bytes (16 for A, 16
    // for B); wave w issues A and B instructions 4w .. 4w + 3.  Lane l of
    // instruction i fills slot 64 i + l: row 16 i + l / 4, slot chunk l % 4,
    // which holds global chunk (l % 4) ^ ((row >> 2) & 3).  Offsets are
    // bytes from the tile's first A (B) row; A rows past M repeat row M - 1.
    const uint16_t* abase = p.a + (int64_t)m0 * p.lda;
    const uint16_t* bbase = p.b + (int64_t)n0 * p.ldb;
    // instruction i of an operand (UG_CPR per wave): rows (64 / UG_CPR) i ..,
    // lane l fills slot 64 i + l = (row, slot chunk l % UG_CPR)
    uint32_t voff[UG_DPW];
#pragma unroll
    for (int q = 0; q < UG_DPW; ++q) {
        const int i = UG_CPR * w + q % UG_CPR;
        const int row = (64 / UG_CPR) * i + l / UG_CPR;
        const int sc = l % UG_CPR;
        const int c = UG_CPR == 4 ? sc ^ ((row >> 2) & 3) : sc ^ ((row >> 1) & 7);
        voff[q] = q < UG_CPR ? (uint32_t)(((int64_t)min(row, p.M - 1 - m0) * p.lda + 8 * c) * 2)
                             : (uint32_t)(((int64_t)row * p.ldb + 8 * c) * 2);
    }
    const int wu = __builtin_amdgcn_readfirstlane(w);
    auto issue = [&](int kt) {
        uint16_t* st = lds + (kt % UG_STAGES) * 2 * UG_STAGE_HALF;
        const uint32_t ko = (uint32_t)kt * UG_BK * 2;
#pragma unroll
        for (int q = 0; q < UG_CPR; ++q) dma16_off(abase, voff[q] + ko, st + 512 * (UG_CPR * wu + q));
#pragma unroll
        for (int q = 0; q < UG_CPR; ++q)
            dma16_off(bbase, voff[UG_CPR + q] + ko, st + UG_STAGE_HALF + 512 * (UG_CPR * wu + q));
    };
    // this wave's part of stage kt + 1 has landed once only the stages after
    // it that were issued (up to kt + UG_STAGES - 1) are pending
    auto wait_next = [&](int kt) {
        const int later = min(KT - 1, kt + UG_STAGES - 1) - (kt + 1);
        static_assert(UG_STAGES <= 5, "wait ladder");
        if (later >= 3)
            wait_vmcnt<3 * UG_DPW>();
        else if (later == 2)
            wait_vmcnt<2 * UG_DPW>();
        else if (later == 1)
            wait_vmcnt<UG_DPW>();
        else
            wait_vmcnt<0>();
    };

    const int wm = w >> 1, wn = w & 1;  // rows wm*128.., columns wn*128..
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    auto read = [&](int kt, int ks, bf16x8(&a)[4], bf16x8(&b)[4]) {
        const uint16_t* sa = lds + (kt % UG_STAGES) * 2 * UG_STAGE_HALF;
        const uint16_t* sb = sa + UG_STAGE_HALF;
        const int ch = 2 * ks + (l >> 5);
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *(const bf16x8*)(sa + 8 * ug_slot(wm * 128 + i * 32 + (l & 31), ch));
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = *(const bf16x8*)(sb + 8 * ug_slot(wn * 128 + j * 32 + (l & 31), ch));
    };
    auto mma = [&](const bf16x8(&a)[4], const bf16x8(&b)[4]) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma32(b[j], a[i], acc[i][j]);
    };

    // KT >= UG_STAGES (the launcher checks): stages 0 .. UG_STAGES - 1 in
    // flight, UG_DPW DMA instructions per wave each
#pragma unroll
    for (int s = 0; s < UG_STAGES; ++s) issue(s);
    wait_vmcnt<UG_DPW * (UG_STAGES - 1)>();
    lds_barrier_seen();
    bf16x8 fa[2][4], fb[2][4];  // fragments of two consecutive 16-deep steps
    read(0, 0, fa[0], fb[0]);
    // the last stage is peeled off so every path through the loop body is
    // the same for the compiler's LDS wait counts
    for (int kt = 0; kt + 1 < KT; ++kt) {
#pragma unroll
        for (int ks = 0; ks < UG_KS; ++ks) {
            const int nx = (ks + 1) & 1;
            if (ks + 1 < UG_KS) {
                read(kt, ks + 1, fa[nx], fb[nx]);
            } else {
                wait_next(kt);
                lds_barrier_seen();  // every wave's part landed; every wave is done with stage kt
                if (kt + UG_STAGES < KT) issue(kt + UG_STAGES);
                read(kt + 1, 0, fa[nx], fb[nx]);
            }
            mma(fa[ks & 1], fb[ks & 1]);
        }
    }
#pragma unroll
    for (int ks = 0; ks < UG_KS; ++ks) {
        if (ks + 1 < UG_KS) read(KT - 1, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
        mma(fa[ks & 1], fb[ks & 1]);
    }
    lds_barrier_seen();  // the ring is free

    // acc[i][j][4g + e]: C row wm*128 + i*32 + l%32, column
    // wn*128 + j*32 + 8g + 4(l/32) + e
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = wm * 128 + i * 32 + (l & 31);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int col = wn * 128 + j * 32 + 8 * g + 4 * (l >> 5);
                const int q = (col >> 3) ^ (row & 31);
                u32x2 v;
                v[0] = pack_bf16x2_hw(acc[i][j][4 * g], acc[i][j][4 * g + 1]);
                v[1] = pack_bf16x2_hw(acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                *(u32x2*)(lds + row * UG_TN + 8 * q + (col & 7)) = v;
            }
    }
    __syncthreads();
    uint16_t* cb = p.c + (int64_t)nt * p.c_hs + (int64_t)m0 * p.ldc;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        constexpr int PER = (UG_TM * UG_TN / 8) / UG_THREADS / 2;
        u32x4 v[PER];
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int idx = tid + UG_THREADS * (it + PER * half), row = idx >> 5, q = idx & 31;
            v[it] = *(const u32x4*)(lds + row * UG_TN + 8 * (q ^ (row & 31)));
        }
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int idx = tid + UG_THREADS * (it + PER * half), row = idx >> 5, q = idx & 31;
            if (m0 + row < p.M) *(u32x4*)(cb + (int64_t)row * p.ldc + 8 * q) = v[it];
        }
    }
}

// ---------------------------------------------------------------- attention
constexpr int AT_Q = 128;   // queries per workgroup (32 per wave)
constexpr int AT_K = 64;    // keys per tile
constexpr int AT_DV = 128;
constexpr float AT_TAU = 8.f;  // log2 headroom of the running max

// One tile: K nope [64][128] (256-byte rows), K rope [64][64] (128-byte
// rows), V [64][128].  LDS holds each region for both buffers side by side
// (Kn0 Kn1 | Kr0 Kr1 | V0 V1), so every read address is a per-lane base plus
// an immediate.  Chunk c (16 bytes) of nope row r sits at c ^ (r & 15); of
// rope row r at c ^ kr_swz(r); of V row r at c ^ ((r & 3) << 2).  The K
// reads below (lane = key row, one chunk for all lanes) hit distinct bank
// groups for every 8 and every 16 consecutive rows; in a V transposed read
// the 32 lanes of each half-wave cover 4 rows x 16 chunk halves, which the
// V swizzle spreads over all 64 banks.
constexpr int AT_KN_SZ = AT_K * 128, AT_KR_SZ = AT_K * 64, AT_V_SZ = AT_K * AT_DV;
constexpr int AT_NBUF = 2;  // tiles in LDS: one in use, one in flight
constexpr int AT_KR0 = AT_NBUF * AT_KN_SZ;          // rope region (elements)
constexpr int AT_V0 = AT_KR0 + AT_NBUF * AT_KR_SZ;  // V region
constexpr int AT_LDS = AT_V0 + AT_NBUF * AT_V_SZ;   // 80 KB
__device__ __forceinline__ int kr_swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
__device__ __forceinline__ int kn_off(int r, int c) { return r * 128 + ((c ^ (r & 15)) << 3); }
__device__ __forceinline__ int kr_off(int r, int c) { return r * 64 + ((c ^ kr_swz(r)) << 3); }
__device__ __forceinline__ int v_off(int r, int d) { return r * AT_DV + ((((d >> 3) ^ ((r & 3) << 2))) << 3) + (d & 7); }

__global__ void __launch_bounds__(256, 2) prefill_attn_kernel(PrefillAttnParams p) {
    __shared__ __attribute__((aligned(1024))) uint16_t lds[AT_LDS];  // 80 KB: two workgroups per CU
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, lq = l & 31, hh = l >> 5;

    // work item: (head, query tile); one XCD takes all query tiles of a head
    // (heaviest first) so that head's keys and values stay in its L2
    const int qtiles = (p.T + AT_Q - 1) / AT_Q;
    const int total = qtiles * p.H;
    int head, qt;
    if ((p.H & 7) == 0) {
        const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
        head = (slot / qtiles) * 8 + xcd;
        qt = qtiles - 1 - slot % qtiles;
    } else {
        head = blockIdx.x / qtiles;
        qt = qtiles - 1 - blockIdx.x % qtiles;
    }
    if (head >= p.H || blockIdx.x >= total) return;
    const int q0 = qt * AT_Q;
    const int off = p.P - p.T;  // query i sits at position off + i

    // this lane's query as a column of S^T; its 192 features as the B operand
    const int qi = q0 + 32 * w + lq;
    const uint16_t* qp = p.q + (int64_t)min(qi, p.T - 1) * p.q_ts + (int64_t)head * p.q_hs;
    bf16x8 qf[12];
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) qf[ks] = *(const bf16x8*)(qp + 16 * ks + 8 * hh);
    // take the Q loads as complete here: otherwise the compiler's own wait
    // for them lands inside the tile loop, where it would also wait for the
    // tile DMA in flight
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) asm volatile("" ::"v"(qf[ks]));
    const int q_limit = off + qi;  // keys <= q_limit are visible

    const int wg_kend = off + min(q0 + AT_Q, p.T);  // keys [0, wg_kend) for the workgroup
    const int ntiles = (wg_kend + AT_K - 1) / AT_K;
    const int wave_first = off + q0 + 32 * w;              // smallest visible limit in this wave
    // keys this wave can see (none when all its queries lie past T)
    const int wave_kend = q0 + 32 * w < p.T ? off + min(q0 + 32 * w + 32, p.T) : 0;

    // Tile DMA (buffer_load_dwordx4 ... lds, 1 KB per wave instruction, 10
    // per wave): LDS slot s of a region holds the swizzled chunk, so its
    // source is the inverse-swizzled chunk.  The byte offsets within a tile
    // are the same for every tile; the tile base and its length ride in the
    // buffer resources, so rows past the last key load as zeros (their
    // scores are masked and their P entries are zero).
    const uint32_t kv_rb = (uint32_t)p.kv_rs * 2u, rope_rb = (uint32_t)p.rope_rs * 2u;
    uint32_t vo_n[4], vo_v[4], vo_r[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int sl = 64 * (w + 4 * i) + l, r = sl >> 4, pc = sl & 15;
        vo_n[i] = r * kv_rb + ((pc ^ (r & 15)) << 4);
        vo_v[i] = r * kv_rb + 256u + ((pc ^ ((r & 3) << 2)) << 4);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int sl = 64 * (w + 4 * i) + l, r = sl >> 3, pc = sl & 7;
        vo_r[i] = r * rope_rb + ((pc ^ kr_swz(r)) << 4);
    }
    const uint16_t* kv_h = p.kv + (int64_t)head * p.kv_hs;
    const int wu = __builtin_amdgcn_readfirstlane(w);  // LDS destinations in SGPRs
    auto issue = [&](int kt, int buf) {
        const uint32_t rows = (uint32_t)min(p.P - kt * AT_K, AT_K);
        const i32x4 rkv = buffer_rsrc(kv_h + (int64_t)kt * AT_K * p.kv_rs, rows * kv_rb);
        const i32x4 rro = buffer_rsrc(p.rope + (int64_t)kt * AT_K * p.rope_rs, rows * rope_rb);
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16_buf(rkv, vo_n[i], lds + buf * AT_KN_SZ + 512 * (wu + 4 * i));
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16_buf(rro, vo_r[i], lds + AT_KR0 + buf * AT_KR_SZ + 512 * (wu + 4 * i));
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16_buf(rkv, vo_v[i], lds + AT_V0 + buf * AT_V_SZ + 512 * (wu + 4 * i));
    };

    float m_run = -INFINITY, l_part = 0.f;
    f32x16 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = f32x16{};

    // tr-read addressing for the V^T operand (fixed per lane)
    const int g = l >> 4, j = l & 15;
    const int tr_key = 4 * (g >> 1) + (j >> 2);
    const int tr_d = 16 * (g & 1) + 4 * (j & 3);

    // one 64-key tile for this wave's 32 queries; DIAG applies the causal mask
    auto tile = [&](auto diag_tag, auto buf_tag, int k0) {
        constexpr bool DIAG = decltype(diag_tag)::value;
        constexpr int B = decltype(buf_tag)::value;
        const uint16_t* kn = lds + B * AT_KN_SZ;
        const uint16_t* kr = lds + AT_KR0 + B * AT_KR_SZ;
        const uint16_t* vt = lds + AT_V0 + B * AT_V_SZ;
        // S^T = K . Q^T: two 32-key blocks, 12 k-steps of 16 features (8
        // nope, 4 rope); the A operands come in double-buffered groups of 4
        // (two k-steps x both blocks), so each group's LDS reads overlap the
        // previous group's MFMAs (the fences keep the scheduler from
        // hoisting all 24 reads)
        f32x16 s[2] = {f32x16{}, f32x16{}};
        bf16x8 ga[2][4];
        auto qk_a = [&](int ks, int kb) -> bf16x8 {
            const int r = kb * 32 + lq, c = 2 * ks + hh;
            return *(const bf16x8*)(ks < 8 ? kn + kn_off(r, c) : kr + kr_off(r, c - 16));
        };
#pragma unroll
        for (int e = 0; e < 4; ++e) ga[0][e] = qk_a(e >> 1, e & 1);
        // the two waves sharing a SIMD (one from each workgroup) take turns:
        // the wave in an MFMA phase issues first, the other's softmax fills in
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int gq = 0; gq < 6; ++gq) {
            if (gq + 1 < 6) {
#pragma unroll
                for (int e = 0; e < 4; ++e) ga[(gq + 1) & 1][e] = qk_a(2 * (gq + 1) + (e >> 1), e & 1);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int e = 0; e < 4; ++e) s[e & 1] = mfma32(ga[gq & 1][e], qf[2 * gq + (e >> 1)], s[e & 1]);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
        // causal mask on raw scores, running max (lane = query, 32 of its keys)
        float mx = -INFINITY;
        const int lim = q_limit - k0 - 4 * hh;  // tile key index kb*32 + 8*(i>>2) + (i&3) visible iff <= lim
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (DIAG && kb * 32 + 8 * (i >> 2) + (i & 3) > lim) s[kb][i] = -INFINITY;
                mx = fmaxf(mx, s[kb][i]);
            }
        mx = xor32_max(mx) * p.scale_log2;  // scale > 0 keeps the order
        // the reference max rises only when a score passes it by AT_TAU
        // (log2 units), so O is rescaled on few tiles (P <= 2^AT_TAU); key 0
        // is visible to every query, so the first tile always sets a finite
        // reference
        const bool raise = mx > m_run + AT_TAU;  // false while mx is -inf
        if (__builtin_amdgcn_ballot_w64(raise)) {
            const float m_new = raise ? mx : m_run;
            const float alpha = raise ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.f;
            m_run = m_new;
            l_part *= alpha;
#pragma unroll
            for (int d = 0; d < 4; ++d) o[d] *= alpha;
        }
        // four partial sums, so the additions are not one serial chain
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float e = __builtin_amdgcn_exp2f(fmaf(s[kb][i], p.scale_log2, -m_run));
                s[kb][i] = e;
                ls[i & 3] += e;
            }
        l_part += (ls[0] + ls[1]) + (ls[2] + ls[3]);

        // O^T += V^T . P^T: k-step t covers tile keys 16t .. 16t+15.  The
        // transposed V reads of step t + 1 go out before step t's products
        // (two fragment sets), so no product waits for its own reads.
        __builtin_amdgcn_s_setprio(1);
        bf16x8 va[2][4];
        auto vread = [&](int t, bf16x8(&a)[4]) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const int d = 32 * db + tr_d;
                const bf16x4 lo = ds_read_tr16(vt + v_off(16 * t + tr_key, d));
                const bf16x4 hi = ds_read_tr16(vt + v_off(16 * t + 8 + tr_key, d));
                a[db] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
        };
        vread(0, va[0]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (t + 1 < 4) vread(t + 1, va[(t + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            const int kb = t >> 1, base = 8 * (t & 1);
            bf16x8 pb;
#pragma unroll
            for (int e = 0; e < 8; ++e) pb[e] = (__bf16)s[kb][base + e];
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] = mfma32(va[t & 1][db], pb, o[db]);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
    };

    // tile 0 in flight, wait for it
    issue(0, 0);
    wait_vmcnt<0>();
    lds_barrier();
    // tile kt lives in buffer kt & 1; the loop takes two tiles per trip so
    // the buffer of each is a constant
    auto step = [&](int kt, auto buf_tag) {
        constexpr int B = decltype(buf_tag)::value;
        // refill the other buffer (tile kt-1, read before the last barrier)
        if (kt + 1 < ntiles) issue(kt + 1, B ^ 1);
        const int k0 = kt * AT_K;
        if (k0 < wave_kend) {  // else every query of this wave is past this tile
            if (k0 + AT_K - 1 > wave_first)
                tile(std::true_type{}, buf_tag, k0);
            else
                tile(std::false_type{}, buf_tag, k0);
        }
        // tile kt+1 must have landed
        if (kt + 1 < ntiles) wait_vmcnt<0>();
        lds_barrier();
    };
    for (int kt = 0; kt < ntiles; kt += 2) {
        step(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < ntiles) step(kt + 1, std::integral_constant<int, 1>{});
    }

    // the gate chunks this lane stores below, requested before the
    // normalisation and the LDS staging so that their latency overlaps them;
    // the gate and the output stream past L2 (nontemporal), which keeps the
    // keys and values that later query tiles of this head read
    u32x4 gv[8];
    const bool gated = p.gate != nullptr && !p.out_f32;
    if (gated) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = l + 64 * i, qq = min(q0 + 32 * w + (q >> 4), p.T - 1);
            gv[i] = __builtin_nontemporal_load((const u32x4*)(p.gate + (int64_t)qq * p.gate_ts + head * AT_DV +
                                                              (q & 15) * 8));
        }
    }

    // normalise: the two halves of the wave hold partial sums of one query
    const float l_tot = xor32_sum(l_part);
    const float inv = 1.f / l_tot;
    const bool q_ok = qi < p.T;
    if (p.out_f32) {
        float* op = (float*)p.out + (int64_t)qi * p.out_ts + (int64_t)head * p.out_hs;
        if (q_ok) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int d = 32 * db + 8 * r4 + 4 * hh;
                    *(f32x4*)(op + d) = f32x4{o[db][4 * r4] * inv, o[db][4 * r4 + 1] * inv, o[db][4 * r4 + 2] * inv,
                                              o[db][4 * r4 + 3] * inv};
                }
        }
        return;
    }
    // bf16: stage this wave's [32 queries][128] tile in LDS, then store rows.
    // The 8-byte piece (query lq, chunk c, half hh) sits at chunk c ^ (lq & 15),
    // half hh ^ (lq >> 4): the 32 lanes of a half-wave write 32 distinct bank
    // pairs, and a row read back is one row's 16 chunks.
    __syncthreads();
    uint16_t* st = lds + w * 32 * AT_DV;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int c = 4 * db + r4;
            u32x2 v;
            v[0] = pack_bf16x2(o[db][4 * r4] * inv, o[db][4 * r4 + 1] * inv);
            v[1] = pack_bf16x2(o[db][4 * r4 + 2] * inv, o[db][4 * r4 + 3] * inv);
            *(u32x2*)(st + lq * AT_DV + ((c ^ (lq & 15)) << 3) + 4 * (hh ^ (lq >> 4))) = v;
        }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = l + 64 * i, row = q >> 4, ch = q & 15;  // 32 rows x 16 chunks
        const int qq = q0 + 32 * w + row;
        u32x4 v = *(const u32x4*)(st + row * AT_DV + ((ch ^ (row & 15)) << 3));
        if (row >> 4) v = u32x4{v[2], v[3], v[0], v[1]};
        if (qq >= p.T) continue;
        if (gated) {
#pragma unroll
            for (int k = 0; k < 4; ++k) v[k] = gated_bf16x2(v[k], gv[i][k]);
        }
        __builtin_nontemporal_store(v, (u32x4*)((uint16_t*)p.out + (int64_t)qq * p.out_ts + (int64_t)head * p.out_hs +
                                                ch * 8));
    }
}

}  // namespace

hipError_t launch_upproj(const UpProjParams& p, hipStream_t st) {
    // N a multiple of 256, K a multiple of 32 with at least UG_STAGES steps,
    // rows 16-byte aligned, one tile's A / B rows within 32-bit byte offsets
    if (p.N % UG_TN || p.K % UG_BK || p.K < UG_BK * UG_STAGES || (int64_t)UG_TM * p.lda * 2 >= (1ll << 32) ||
        (int64_t)UG_TN * p.ldb * 2 >= (1ll << 32))
        return hipErrorInvalidValue;
    const int m_tiles = (p.M + UG_TM - 1) / UG_TM;
    const unsigned grid = (unsigned)(m_tiles * (p.N / UG_TN));
    const size_t lds = sizeof(uint16_t) * UG_STAGES * 2 * UG_STAGE_HALF;
    const hipError_t attr =
        hipFuncSetAttribute((const void*)upproj_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(upproj_kernel, dim3(grid), dim3(UG_THREADS), lds, st, p);
    return hipGetLastError();
}

hipError_t launch_prefill_attn(const PrefillAttnParams& p, hipStream_t st) {
    const int qtiles = (p.T + AT_Q - 1) / AT_Q;
    const unsigned grid = (unsigned)(qtiles * p.H);
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
