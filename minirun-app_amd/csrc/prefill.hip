// Causal MLA prefill on gfx950 (K3MLA.forward eager branch, MLA.swift:159-168,
// 198-206; expand :231-245; causal mask :257-275).
//
// Two kernels:
//   upproj_kernel       kv[p][h*256 + e] = latent[p] . kv_b[h*256 + e]: the
//                       per-head keys (e < 128, W_UK rows) and values (e >= 128,
//                       W_UV rows) of every cached position, one NT GEMM on
//                       32x32x16 bf16 MFMA, fp32 accumulation, bf16 out.
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
constexpr int UG_TILE = 128;  // M and N tile
constexpr int UG_BK = 32;     // K per stage

// 64-byte LDS rows of 4 x 16-byte chunks; chunk c of row r sits at
// c ^ ((r >> 2) & 3): 16 consecutive rows read at one chunk hit 16
// distinct bank groups.
__device__ __forceinline__ int ug_off(int r, int c) { return r * UG_BK + ((c ^ ((r >> 2) & 3)) << 3); }

__global__ void __launch_bounds__(256, 2) upproj_kernel(UpProjParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[4 * UG_TILE * UG_BK];  // 2 stages x (A, B): 32 KB
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int m_tiles = (p.M + UG_TILE - 1) / UG_TILE;
    const int total = m_tiles * (p.N / UG_TILE);
    // XCD-aware order: the workgroups one XCD runs are consecutive tiles,
    // which share an N tile (kv_b rows) across all M tiles
    int bid = blockIdx.x;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
    const int mt = bid % m_tiles, nt = bid / m_tiles;
    const int m0 = mt * UG_TILE, n0 = nt * UG_TILE;

    // stage s: A tile at lds + 2s * 4096, B tile right after it
    auto sa = [&](int s) { return lds + (2 * s) * UG_TILE * UG_BK; };
    auto sb = [&](int s) { return lds + (2 * s + 1) * UG_TILE * UG_BK; };
    u32x4 ra[2], rb[2];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int q = tid + 256 * i, row = q >> 2, ch = q & 3;
            const int am = min(m0 + row, p.M - 1);
            ra[i] = *(const u32x4*)(p.a + (int64_t)am * p.lda + k0 + ch * 8);
            rb[i] = *(const u32x4*)(p.b + (int64_t)(n0 + row) * p.ldb + k0 + ch * 8);
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int q = tid + 256 * i, row = q >> 2, ch = q & 3;
            *(u32x4*)(sa(buf) + ug_off(row, ch)) = ra[i];
            *(u32x4*)(sb(buf) + ug_off(row, ch)) = rb[i];
        }
    };

    const int wm = w >> 1, wn = w & 1;  // this wave's 64 x 64 sub-tile
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    const int ksteps = p.K / UG_BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < ksteps; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ksteps) gload((kt + 1) * UG_BK);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            bf16x8 av[2], bv[2];
            const int ch = 2 * ks + (l >> 5);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                av[i] = *(const bf16x8*)(sa(buf) + ug_off(wm * 64 + i * 32 + (l & 31), ch));
                bv[i] = *(const bf16x8*)(sb(buf) + ug_off(wn * 64 + i * 32 + (l & 31), ch));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = mfma32(av[i], bv[j], acc[i][j]);
        }
        if (kt + 1 < ksteps) sstore(buf ^ 1);
        __syncthreads();
    }

    // epilogue: the 128 x 128 bf16 tile through LDS (32 KB), then 16-byte
    // row-contiguous stores
    uint16_t* tile = lds;  // [128][128]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
                const int col = wn * 64 + j * 32 + (l & 31);
                tile[row * UG_TILE + col] = f32_to_bf16_bits(acc[i][j][r]);
            }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = tid + 256 * i, row = q >> 4, ch = q & 15;
        if (m0 + row < p.M)
            *(u32x4*)(p.c + (int64_t)(m0 + row) * p.ldc + n0 + ch * 8) = *(const u32x4*)(tile + row * UG_TILE + ch * 8);
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
    const uint16_t* kv_h = p.kv + (int64_t)head * 256;
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
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float e = __builtin_amdgcn_exp2f(fmaf(s[kb][i], p.scale_log2, -m_run));
                s[kb][i] = e;
                ls += e;
            }
        l_part += ls;

        // O^T += V^T . P^T: k-step t covers tile keys 16t .. 16t+15
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int kb = t >> 1, base = 8 * (t & 1);
            bf16x8 pb;
#pragma unroll
            for (int e = 0; e < 8; ++e) pb[e] = (__bf16)s[kb][base + e];
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const int d = 32 * db + tr_d;
                const bf16x4 lo = ds_read_tr16(vt + v_off(16 * t + tr_key, d));
                const bf16x4 hi = ds_read_tr16(vt + v_off(16 * t + 8 + tr_key, d));
                const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[db] = mfma32(a, pb, o[db]);
            }
        }
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
        if (qq < p.T) *(u32x4*)((uint16_t*)p.out + (int64_t)qq * p.out_ts + (int64_t)head * p.out_hs + ch * 8) = v;
    }
}

}  // namespace

hipError_t launch_upproj(const UpProjParams& p, hipStream_t st) {
    const int m_tiles = (p.M + UG_TILE - 1) / UG_TILE;
    const unsigned grid = (unsigned)(m_tiles * (p.N / UG_TILE));
    hipLaunchKernelGGL(upproj_kernel, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_prefill_attn(const PrefillAttnParams& p, hipStream_t st) {
    const int qtiles = (p.T + AT_Q - 1) / AT_Q;
    const unsigned grid = (unsigned)(qtiles * p.H);
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace mr
