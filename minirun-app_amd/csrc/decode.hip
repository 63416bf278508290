// Absorbed-latent MLA decode and index-driven sparse decode for gfx950.
//
// Computes, per (batch b, head h), over the selected cache rows c_n:
//   s_n   = (q_lat[h] . c_n[0:R] + q_rope[h] . c_n[R:R+dr]) * scale
//   out_h = sum_n softmax(s)_n * c_n[0:R]              (R = 512)
// which is the absorbed branch of K3MLA.forward (MLA.swift:188-196) and, with
// an index list and optional sinks, DeepSeekV4SparseAttention.expressingBatched
// (DeepSeekV4Attention.swift:861-920) with K = row[0:R+dr], V = row[0:R].
//
// Decomposition (one workgroup per CU; mla_decode_ws below has the details):
//   grid unit   = (batch, context split) x head group of 64 heads (32 when
//                 there are at most 32 heads)
//   blockIdx    -> XCD-aware: the head groups of one unit share blockIdx % 8,
//                  so they run on one XCD and read the same rows through its L2
//   sub-chunk   = 32 cache rows, global -> LDS by DMA (global_load_lds_dwordx4),
//                 4 buffers; 16-byte chunks XOR-swizzled
//   QK waves    = Q straight from global memory into registers, then
//                 S^T = K . Q^T on MFMA, online base-2 softmax, P to LDS
//   PV waves    = O^T = V^T . P^T on MFMA (V^T by ds_read_b64_tr_b16), one
//                 sub-chunk behind the QK waves; they issue all the DMA
//   epilogue    = O_s / l_s and (m_s, l_s) per (unit, head) into the
//                 workspace; mla_combine merges the splits (and the sink term)
//   index check = with a device status buffer, `batch` extra workgroups at the
//                 front of the gathered launch check each token's list
//                 (validate_token) while the others attend
#include <type_traits>

#include "mr_kernels.hpp"

namespace mr {

namespace {

constexpr int R = 512;
constexpr int ROWS = 32;      // rows per sub-chunk
constexpr int NBUF = 4;       // LDS sub-chunk buffers (3 in flight while one is consumed)
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
    // c < 64: c ^ (r & 15); the rope chunks 64 + j (j < 8): 64 + (j ^ (r & 7)),
    // which is c ^ (r & 7) -- one select, no branch
    return c ^ (r & (c < 64 ? 15 : 7));
}

constexpr float TAU = 8.f;  // log2 headroom before the running max is raised

// Partial record of (batch b, head, split): [batch][h_pad][splits] order, so
// the splits of one head are contiguous for the combine.
__device__ __forceinline__ int64_t part_rec(const DecodeParams& p, int b, int head, int split) {
    return ((int64_t)b * p.h_pad + head) * p.splits + split;
}

// Index checks of one token's list, DeepSeekV4SparseAttention
// (DeepSeekV4Attention.swift:884-895): the reference walks the entries in
// order, skips -1, and stops at the first entry outside [0, n_rows) or equal
// to an earlier entry.  One workgroup does it with no sort: every in-range
// value goes into an open-addressing table (linear probing, Fibonacci hash
// mapped onto `slots` by a multiply-high; a power of two with at least two
// slots per entry for lists of up to 8192, else at least 1.6 per entry) that
// keeps the smallest position holding the value; an entry is a repeat
// exactly when its position is not its value's smallest.  The first error is
// the smallest position that is out of range or a repeat.  res = (status,
// position, value), (MR_OK, -1, -1) for a valid list.  `table` holds
// 2 * validate_slots(n_idx) int32: in LDS for lists of up to
// VALIDATE_LDS_MAX_IDX entries, else in global memory (the workspace), where
// every access is a workgroup-scope atomic so the workgroup's own updates
// are what it reads.
__host__ __device__ constexpr int validate_slots(int n_idx) {
    if (n_idx <= 8192) {  // a power of two, at least twice the entries (the multiply-high below is then a shift)
        int slots = 64;
        while (slots < 2 * n_idx) slots *= 2;
        return slots;
    }
    return ((n_idx * 8 + 4) / 5 + 1 + 63) / 64 * 64;  // at least 1.6 slots per entry
}
constexpr int VALIDATE_LDS_BYTES = 131072;  // a check workgroup's LDS table (the smallest decode row ring)
constexpr int VALIDATE_LDS_MAX_IDX = 10176;
static_assert(validate_slots(VALIDATE_LDS_MAX_IDX) * 8 <= VALIDATE_LDS_BYTES, "LDS index table");
constexpr int VALIDATE_MAX_IDX = 1 << 22;  // longest list the checks take (table in the workspace)

template <bool GLOBAL_TABLE>
__device__ void validate_token(const int32_t* __restrict__ ind, int32_t n_idx, int32_t n_rows, int32_t* table, int nt,
                               int tid, int32_t* res) {
    __shared__ int32_t first_range, first_dup;
    const uint32_t slots = (uint32_t)validate_slots(n_idx);
    int32_t* key = table;
    int32_t* minpos = table + slots;
    // LDS: plain ds operations; global memory: workgroup-scope atomics
    auto ld = [](int32_t* a) {
        if constexpr (GLOBAL_TABLE) return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else return *a;
    };
    auto st = [](int32_t* a, int32_t v) {
        if constexpr (GLOBAL_TABLE) __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else *a = v;
    };
    for (uint32_t i = tid; i < slots; i += nt) {
        st(key + i, -1);
        st(minpos + i, 0x7fffffff);
    }
    if (tid == 0) {
        first_range = 0x7fffffff;
        first_dup = 0x7fffffff;
    }
    __syncthreads();
    auto home = [&](int32_t v) { return (uint32_t)(((uint64_t)((uint32_t)v * 2654435761u) * slots) >> 32); };
    auto next = [&](uint32_t h) { return h + 1 == slots ? 0u : h + 1; };
    for (int i = tid; i < n_idx; i += nt) {
        const int32_t v = ind[i];
        if (v == -1) continue;
        if (v < 0 || v >= n_rows) {
            atomicMin(&first_range, i);
            continue;
        }
        uint32_t h = home(v);
        for (uint32_t t = 0; t < slots; ++t) {  // the table is never full: ends within `slots` probes
            int32_t prev;
            if constexpr (GLOBAL_TABLE) {
                prev = -1;
                __hip_atomic_compare_exchange_strong(key + h, &prev, v, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP);
            } else {
                prev = atomicCAS(key + h, -1, v);
            }
            if (prev == -1 || prev == v) {
                if constexpr (GLOBAL_TABLE)
                    __hip_atomic_fetch_min(minpos + h, i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                else
                    atomicMin(minpos + h, i);
                break;
            }
            h = next(h);
        }
    }
    __syncthreads();
    for (int i = tid; i < n_idx; i += nt) {
        const int32_t v = ind[i];
        if (v < 0 || v >= n_rows) continue;
        uint32_t h = home(v);
        for (uint32_t t = 0; t < slots && ld(key + h) != v; ++t) h = next(h);
        if (ld(minpos + h) != i) atomicMin(&first_dup, i);
    }
    __syncthreads();
    if (tid == 0) {
        const int32_t fr = first_range, fd = first_dup;
        if (fr == 0x7fffffff && fd == 0x7fffffff) {
            res[0] = 0;
            res[1] = -1;
            res[2] = -1;
        } else {
            const int32_t pos = fr < fd ? fr : fd;
            res[0] = fr < fd ? 3 /* MR_INDEX_OUT_OF_RANGE */ : 4 /* MR_DUPLICATE_INDEX */;
            res[1] = pos;
            res[2] = ind[pos];
        }
    }
}

// ---------------------------------------------------------------------------
// Role-split variant for head groups of HGS heads (32, 48 or 64).  HGS/32 QK
// waves score 32 heads each over all 32 rows of a sub-chunk as
// S^T = K . Q^T on 32x32x16 MFMA: a lane owns one head, so its running max
// and sum stay in the lane (one exchange between the wave halves), and each
// cache row is read from LDS once per 32 heads; P goes to LDS as
// [head][key].  Four PV waves own 128 output columns each, run one
// sub-chunk behind the QK waves and issue all the DMA.  One barrier per phase: in phase j the QK
// waves turn sub-chunk j into P buffer j&1 while the PV waves consume P
// buffer (j-1)&1 with the rows of j-1 and refill the buffer of j-2 with
// j+2.  Each role runs its own loop, so neither carries the other's
// registers.
// Key row behind k position p of a 32-row sub-chunk in the role-split
// kernel: within each group of eight, positions 0..3 take the even rows and
// 4..7 the odd ones, so the four rows of a transposed read fall on distinct
// swizzle classes (bank-conflict free) while S^T rows and P columns keep the
// same order.
__device__ __forceinline__ int ksig(int p) {
    const int j = p & 7;
    return (p & ~7) | (j < 4 ? 2 * j : 2 * (j - 4) + 1);
}

// QK waves of 32 heads (32x32x16 MFMA) or, with QK16, of 16 heads (16x16x32
// MFMA): a 64-head group then has one QK wave per SIMD beside each PV wave.
template <int HGS, bool QK16>
struct WsShape {
    static constexpr int QKW = QK16 ? HGS / 16 : HGS / 32;  // QK waves
    static constexpr int THREADS = 64 * (QKW + 4);          // + 4 PV waves
};

template <int DR, bool GATHER, bool PACKED, int HGS, bool QK16>
__global__ void __launch_bounds__((WsShape<HGS, QK16>::THREADS), 1) mla_decode_ws(DecodeParams p_arg) {
    // every launch parameter in one batch of scalar loads: loaded where each
    // is first used, they would be several dependent memory round trips
    // before the first row load
    const DecodeParams p = load_params(p_arg);
    using G = Geo<DR>;
    constexpr int QKW = WsShape<HGS, QK16>::QKW;
    constexpr int NT = WsShape<HGS, QK16>::THREADS;
    constexpr int HT = HGS / 16;  // 16-head tiles of a PV wave
    __shared__ __attribute__((aligned(1024))) char cbuf[NBUF * G::BUF];
    __shared__ __attribute__((aligned(16))) char pbuf[2][HGS * PSTR];
    __shared__ __attribute__((aligned(16))) float alpha_s[2][HGS];
    __shared__ __attribute__((aligned(16))) float l_s[HGS];
    __shared__ int flag_s[2][QKW];
    __shared__ int32_t idx_s[GATHER ? MAX_GATHER_ROWS : 1];

    if (GATHER && (int)blockIdx.x < p.check_blocks) {  // index-check workgroups
        if ((int)blockIdx.x < p.batch)
        {
            const int32_t* ind = p.indices + (int64_t)blockIdx.x * p.n_idx;
            int32_t* res = p.index_status + 3 * blockIdx.x;
            if (p.check_table)
                validate_token<true>(ind, p.n_idx, p.n_ctx, p.check_table + (int64_t)blockIdx.x * 2 * validate_slots(p.n_idx),
                                     NT, threadIdx.x, res);
            else
                validate_token<false>(ind, p.n_idx, p.n_ctx, (int32_t*)cbuf, NT, threadIdx.x, res);
        }
        return;
    }
    const int bid = blockIdx.x - (GATHER ? p.check_blocks : 0);
    const int xcd = bid & 7;
    const int qb = bid >> 3;
    // the divisions by multiply-high: the code before the first loads is
    // fetched cold by every CU at each launch, so it is kept short
    const int qg = p.hg_magic ? (int)__umulhi((uint32_t)qb, p.hg_magic) : qb / p.head_groups;
    const int hg = qb - qg * p.head_groups;
    const int unit = qg * 8 + xcd;
    if (unit >= p.batch * p.splits) return;
    const int b = p.split_magic ? (int)__umulhi((uint32_t)unit, p.split_magic) : unit / p.splits;
    const int split = unit - b * p.splits;
    const int row_begin = split * p.rows_per_split;
    const int row_end = min(row_begin + p.rows_per_split, p.n_rows);
    const int nrows = max(row_end - row_begin, 0);
    const int nsub = (nrows + ROWS - 1) / ROWS;

    const int tid = threadIdx.x;
    const int l = tid & 63;
    const int lg = l >> 4;
    const int lc = l & 15;
    const int wu = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform role choice
    const bool is_qk = wu < QKW;
    const int qw = wu;        // QK wave: 32-head tile
    const int pw = wu - QKW;  // PV wave: 128-column quarter

    const uint16_t* lat = p.latent + (int64_t)b * p.lat_bs;
    const uint16_t* rop = DR ? p.rope + (int64_t)b * p.rope_bs : nullptr;

    if (GATHER) {
        const int32_t* ind = p.indices + (int64_t)b * p.n_idx;
        for (int i = tid; i < nrows; i += NT) {
            const int32_t v = ind[row_begin + i];
            idx_s[i] = (v >= 0 && v < p.n_ctx) ? v : -1;
        }
        __syncthreads();
    }

    const float scale2 = p.scale_log2;
    // staging of the partial record after the last phase: rows of 512 values
    // padded by 16 bytes, so the four lane groups' rows fall on distinct banks
    const int esz = p.ws_f32 ? 4 : 2;
    const int srow = R * esz + 16;

    if (is_qk) {
        if constexpr (QK16) {
        // ---------------------------------------------------------- QK role, 16 heads
        // B operand of 16x16x32: head 16qw + l%16, k = 32ks + 8(l/16)..+7
        const int hq = 16 * qw + (l & 15);  // this lane's head within the group
        const int kg = l >> 4;              // k group; output row group
        // Q straight from global memory into registers, in flight with the
        // PV waves' first row loads (16-byte pieces: chunk 4ks + kg of head hq)
        bf16x8 qreg[G::KS];
        {
            const int h0 = hg * HGS + hq;
            const int hh = h0 < p.heads ? h0 : 0;  // padding heads score head 0's query
            const uint16_t* ql = p.q_lat + (int64_t)b * p.q_lat_bs + (int64_t)hh * p.q_lat_hs;
            const uint16_t* qr = DR ? p.q_rope + (int64_t)b * p.q_rope_bs + (int64_t)hh * p.q_rope_hs : nullptr;
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks) {
                const int c = 4 * ks + kg;
                qreg[ks] = c < R / 8 ? *(const bf16x8*)(ql + 8 * c) : *(const bf16x8*)(qr + 8 * (c - R / 8));
            }
        }
        // A operand of row tile rt: key row ksig(16rt + l%16) of the
        // sub-chunk, chunk 4ks + kg; with the row swizzle, latent chunk
        // 16v + 4u + kg sits at 256v + qo[rt][u], rope k-steps at ro[rt][.]
        int qo[2][4], ro[2][2];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
            const int ar = ksig(16 * rt + (l & 15));
#pragma unroll
            for (int u = 0; u < 4; ++u) qo[rt][u] = ar * G::ROWB + 16 * ((4 * u + kg) ^ (ar & 15));
#pragma unroll
            for (int u = 0; u < 2; ++u) ro[rt][u] = ar * G::ROWB + 1024 + 16 * ((4 * u + kg) ^ (ar & 7));
        }
        auto qk_a = [&](const char* cur, int ks, int rt) -> bf16x8 {
            return ks < 16 ? *(const bf16x8*)(cur + qo[rt][ks & 3] + 256 * (ks >> 2))
                           : *(const bf16x8*)(cur + ro[rt][ks - 16]);
        };
        float m_run = NEG_INF;  // reference max (base 2) of this lane's head
        float l_run = 0.f;      // this lane's share of that head's sum
        lds_barrier();  // sub-chunk 0 landed
#pragma unroll 1
        for (int s = 0; s <= nsub; ++s) {
            if (s < nsub) {
                const char* cur = cbuf + (s & (NBUF - 1)) * G::BUF;
                const int par = s & 1;
                // KS k-steps x 2 row tiles in operand groups of 4 (two k-steps
                // x both tiles), double-buffered, on four accumulator chains
                // (tile x k-step parity); the fences keep the scheduler from
                // hoisting every LDS read
                constexpr int NG = G::KS / 2;
                f32x4 sacc[2][2] = {{f32x4{}, f32x4{}}, {f32x4{}, f32x4{}}};
                bf16x8 ga[2][4];
#pragma unroll
                for (int e = 0; e < 4; ++e) ga[0][e] = qk_a(cur, e >> 1, e & 1);
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    if (g + 1 < NG) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) ga[(g + 1) & 1][e] = qk_a(cur, 2 * (g + 1) + (e >> 1), e & 1);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int k = 2 * g + (e >> 1), rt = e & 1;
                        sacc[rt][k & 1] = mfma16(ga[g & 1][e], qreg[k], sacc[rt][k & 1]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // S^T: tile rt, acc j -> k position 16rt + 4kg + j, key row
                // ksig of it, head hq
                float sv[8];
                const int rbase = row_begin + s * ROWS;
#pragma unroll
                for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) sv[4 * rt + j] = (sacc[rt][0][j] + sacc[rt][1][j]) * scale2;
                // branch-free: the index entry is read whatever the row (a
                // split's sub-chunks stay inside idx_s) and the tests combine
                // as plain values, with no short-circuit control flow
                if (__builtin_amdgcn_readfirstlane(GATHER || rbase + ROWS > row_end)) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const int r = rbase + ksig(16 * (i >> 2) + 4 * kg + (i & 3));
                        const int v = GATHER ? idx_s[r - row_begin] : 0;
                        const bool ok = (r < row_end) & (v >= 0);
                        sv[i] = ok ? sv[i] : NEG_INF;
                    }
                }
                float cm = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                                 fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
                cm = xor32_max(xor16_max(cm));
                // reference max raised only when a score passes it by TAU, so
                // O is rarely rescaled; P <= 2^TAU
                const bool raise = cm > m_run + TAU;  // false while cm is -inf
                const float m_new = raise ? cm : m_run;
                const float alpha = raise ? exp2f(m_run - m_new) : 1.f;
                m_run = m_new;
                // while every row so far is masked, m is -inf and so is every
                // score: a finite reference keeps exp2 at 0 (not -inf - -inf)
                const float m_ref = m_new == NEG_INF ? 0.f : m_new;
                float ls = 0.f;
#pragma unroll
                for (int rt = 0; rt < 2; ++rt) {
                    float pv[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) pv[e] = __builtin_amdgcn_exp2f(sv[4 * rt + e] - m_ref);
                    typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
                    const bf16x2v lo = {(__bf16)pv[0], (__bf16)pv[1]};
                    const bf16x2v hi = {(__bf16)pv[2], (__bf16)pv[3]};
                    // the sum of the P values the PV product uses (bf16), so
                    // each output is a weighted mean of its rows with no bias
                    // from the rounding of P
                    ls += ((float)lo[0] + (float)lo[1]) + ((float)hi[0] + (float)hi[1]);
                    *(u32x2*)(pbuf[par] + hq * PSTR + 2 * (16 * rt + 4 * kg)) =
                        u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
                }
                l_run = l_run * alpha + ls;
                if (kg == 0) alpha_s[par][hq] = alpha;
                const bool any = __builtin_amdgcn_ballot_w64(raise) != 0;
                if (l == 0) flag_s[par][qw] = any;
            }
            lds_barrier();  // end of phase s
        }
        l_run = xor32_sum(xor16_sum(l_run));
        if (kg == 0) {
            l_s[hq] = l_run;
            const int64_t r = part_rec(p, b, hg * HGS + hq, split);
            p.ws_ml[r * 2 + 0] = m_run;
            p.ws_ml[r * 2 + 1] = l_run;
        }
        lds_barrier();  // l_s ready
        lds_barrier();  // staging written
        } else {
        // ---------------------------------------------------------- QK role
        // B operand of 32x32x16: head 32qw + l%32, k = 16ks + 8(l/32)..+7
        const int hq = 32 * qw + (l & 31);  // this lane's head within the group
        const int kh = l >> 5;              // k half / key half
        // Q straight from global memory into registers (chunk 2ks + kh of
        // head hq), in flight with the PV waves' first row loads
        bf16x8 qreg[2 * G::KS];
        {
            const int h0 = hg * HGS + hq;
            const int hh = h0 < p.heads ? h0 : 0;  // padding heads score head 0's query
            const uint16_t* ql = p.q_lat + (int64_t)b * p.q_lat_bs + (int64_t)hh * p.q_lat_hs;
            const uint16_t* qr = DR ? p.q_rope + (int64_t)b * p.q_rope_bs + (int64_t)hh * p.q_rope_hs : nullptr;
#pragma unroll
            for (int ks = 0; ks < 2 * G::KS; ++ks) {
                const int c = 2 * ks + kh;
                qreg[ks] = c < R / 8 ? *(const bf16x8*)(ql + 8 * c) : *(const bf16x8*)(qr + 8 * (c - R / 8));
            }
        }
        // A operand: row (key) ksig(l%32) of the sub-chunk, chunk 2ks + kh;
        // with the row swizzle, chunk 16v + u2 sits at 256v + qo[u2/2 ...]:
        // latent k-steps ks -> qo[ks%8] + 256 (ks/8), rope k-steps -> ro[ks-32]
        const int arow = ksig(l & 31);
        int qo[8], ro[4];
#pragma unroll
        for (int u = 0; u < 8; ++u) qo[u] = arow * G::ROWB + 16 * ((2 * u + kh) ^ (arow & 15));
#pragma unroll
        for (int u = 0; u < 4; ++u) ro[u] = arow * G::ROWB + 1024 + 16 * ((2 * u + kh) ^ (arow & 7));
        auto qk_a = [&](const char* cur, int ks) -> bf16x8 {
            return ks < 32 ? *(const bf16x8*)(cur + qo[ks & 7] + 256 * (ks >> 3))
                           : *(const bf16x8*)(cur + ro[ks - 32]);
        };
        float m_run = NEG_INF;  // reference max (base 2) of this lane's head
        float l_run = 0.f;      // this lane's share of that head's sum
        lds_barrier();  // sub-chunk 0 landed
#pragma unroll 1
        for (int s = 0; s <= nsub; ++s) {
            if (s < nsub) {
                const char* cur = cbuf + (s & (NBUF - 1)) * G::BUF;
                const int par = s & 1;
                // 2 KS k-steps in operand groups of QG, double-buffered, on two
                // accumulator chains (even / odd k-steps) so consecutive MFMAs
                // do not wait on each other; the fences keep the scheduler from
                // hoisting every LDS read
                constexpr int NK = 2 * G::KS;
                constexpr int QG = 4;
                constexpr int NG = NK / QG;
                f32x16 sacc[2] = {f32x16{}, f32x16{}};
                bf16x8 ga[2][QG];
#pragma unroll
                for (int e = 0; e < QG; ++e) ga[0][e] = qk_a(cur, e);
#pragma unroll
                for (int g = 0; g < NG; ++g) {
                    if (g + 1 < NG) {
#pragma unroll
                        for (int e = 0; e < QG; ++e) ga[(g + 1) & 1][e] = qk_a(cur, (g + 1) * QG + e);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int e = 0; e < QG; ++e) {
                        const int k = g * QG + e;
                        sacc[k & 1] = mfma32(ga[g & 1][e], qreg[k], sacc[k & 1]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                // S^T: acc i -> key 8(i/4) + 4kh + i%4 of the sub-chunk, head hq
                float sv[16];
                const int rbase = row_begin + s * ROWS;
#pragma unroll
                for (int i = 0; i < 16; ++i) sv[i] = (sacc[0][i] + sacc[1][i]) * scale2;
                // masking only on a sub-chunk past the split end or gathered
                // (a wave-uniform branch: full dense sub-chunks skip it)
                if (__builtin_amdgcn_readfirstlane(GATHER || rbase + ROWS > row_end)) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int r = rbase + ksig(8 * (i >> 2) + 4 * kh + (i & 3));
                        const int v = GATHER ? idx_s[r - row_begin] : 0;  // inside idx_s for every sub-chunk row
                        const bool ok = (r < row_end) & (v >= 0);
                        sv[i] = ok ? sv[i] : NEG_INF;
                    }
                }
                float cm = sv[0];
#pragma unroll
                for (int i = 1; i < 16; ++i) cm = fmaxf(cm, sv[i]);
                cm = xor32_max(cm);
                // reference max raised only when a score passes it by TAU, so
                // O is rarely rescaled; P <= 2^TAU
                const bool raise = cm > m_run + TAU;  // false while cm is -inf
                const float m_new = raise ? cm : m_run;
                const float alpha = raise ? exp2f(m_run - m_new) : 1.f;
                m_run = m_new;
                // while every row so far is masked, m is -inf and so is every
                // score: a finite reference keeps exp2 at 0 (not -inf - -inf)
                const float m_ref = m_new == NEG_INF ? 0.f : m_new;
                float ls = 0.f;
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    float pv[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) pv[e] = __builtin_amdgcn_exp2f(sv[4 * i4 + e] - m_ref);
                    typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
                    const bf16x2v lo = {(__bf16)pv[0], (__bf16)pv[1]};
                    const bf16x2v hi = {(__bf16)pv[2], (__bf16)pv[3]};
                    // the sum of the P values the PV product uses (bf16), so
                    // each output is a weighted mean of its rows with no bias
                    // from the rounding of P
                    ls += ((float)lo[0] + (float)lo[1]) + ((float)hi[0] + (float)hi[1]);
                    *(u32x2*)(pbuf[par] + hq * PSTR + 2 * (8 * i4 + 4 * kh)) =
                        u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
                }
                l_run = l_run * alpha + ls;
                if (kh == 0) alpha_s[par][hq] = alpha;
                const bool any = __builtin_amdgcn_ballot_w64(raise) != 0;
                if (l == 0) flag_s[par][qw] = any;
            }
            lds_barrier();  // end of phase s
        }
        l_run = xor32_sum(l_run);
        if (kh == 0) {
            l_s[hq] = l_run;
            const int64_t r = part_rec(p, b, hg * HGS + hq, split);
            p.ws_ml[r * 2 + 0] = m_run;
            p.ws_ml[r * 2 + 1] = l_run;
        }
        lds_barrier();  // l_s ready
        lds_barrier();  // staging written
        }
    } else {
        // ---------------------------------------------------------- PV role
        int dma_row[G::NLD], dma_c16[G::NLD];
#pragma unroll
        for (int k = 0; k < G::NLD; ++k) {
            const int slot = 64 * (pw + 4 * k) + l;
            dma_row[k] = slot / G::CPR;
            dma_c16[k] = 16 * swz(slot - dma_row[k] * G::CPR, dma_row[k]);
        }
        const uint32_t rs_b = (uint32_t)(p.lat_rs * 2);
        // every PV lane always loads (rows past the split read a valid row and
        // are masked), so each PV wave issues exactly NLD loads per sub-chunk
        auto issue = [&](int s, char* base) {
            const int rbase = row_begin + s * ROWS;
#pragma unroll
            for (int k = 0; k < G::NLD; ++k) {
                int rr = dma_row[k];
                int src_row;
                if (GATHER) {
                    const int v = (rbase + rr < row_end) ? idx_s[rbase + rr - row_begin] : -1;
                    src_row = v >= 0 ? v : 0;
                } else {
                    rr = min(rr, row_end - 1 - rbase);  // rows past the split repeat its last row
                    src_row = rbase + rr;
                }
                char* dst = base + 1024 * (pw + 4 * k);
                if (PACKED) {
                    if (GATHER)
                        dma16_off(lat, (uint32_t)src_row * rs_b + (uint32_t)dma_c16[k], dst);
                    else
                        dma16_off((const char*)lat + (int64_t)rbase * rs_b, (uint32_t)rr * rs_b + (uint32_t)dma_c16[k],
                                  dst);
                } else {
                    const int c = dma_c16[k] >> 4;
                    const uint16_t* src = c < R / 8 ? lat + (int64_t)src_row * p.lat_rs + c * 8
                                                    : rop + (int64_t)src_row * p.rope_rs + (c - R / 8) * 8;
                    dma16(src, dst);
                }
            }
        };
        // prologue: sub-chunks 0 .. NBUF-2 at once (the QK waves load Q
        // themselves), issued before the rest of the set-up
        const int pro0 = min(nsub, NBUF - 1);
        for (int s = 0; s < pro0; ++s) issue(s, cbuf + s * G::BUF);
        // B operand of PV: k position p holds key row ksig(p), so lane group
        // lg takes rows 8lg + {0,2,4,6} (tr0) and 8lg + {1,3,5,7} (tr1) of
        // column block 16J by transposed reads; lane lc addresses row
        // 8lg + 2(lc/4) (+1), columns 4(lc%4)
        int tr0[8], tr1[8];
        {
            const int r0 = 8 * lg + 2 * (lc >> 2), r1 = r0 + 1;
#pragma unroll
            for (int J = 0; J < 8; ++J) {
                const int c = 16 * pw + 2 * J + ((lc & 3) >> 1);  // 16-byte chunk of the column
                tr0[J] = r0 * G::ROWB + 16 * swz(c, r0) + 8 * (lc & 1);
                tr1[J] = r1 * G::ROWB + 16 * swz(c, r1) + 8 * (lc & 1);
            }
        }
        // O^T tiles (A = V^T from the transposed reads, B = P^T): lane holds
        // head 16T + lc, columns 128pw + 16J + 4lg + 0..3
        f32x4 oacc[HT][8];
#pragma unroll
        for (int T = 0; T < HT; ++T)
#pragma unroll
            for (int J = 0; J < 8; ++J) oacc[T][J] = f32x4{0.f, 0.f, 0.f, 0.f};
        // wait for sub-chunk 0
        const int pro = min(nsub, NBUF - 1);
        if (pro >= 3)
            wait_vmcnt<2 * G::NLD>();
        else if (pro == 2)
            wait_vmcnt<G::NLD>();
        else
            wait_vmcnt<0>();
        lds_barrier();  // sub-chunk 0 landed
#pragma unroll 1
        for (int s = 0; s <= nsub; ++s) {
            // refill the buffer of s-2 (PV(s-2) ran in phase s-1) with s+2
            if (s >= 1 && s + 2 < nsub) issue(s + 2, cbuf + ((s + 2) & (NBUF - 1)) * G::BUF);
            if (s >= 1) {
                const int t = s - 1;  // PV(t): P buffer t&1, rows of buffer t%4
                const int par = t & 1;
                const char* cur = cbuf + (t & (NBUF - 1)) * G::BUF;
                bool rescale = false;
#pragma unroll
                for (int q = 0; q < QKW; ++q) rescale |= flag_s[par][q] != 0;
                if (rescale) {
#pragma unroll
                    for (int T = 0; T < HT; ++T) {
                        const float a = alpha_s[par][16 * T + lc];
#pragma unroll
                        for (int J = 0; J < 8; ++J) oacc[T][J] *= a;
                    }
                }
                bf16x8 pa[HT];
#pragma unroll
                for (int T = 0; T < HT; ++T) pa[T] = *(const bf16x8*)(pbuf[par] + (16 * T + lc) * PSTR + 16 * lg);
                bf16x4 b0[8], b1[8];
#pragma unroll
                for (int J = 0; J < 8; ++J) {
                    b0[J] = ds_read_tr16(cur + tr0[J]);
                    b1[J] = ds_read_tr16(cur + tr1[J]);
                }
                __builtin_amdgcn_sched_barrier(0);  // all 16 reads in flight before the MFMAs
#pragma unroll
                for (int J = 0; J < 8; ++J) {
                    const bf16x8 bb = __builtin_shufflevector(b0[J], b1[J], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                    for (int T = 0; T < HT; ++T) oacc[T][J] = mfma16(bb, pa[T], oacc[T][J]);
                }
            }
            // sub-chunk s+1 must have landed before the barrier; only s+2 may
            // still be in flight
            if (s + 1 < nsub) {
                if (s + 2 < nsub)
                    wait_vmcnt<G::NLD>();
                else
                    wait_vmcnt<0>();
            }
            lds_barrier();  // end of phase s
        }
        lds_barrier();  // l_s ready
        // O / l into the staging area [HGS heads][srow bytes], partial
        // precision: per (T, J) a lane writes its head's four consecutive
        // columns (8 bytes bf16, 16 bytes f32)
        float inv[HT];
#pragma unroll
        for (int T = 0; T < HT; ++T) {
            const float lv = l_s[16 * T + lc];
            inv[T] = lv > 0.f ? 1.f / lv : 0.f;
        }
        if (p.ws_f32) {
#pragma unroll
            for (int T = 0; T < HT; ++T) {
                float* row = (float*)(cbuf + (16 * T + lc) * srow) + 128 * pw + 4 * lg;
#pragma unroll
                for (int J = 0; J < 8; ++J) *(f32x4*)(row + 16 * J) = oacc[T][J] * inv[T];
            }
        } else {
            typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
#pragma unroll
            for (int T = 0; T < HT; ++T) {
                __bf16* row = (__bf16*)(cbuf + (16 * T + lc) * srow) + 128 * pw + 4 * lg;
#pragma unroll
                for (int J = 0; J < 8; ++J) {
                    const f32x4 o = oacc[T][J] * inv[T];
                    const bf16x2v lo = {(__bf16)o[0], (__bf16)o[1]};
                    const bf16x2v hi = {(__bf16)o[2], (__bf16)o[3]};
                    *(u32x2*)(row + 16 * J) = u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
                }
            }
        }
        lds_barrier();  // staging written
    }
    // the partial records: one row of 512 values per head, 16-byte stores
    const int cpr = R * esz / 16;  // 16-byte chunks per row
    for (int e = tid; e < HGS * cpr; e += NT) {
        const int r = e / cpr, c = e - r * cpr;
        // streamed past L2: the combine on other XCDs reads them from memory
        __builtin_nontemporal_store(*(const u32x4*)(cbuf + r * srow + 16 * c),
                                    (u32x4*)((char*)p.ws_o + part_rec(p, b, hg * HGS + r, split) * R * esz + 16 * c));
    }
}

// Merge the split partials.  A partial is O_s / l_s (bf16 for bf16 output,
// f32 for f32 output) with its running max m_s and sum l_s (fp32):
//   out = sum_s w_s (O_s / l_s) / (sum_s w_s + sink),  w_s = l_s 2^(m_s - M).
// One 256-thread block per (batch, head, 256-byte column block of the
// record): 128 columns of bf16 partials or 64 of f32, so a (batch, head)
// spreads over 4 or 8 blocks and the grid covers every CU.  Lane l of wave w
// takes the 16 bytes l%16 of splits 16k + 4w + l/16: one load instruction of
// a wave reads four whole 256-byte pieces, and the first COMBINE_PF loads of
// every lane are in flight before the weights are computed.
constexpr int COMBINE_THREADS = 256;

// PF record loads per lane in flight (16 PF splits) and MLK (m, l) loads per
// thread (256 MLK splits), both at least the launch's split count needs, so
// the unconditional loads below are not mostly duplicates of the last split.
template <bool F32, int PF, int MLK>
__global__ void __launch_bounds__(COMBINE_THREADS) mla_combine(CombineParams p) {
    constexpr int VPL = F32 ? 4 : 8;  // values per lane (16 bytes)
    constexpr int CB = 16 * VPL;      // columns per block
    constexpr int NCB = R / CB;
    constexpr int COMBINE_PF = PF;
    static_assert(MLK * COMBINE_THREADS <= MAX_COMBINE_SPLITS, "split weights");
    __shared__ float wgt[MAX_COMBINE_SPLITS];
    __shared__ float red_m[4], red_l[4];
    __shared__ __attribute__((aligned(16))) float part[4][16][VPL];
    const int bh = blockIdx.x / NCB;
    const int cb = blockIdx.x - bh * NCB;
    const int b = bh / p.heads;
    const int h = bh - b * p.heads;
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int l = tid & 63;
    const int sg = l >> 4;  // split within the wave's four
    const int ch = l & 15;  // 16-byte chunk of the column block
    const int64_t rec0 = ((int64_t)b * p.h_pad + h) * p.splits;  // the splits of (b, h) are contiguous
    constexpr int RB = R * (F32 ? 4 : 2);  // bytes per record
    const char* base = (const char*)p.ws_o + rec0 * RB + 256 * cb + 16 * ch;

    // (m, l) of every split first: the weights wait only on these.  Every
    // load is issued unconditionally (indices clamped to the last split, the
    // extra values weighted out), so the compiler's waits count exactly and
    // the max and the sum run while the records are still in flight.
    float ml_m[MLK], ml_l[MLK];
#pragma unroll
    for (int k = 0; k < MLK; ++k) {
        const int s = tid + COMBINE_THREADS * k;
        const f32x2 ml = *(const f32x2*)(p.ws_ml + (rec0 + min(s, p.splits - 1)) * 2);
        ml_m[k] = s < p.splits ? ml[0] : NEG_INF;
        ml_l[k] = s < p.splits ? ml[1] : 0.f;
    }
    u32x4 x[COMBINE_PF];
#pragma unroll
    for (int k = 0; k < COMBINE_PF; ++k) {
        const int s = 16 * k + 4 * w + sg;
        x[k] = *(const u32x4*)(base + (int64_t)min(s, p.splits - 1) * RB);
    }
    float M = NEG_INF;
#pragma unroll
    for (int k = 0; k < MLK; ++k)
        if (ml_l[k] > 0.f) M = fmaxf(M, ml_m[k]);
    M = wave_max(M);
    if (l == 0) red_m[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    const bool any = M != NEG_INF;
    const float sink2 = p.sinks ? p.sinks[h] * LOG2E : NEG_INF;
    M = fmaxf(M, sink2);
    float L = 0.f;
#pragma unroll
    for (int k = 0; k < MLK; ++k) {
        const int s = tid + COMBINE_THREADS * k;
        if (s < p.splits) {
            const float wv = ml_l[k] > 0.f ? ml_l[k] * exp2f(ml_m[k] - M) : 0.f;
            wgt[s] = wv;
            L += wv;
        }
    }
    L = wave_sum(L);
    if (l == 0) red_l[w] = L;
    __syncthreads();
    L = (red_l[0] + red_l[1]) + (red_l[2] + red_l[3]);
    if (p.sinks) L += exp2f(sink2 - M);

    float acc[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) acc[v] = 0.f;
    // a split with no valid row has weight 0: select, never multiply it in
    auto add = [&](const u32x4& u, float wv) {
        if (wv == 0.f) return;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
            const float xv = F32 ? __uint_as_float(u[v]) : __uint_as_float(v & 1 ? u[v >> 1] & 0xffff0000u : u[v >> 1] << 16);
            acc[v] += wv * xv;
        }
    };
#pragma unroll
    for (int k = 0; k < COMBINE_PF; ++k) {
        const int s = 16 * k + 4 * w + sg;
        if (s < p.splits) add(x[k], wgt[s]);
    }
    for (int s = 16 * COMBINE_PF + 4 * w + sg; s < p.splits; s += 16) add(*(const u32x4*)(base + (int64_t)s * RB), wgt[s]);
    // the four splits of a wave, then the four waves
#pragma unroll
    for (int v = 0; v < VPL; ++v) {
        acc[v] = xor32_sum(xor16_sum(acc[v]));
    }
    if (sg == 0) {
#pragma unroll
        for (int v = 0; v < VPL; ++v) part[w][ch][v] = acc[v];
    }
    __syncthreads();
    if (tid >= 16) return;
    const float sc = any ? 1.f / L : 0.f;
    float o[VPL];
#pragma unroll
    for (int v = 0; v < VPL; ++v) o[v] = ((part[0][ch][v] + part[1][ch][v]) + (part[2][ch][v] + part[3][ch][v])) * sc;
    const int64_t oo = (int64_t)b * p.out_bs + (int64_t)h * p.out_hs + CB * cb + VPL * ch;
    if (p.out_f32) {
#pragma unroll
        for (int v = 0; v < VPL; v += 4) *(f32x4*)((float*)p.out + oo + v) = f32x4{o[v], o[v + 1], o[v + 2], o[v + 3]};
    } else if (F32) {  // fp32 partials, bf16 output: 8 bytes per lane
        *(u32x2*)((uint16_t*)p.out + oo) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
    } else {
        *(u32x4*)((uint16_t*)p.out + oo) = u32x4{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]),
                                                 pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7])};
    }
}

// The split merge of one head fused with its value un-absorption (the decode
// block's W_UV stage).  512 threads per head: waves 0-3 merge the splits as
// mla_combine does (lane l of wave w takes 16-byte chunk l of the records of
// splits w, w+4, ..., all in flight at once) while waves 4-7 copy the head's
// W_UV rows into LDS by DMA (a dense bf16 row is one 1 KB load; the 4-bit
// rows, scales and biases are contiguous KB blocks) once the records have
// been requested (a CU keeps a bounded number of requests in flight, and the
// records are needed first).  The context, rounded to bf16 as mla_combine's
// output is, goes to LDS, and all eight waves then form the head's v_dim
// outputs from LDS, 8 lanes per row.  (Spreading a head over its column
// blocks, with a second launch adding the blocks' partial sums, measured
// slower: that launch alone took 4.3 us.)
constexpr int CU_PF = 32;  // split records in flight per lane (bf16 records)

template <bool F32, bool AFF>
__global__ void __launch_bounds__(512) mla_combine_unabsorb(CombineUnabsorbParams p) {
    extern __shared__ __attribute__((aligned(1024))) char wlds[];  // the head's W_UV rows
    __shared__ float wgt[MAX_COMBINE_SPLITS];
    __shared__ float red_m[4], red_l[4];
    __shared__ __attribute__((aligned(16))) float ctx_part[4][R];
    __shared__ __attribute__((aligned(16))) float ctx_s[R];
    __shared__ float gsum[8];
    const int h = blockIdx.x;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int V = p.v_dim;
    const int64_t row_base = (int64_t)h * p.row_step + p.row0;
    const int64_t rec0 = (int64_t)h * p.splits;  // batch 1: the splits of head h are contiguous
    constexpr int RB = R * (F32 ? 4 : 2);        // bytes per record
    constexpr int PF = F32 ? CU_PF / 2 : CU_PF;  // splits per batch (F32: two loads per split)

    if (w >= 4) {
        // ------------------------------------------------ DMA waves
        lds_barrier();  // 1: max
        lds_barrier();  // 2: sum
        const int dw = w - 4;
        if (AFF) {
            // V rows of 256 packed bytes, then V x 16 bytes of scales and of
            // biases (8 groups of 64 inputs per row), all contiguous
            const char* pk = (const char*)(p.packed + row_base * (R / 8));
            const char* sc = (const char*)(p.scales + row_base * (R / 64));
            const char* bi = (const char*)(p.biases + row_base * (R / 64));
            const int npk = V / 4, nsb = V / 64;  // KB blocks
            for (int k = dw; k < npk + 2 * nsb; k += 4) {
                const char* src = k < npk ? pk + 1024 * k : (k < npk + nsb ? sc + 1024 * (k - npk) : bi + 1024 * (k - npk - nsb));
                dma16(src + 16 * l, wlds + 1024 * k);
            }
        } else {
            for (int j = dw; j < V; j += 4) dma16(p.w + (row_base + j) * p.w_rs + 8 * l, wlds + 1024 * j);
        }
        lds_barrier();  // 3: per-wave context
        wait_vmcnt<0>();
        lds_barrier();  // 4: context and weights in LDS
    } else {
        // ------------------------------------------------ merge waves
        constexpr int MLK = MAX_COMBINE_SPLITS / 256;
        float ml_m[MLK], ml_l[MLK];
        float M = NEG_INF;
        // every load is issued unconditionally (indices clamped to the last
        // split, the extra values weighted out), so the compiler's waits
        // count exactly and the (m, l) loads do not wait for the records
#pragma unroll
        for (int k = 0; k < MLK; ++k) {
            const int s = tid + 256 * k;
            const f32x2 ml = *(const f32x2*)(p.ws_ml + (rec0 + min(s, p.splits - 1)) * 2);
            ml_m[k] = s < p.splits ? ml[0] : NEG_INF;
            ml_l[k] = s < p.splits ? ml[1] : 0.f;
        }
        const char* base = (const char*)p.ws_o + rec0 * RB + 16 * l;
        u32x4 x[PF][F32 ? 2 : 1];
        auto fetch = [&](int s0) {
#pragma unroll
            for (int k = 0; k < PF; ++k) {
                const int s = min(s0 + 4 * k, p.splits - 1);
#pragma unroll
                for (int c = 0; c < (F32 ? 2 : 1); ++c) x[k][c] = *(const u32x4*)(base + (int64_t)s * RB + 1024 * c);
            }
        };
        fetch(w);
#pragma unroll
        for (int k = 0; k < MLK; ++k)
            if (ml_l[k] > 0.f) M = fmaxf(M, ml_m[k]);
        M = wave_max(M);
        if (l == 0) red_m[w] = M;
        lds_barrier();  // 1
        M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
        float L = 0.f;
#pragma unroll
        for (int k = 0; k < MLK; ++k) {
            const int s = tid + 256 * k;
            if (s < p.splits) {
                const float wv = ml_l[k] > 0.f ? ml_l[k] * exp2f(ml_m[k] - M) : 0.f;
                wgt[s] = wv;
                L += wv;
            }
        }
        L = wave_sum(L);
        if (l == 0) red_l[w] = L;
        lds_barrier();  // 2
        L = (red_l[0] + red_l[1]) + (red_l[2] + red_l[3]);
        constexpr int VPL = 8;  // values per lane: 8 bf16, or 2 x 4 f32
        float acc[VPL];
#pragma unroll
        for (int v = 0; v < VPL; ++v) acc[v] = 0.f;
        for (int s0 = w;; s0 += 4 * PF) {
#pragma unroll
            for (int k = 0; k < PF; ++k) {
                const int s = s0 + 4 * k;
                const float wv = s < p.splits ? wgt[s] : 0.f;
                if (wv == 0.f) continue;  // an empty split is selected out, never multiplied in
#pragma unroll
                for (int v = 0; v < VPL; ++v) {
                    float xv;
                    if (F32)
                        xv = __uint_as_float(x[k][v >> 2][v & 3]);
                    else
                        xv = __uint_as_float(v & 1 ? x[k][0][v >> 1] & 0xffff0000u : x[k][0][v >> 1] << 16);
                    acc[v] += wv * xv;
                }
            }
            if (s0 + 4 * PF >= p.splits) break;
            fetch(s0 + 4 * PF);
        }
        // columns of the lane: bf16 8l .. 8l+7; f32 4l .. 4l+3 and 256+4l .. +3
        if (F32) {
            *(f32x4*)(&ctx_part[w][4 * l]) = f32x4{acc[0], acc[1], acc[2], acc[3]};
            *(f32x4*)(&ctx_part[w][256 + 4 * l]) = f32x4{acc[4], acc[5], acc[6], acc[7]};
        } else {
            *(f32x4*)(&ctx_part[w][8 * l]) = f32x4{acc[0], acc[1], acc[2], acc[3]};
            *(f32x4*)(&ctx_part[w][8 * l + 4]) = f32x4{acc[4], acc[5], acc[6], acc[7]};
        }
        lds_barrier();  // 3
        // the context, bf16-rounded as mla_combine writes it: thread t holds
        // columns 2t, 2t+1; the 4-bit path also needs each group's sum
        const float sc = M != NEG_INF ? 1.f / L : 0.f;
        float cv[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int c = 2 * tid + e;
            const float o = ((ctx_part[0][c] + ctx_part[1][c]) + (ctx_part[2][c] + ctx_part[3][c])) * sc;
            cv[e] = bf16_bits_to_f32(f32_to_bf16_bits(o));
            ctx_s[c] = cv[e];
        }
        if (AFF) {
            const float gs = group_sum(cv[0] + cv[1], 32);  // 32 threads = one group of 64 columns
            if ((tid & 31) == 0) gsum[tid >> 5] = gs;
        }
        lds_barrier();  // 4
    }

    // ---------------------------------------------------- W_UV rows, 8 lanes per row
    const int i = l & 7;
    for (int r = 8 * w + (l >> 3); r < V; r += 64) {
        float y = 0.f;
        if (AFF) {
            // lane i takes group i of row r: 8 packed words, its scale and bias
            const u32x4 q0 = *(const u32x4*)(wlds + r * 256 + 32 * i);
            const u32x4 q1 = *(const u32x4*)(wlds + r * 256 + 32 * i + 16);
            const uint16_t* sc = (const uint16_t*)(wlds + V * 256);
            const uint16_t* bi = (const uint16_t*)(wlds + V * 256 + V * 16);
            const float s = bf16_bits_to_f32(sc[8 * r + i]), b = bf16_bits_to_f32(bi[8 * r + i]);
            const uint32_t wd[8] = {q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
            float dot = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const f32x4 c0 = *(const f32x4*)(&ctx_s[64 * i + 8 * k]);
                const f32x4 c1 = *(const f32x4*)(&ctx_s[64 * i + 8 * k + 4]);
#pragma unroll
                for (int n = 0; n < 8; ++n) dot += (float)((wd[k] >> (4 * n)) & 15u) * (n < 4 ? c0[n] : c1[n - 4]);
            }
            y = s * dot + b * gsum[i];
        } else {
            // lane i takes 16-byte chunks 8c + i of row r
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int k = 8 * c + i;
                const u32x4 wv = *(const u32x4*)(wlds + r * 1024 + 16 * k);
                const f32x4 c0 = *(const f32x4*)(&ctx_s[8 * k]);
                const f32x4 c1 = *(const f32x4*)(&ctx_s[8 * k + 4]);
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    y += __uint_as_float(wv[n] << 16) * (n < 2 ? c0[2 * n] : c1[2 * n - 4]);
                    y += __uint_as_float(wv[n] & 0xffff0000u) * (n < 2 ? c0[2 * n + 1] : c1[2 * n - 3]);
                }
            }
        }
        y = group_sum(y, 8);
        if (i == 0) p.out[(int64_t)h * V + r] = f32_to_bf16_bits(y);
    }
}

template <int DR, bool GATHER, bool PACKED>
hipError_t launch_ws(const DecodeParams& p, int grid, hipStream_t st) {
    if (p.hg_size == 64)
        hipLaunchKernelGGL((mla_decode_ws<DR, GATHER, PACKED, 64, true>), dim3(grid), dim3(WsShape<64, true>::THREADS), 0,
                           st, p);
    else if (p.hg_size == 48)
        hipLaunchKernelGGL((mla_decode_ws<DR, GATHER, PACKED, 48, true>), dim3(grid), dim3(WsShape<48, true>::THREADS), 0,
                           st, p);
    else
        hipLaunchKernelGGL((mla_decode_ws<DR, GATHER, PACKED, 32, false>), dim3(grid), dim3(WsShape<32, false>::THREADS),
                           0, st, p);
    return hipGetLastError();
}

template <int DR, bool GATHER>
hipError_t launch_split(const DecodeParams& p, int grid, hipStream_t st) {
    const bool packed = DR == 0 || (p.rope == p.latent + R && p.rope_rs == p.lat_rs && p.rope_bs == p.lat_bs);
    return packed ? launch_ws<DR, GATHER, true>(p, grid, st) : launch_ws<DR, GATHER, false>(p, grid, st);
}

// The same check as a launch of its own: one workgroup per token, the table
// in LDS (dynamic) or, for long lists, at `tables` (2 * slots int32 a token).
__global__ void __launch_bounds__(1024) validate_indices_kernel(const int32_t* indices, int32_t n_idx, int32_t n_rows,
                                                                int32_t* tables, int32_t* result) {
    extern __shared__ int32_t table[];
    const int32_t* ind = indices + (int64_t)blockIdx.x * n_idx;
    if (tables)
        validate_token<true>(ind, n_idx, n_rows, tables + (int64_t)blockIdx.x * 2 * validate_slots(n_idx), 1024,
                             threadIdx.x, result + 3 * blockIdx.x);
    else
        validate_token<false>(ind, n_idx, n_rows, table, 1024, threadIdx.x, result + 3 * blockIdx.x);
}

}  // namespace

size_t validate_table_bytes(int32_t batch, int32_t n_idx) {
    if (n_idx <= VALIDATE_LDS_MAX_IDX) return 0;
    return size_t(batch) * 2 * sizeof(int32_t) * size_t(validate_slots(n_idx));
}

hipError_t launch_validate_indices(const int32_t* indices, int32_t batch, int32_t n_idx, int32_t n_rows,
                                   int32_t* tables, int32_t* result, hipStream_t st) {
    size_t lds = 0;
    if (n_idx <= VALIDATE_LDS_MAX_IDX) {
        tables = nullptr;
        lds = sizeof(int32_t) * 2 * size_t(validate_slots(n_idx));
        if (lds > 65536) {
            const hipError_t e = hipFuncSetAttribute((const void*)validate_indices_kernel,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
    }
    hipLaunchKernelGGL(validate_indices_kernel, dim3(batch), dim3(1024), lds, st, indices, n_idx, n_rows, tables, result);
    return hipGetLastError();
}

int validate_max_indices() { return VALIDATE_MAX_IDX; }

// 32 heads for small layers, else 64, or 48 where that splits the heads
// exactly and 64 would not (96 heads: two groups of 48 instead of two of 64
// with a quarter of the MFMA work and partial records spent on padding)
int decode_head_group_size(int heads) {
    if (heads <= 32) return 32;
    if (heads % 64 != 0 && heads % 48 == 0) return 48;
    return 64;
}

hipError_t launch_combine_unabsorb(const CombineUnabsorbParams& p, hipStream_t st) {
    const size_t lds = p.affine ? size_t(p.v_dim) * (256 + 2 * 16) : size_t(p.v_dim) * 1024;
    auto go = [&](const void* kern, auto launch) {
        if (lds > 65536) {
            const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        launch();
        return hipGetLastError();
    };
    const dim3 grid((unsigned)p.heads), block(512);
    if (p.affine) {
        if (p.ws_f32)
            return go((const void*)mla_combine_unabsorb<true, true>,
                      [&] { hipLaunchKernelGGL((mla_combine_unabsorb<true, true>), grid, block, lds, st, p); });
        return go((const void*)mla_combine_unabsorb<false, true>,
                  [&] { hipLaunchKernelGGL((mla_combine_unabsorb<false, true>), grid, block, lds, st, p); });
    }
    if (p.ws_f32)
        return go((const void*)mla_combine_unabsorb<true, false>,
                  [&] { hipLaunchKernelGGL((mla_combine_unabsorb<true, false>), grid, block, lds, st, p); });
    return go((const void*)mla_combine_unabsorb<false, false>,
              [&] { hipLaunchKernelGGL((mla_combine_unabsorb<false, false>), grid, block, lds, st, p); });
}

// floor(2^32 / d) + 1: x / d == __umulhi(x, magic) for every x <= x_max
// when x_max * d < 2^32; 0 (divide) otherwise
static uint32_t div_magic(uint32_t d, uint32_t x_max) {
    if (d <= 1 || (uint64_t)x_max * d >= (1ull << 32)) return 0;
    return (uint32_t)((1ull << 32) / d + 1);
}

hipError_t launch_mla_decode(const DecodeParams& p_in, const CombineParams& cp, bool split_only,
                             hipEvent_t const* events, hipStream_t st) {
    DecodeParams p = p_in;
    const int units = p.batch * p.splits;
    const int grid = p.check_blocks + 8 * p.head_groups * ((units + 7) / 8);
    p.hg_magic = div_magic((uint32_t)p.head_groups, (uint32_t)grid >> 3);
    p.split_magic = div_magic((uint32_t)p.splits, (uint32_t)units + 8);
    hipError_t e;
    if (events && (e = hipEventRecord(events[0], st)) != hipSuccess) return e;
    const bool g = p.indices != nullptr;
    if (p.rope_dim == 64)
        e = g ? launch_split<64, true>(p, grid, st) : launch_split<64, false>(p, grid, st);
    else
        e = g ? launch_split<0, true>(p, grid, st) : launch_split<0, false>(p, grid, st);
    if (e != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[1], st)) != hipSuccess) return e;
    if (split_only) return events ? hipEventRecord(events[2], st) : hipSuccess;
    // loads in flight for the split count: 16 PF splits of records (at most
    // 128; more are read by the tail loop) and 256 MLK of (m, l) pairs
    const int pf = cp.splits <= 16 ? 1 : cp.splits <= 32 ? 2 : cp.splits <= 64 ? 4 : 8;
    const bool mlk4 = cp.splits > COMBINE_THREADS;
    auto combine = [&](auto f32_tag, auto pf_tag, auto mlk_tag) {
        constexpr bool F = decltype(f32_tag)::value;
        hipLaunchKernelGGL((mla_combine<F, decltype(pf_tag)::value, decltype(mlk_tag)::value>),
                           dim3(p.batch * p.heads * (R / (F ? 64 : 128))), dim3(COMBINE_THREADS), 0, st, cp);
    };
    auto by_pf = [&](auto f32_tag, auto mlk_tag) {
        if (pf == 1)
            combine(f32_tag, std::integral_constant<int, 1>{}, mlk_tag);
        else if (pf == 2)
            combine(f32_tag, std::integral_constant<int, 2>{}, mlk_tag);
        else if (pf == 4)
            combine(f32_tag, std::integral_constant<int, 4>{}, mlk_tag);
        else
            combine(f32_tag, std::integral_constant<int, 8>{}, mlk_tag);
    };
    auto by_mlk = [&](auto f32_tag) {
        if (mlk4)
            by_pf(f32_tag, std::integral_constant<int, MAX_COMBINE_SPLITS / COMBINE_THREADS>{});
        else
            by_pf(f32_tag, std::integral_constant<int, 1>{});
    };
    if (cp.ws_f32)
        by_mlk(std::true_type{});
    else
        by_mlk(std::false_type{});
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (events && (e = hipEventRecord(events[2], st)) != hipSuccess) return e;
    return hipSuccess;
}

}  // namespace mr
