// Shared device-side helpers for the gfx950 kernels of the MLA path.
//
// Operand layouts used throughout (pinned on hardware by selftest.hip and
// tests/test_gpu_selftest.py):
//
//   v_mfma_f32_16x16x32_bf16   A[16][32]: lane l holds row l%16, k = 8*(l/16)+0..7
//                              B[32][16]: lane l holds col l%16, k = 8*(l/16)+0..7
//                              D[16][16]: lane l holds col l%16, rows 4*(l/16)+0..3
//   v_mfma_f32_32x32x16_bf16   A[32][16]: lane l holds row l%32, k = 8*(l/32)+0..7
//                              B[16][32]: lane l holds col l%32, k = 8*(l/32)+0..7
//                              D[32][32]: lane l holds col l%32,
//                                         acc i -> row 8*(i/4) + 4*(l/32) + i%4
//   ds_read_b64_tr_b16         within each 16-lane group, lane j supplies the
//                              address of 4 consecutive b16 of "row" j/4,
//                              "cols" 4*(j%4)..+3 of a 4x16 block; lane i gets
//                              column i of that block (rows 0..3).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mr {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define MR_LDS __attribute__((address_space(3)))

__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// LDS transpose read: 4 x b16 (see the layout note above).
// `p` must point into __shared__ memory (8-byte aligned).
__device__ __forceinline__ bf16x4 ds_read_tr16(const void* p) {
    typedef MR_LDS bf16x4 lds_bf16x4;
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
    return __uint_as_float(((uint32_t)h) << 16);
}

// Round-to-nearest-even float -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

// The same pair through gfx950's v_cvt_pk_bf16_f32 (round to nearest even,
// one instruction for both values); NaNs stay NaNs, their payload bits may
// differ from f32_to_bf16_bits'.
__device__ __forceinline__ uint32_t pack_bf16x2_hw(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// sigmoid(g) = 1 / (1 + 2^(-g log2 e)) on the hardware exp2 and reciprocal
// (each within 1 ulp); 0 and 1 at the extremes.
__device__ __forceinline__ float sigmoid_f32(float g) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// The output gate of MLA.swift:207-211 on two bf16 elements packed in a
// word: bf16(x * sigmoid(g)) per half.
__device__ __forceinline__ uint32_t gated_bf16x2(uint32_t x, uint32_t g) {
    const float lo = __uint_as_float(x << 16) * sigmoid_f32(__uint_as_float(g << 16));
    const float hi = __uint_as_float(x & 0xffff0000u) * sigmoid_f32(__uint_as_float(g & 0xffff0000u));
    return pack_bf16x2_hw(lo, hi);
}

// One correctly rounded fp32 operation each, never fused into an FMA with a
// neighbour (hipcc contracts a*b+c by default; these carry no contract flag).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

template <int N>
__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) {
    return __builtin_bit_cast(bf16x8, v);
}

// v combined with the value of lane l ^ 32 by one VALU op: after
// v_permlane32_swap of two copies of v, the pair (r[0], r[1]) of lane l holds
// {v[l], v[l ^ 32]} (lower-half lane first in both halves), so max and sum
// are the same bits in lanes l and l ^ 32.
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The same with lane l ^ 16 (v_permlane16_swap: rows of 16 lanes).
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum of v over aligned groups of n lanes (n a power of two <= 64, uniform):
// every lane of a group ends with the group's sum.  Butterflies run from
// lane distance 1 upward on DPP and permlane swaps, with no LDS round trip:
// quad_perm(1,0,3,2) (0xB1) and quad_perm(2,3,0,1) (0x4E) are xor 1 and
// xor 2; once the steps below distance d are done, all lanes of a d-group
// hold the same value, so row_half_mirror (0x141) and row_mirror (0x140),
// which map every lane into the neighbouring 4- / 8-lane group, act as xor 4
// and xor 8.
__device__ __forceinline__ float group_sum(float v, int n) {
    if (n > 1) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));
    if (n > 2) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));
    if (n > 4) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));
    if (n > 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));
    if (n > 16) v = xor16_sum(v);
    if (n > 32) v = xor32_sum(v);
    return v;
}

// LDS-only barrier: waits for this wave's LDS traffic, not for its global
// (DMA) loads, so prefetches stay in flight across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Global -> LDS traffic (DMA) is issued with this instruction from inline
// asm, so the compiler neither knows of it nor inserts its conservative
// vmcnt(0) before LDS reads; a kernel waits for it explicitly with
// wait_vmcnt and issues no other vector-memory load after its first DMA,
// which keeps those counts exact.  (Extra loads the compiler does not see
// can only make its own waits stricter.)
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

// Raw (stride 0) buffer resource over `bytes` bytes from `base`: a load at a
// byte offset at or past `bytes` returns zeros.  Word 3 holds the gfx9 data
// format the memory-to-register loads expect (32-bit, no swizzle).
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return i32x4{(int32_t)(uint32_t)a, (int32_t)((a >> 32) & 0xffff), (int32_t)bytes, 0x00020000};
}

// DMA of 16 bytes per lane from a buffer resource at a per-lane byte offset
// (buffer_load_dwordx4 ... lds): lane i lands at lds_dst_wave_base + 16 i;
// a lane whose offset is out of range writes zeros.  Same wait rules as dma16.
__device__ __forceinline__ void dma16_buf(i32x4 rsrc, uint32_t voff, const void* lds_dst_wave_base) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_dst_wave_base;
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(m0) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// A kernel's parameter block read in one batch: each dword passes through
// an empty asm that the compiler must treat as changing it, so every load
// is issued (and waited for once) before any field is used.  Loaded where
// each field is first used, the block costs several dependent scalar-memory
// round trips, which latency-bound kernels pay on their critical path.
template <typename P>
__device__ __forceinline__ P load_params(const P& arg) {
    static_assert(sizeof(P) % 4 == 0, "parameter block of whole dwords");
    constexpr int NW = sizeof(P) / 4;
    uint32_t w[NW];
    const uint32_t* src = reinterpret_cast<const uint32_t*>(&arg);
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = src[i];
#pragma unroll
    for (int i = 0; i < NW; ++i) asm volatile("" : "+s"(w[i]));
    P q;
    __builtin_memcpy(&q, w, sizeof(P));
    return q;
}

// Full-wave max and sum: the group_sum butterfly over all 64 lanes (DPP and
// permlane swaps, no LDS round trips); every lane ends with the result.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false)));
    return xor32_max(xor16_max(v));
}

__device__ __forceinline__ float wave_sum(float v) { return group_sum(v, 64); }

// v plus the value of lane l ^ 8 (DPP row_ror:8 rotates each 16-lane row by
// 8, which is xor 8 there).
__device__ __forceinline__ float xor8_sum(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false));
}

}  // namespace mr
