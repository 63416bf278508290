// Hardware self-tests of the gfx950 operand layouts the MLA kernels rely on
// (16x16x32 / 32x32x16 bf16 MFMA, ds_read_b64_tr_b16).  Built into a separate
// library used only by tests; every access is within the fixed-size buffers
// described per entry point.
#include "mr_device.hpp"

using namespace mr;

// A [16][32] bf16, B [32][16] bf16 (row-major), D [16][16] f32.  One wave.
__global__ void __launch_bounds__(64) k_mfma16(const uint16_t* A, const uint16_t* B, float* D) {
    int l = threadIdx.x;
    u32x4 a, b;
    uint16_t av[8], bv[8];
    for (int j = 0; j < 8; ++j) {
        av[j] = A[(l % 16) * 32 + 8 * (l / 16) + j];
        bv[j] = B[(8 * (l / 16) + j) * 16 + (l % 16)];
    }
    for (int j = 0; j < 4; ++j) {
        a[j] = av[2 * j] | ((uint32_t)av[2 * j + 1] << 16);
        b[j] = bv[2 * j] | ((uint32_t)bv[2 * j + 1] << 16);
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mfma16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc);
    for (int i = 0; i < 4; ++i) D[(4 * (l / 16) + i) * 16 + (l % 16)] = acc[i];
}

// A [32][16], B [16][32], D [32][32].  One wave.
__global__ void __launch_bounds__(64) k_mfma32(const uint16_t* A, const uint16_t* B, float* D) {
    int l = threadIdx.x;
    u32x4 a, b;
    uint16_t av[8], bv[8];
    for (int j = 0; j < 8; ++j) {
        av[j] = A[(l % 32) * 16 + 8 * (l / 32) + j];
        bv[j] = B[(8 * (l / 32) + j) * 32 + (l % 32)];
    }
    for (int j = 0; j < 4; ++j) {
        a[j] = av[2 * j] | ((uint32_t)av[2 * j + 1] << 16);
        b[j] = bv[2 * j] | ((uint32_t)bv[2 * j + 1] << 16);
    }
    f32x16 acc = {};
    acc = mfma32(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc);
    for (int i = 0; i < 16; ++i) D[(8 * (i / 4) + 4 * (l / 32) + (i % 4)) * 32 + (l % 32)] = acc[i];
}

// LDS holds 2048 b16 values v[i] = i.  offsets [64] are byte offsets
// (multiples of 8, < 4096 - 8, checked on the host); out [64][4] b16.
__global__ void __launch_bounds__(64) k_tr16(const int32_t* offsets, uint16_t* out) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2048];
    int l = threadIdx.x;
    for (int i = l; i < 2048; i += 64) lds[i] = (uint16_t)i;
    __syncthreads();
    bf16x4 r = ds_read_tr16((const char*)lds + offsets[l]);
    u32x2 u = __builtin_bit_cast(u32x2, r);
    out[4 * l + 0] = (uint16_t)(u[0] & 0xffff);
    out[4 * l + 1] = (uint16_t)(u[0] >> 16);
    out[4 * l + 2] = (uint16_t)(u[1] & 0xffff);
    out[4 * l + 3] = (uint16_t)(u[1] >> 16);
}

// v_permlane32_swap of two copies of in[l]: out[2l] = r[0], out[2l+1] = r[1].
__global__ void __launch_bounds__(64) k_permlane32(const uint32_t* in, uint32_t* out) {
    const int l = threadIdx.x;
    const uint32_t v = in[l];
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    out[2 * l] = r[0];
    out[2 * l + 1] = r[1];
}

// v_permlane16_swap of two copies of in[l]: out[2l] = r[0], out[2l+1] = r[1].
__global__ void __launch_bounds__(64) k_permlane16(const uint32_t* in, uint32_t* out) {
    const int l = threadIdx.x;
    const uint32_t v = in[l];
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    out[2 * l] = r[0];
    out[2 * l + 1] = r[1];
}


// v_permlane16_swap of two different values a = in[l], b = in[64 + l]:
// out[2l] = r[0], out[2l+1] = r[1] (the decode reduces two head tiles'
// values at once this way).
__global__ void __launch_bounds__(64) k_permlane16_pair(const uint32_t* in, uint32_t* out) {
    const int l = threadIdx.x;
    const auto r = __builtin_amdgcn_permlane16_swap(in[l], in[64 + l], false, false);
    out[2 * l] = r[0];
    out[2 * l + 1] = r[1];
}

// MFMA rate probe: every wave runs `iters` rounds of 8 independent 32x32x16
// bf16 MFMA chains (no memory traffic in the loop).  Thread 0 of each
// workgroup writes the loop's shader cycles (s_memtime) and 100 MHz wall
// ticks to stamps[2 block], [2 block + 1]; every thread writes one value of
// its accumulators to sink[global thread] so the chains stay live.
__global__ void __launch_bounds__(256) k_mfma_rate(int iters, float* sink, uint64_t* stamps) {
    const int t = threadIdx.x;
    bf16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(0.0009765625f * (float)((t + j) & 7));
        b[j] = (__bf16)(0.0009765625f * (float)((t * 3 + j) & 7));
    }
    f32x16 acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = f32x16{};
    const uint64_t c0 = clock64(), w0 = wall_clock64();
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int k = 0; k < 8; ++k) acc[k] = mfma32(a, b, acc[k]);
    }
    const uint64_t c1 = clock64(), w1 = wall_clock64();
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) v += acc[k][t & 15];
    sink[(int64_t)blockIdx.x * 256 + t] = v;
    if (t == 0) {
        stamps[2 * blockIdx.x] = c1 - c0;
        stamps[2 * blockIdx.x + 1] = w1 - w0;
    }
}

extern "C" {
int mr_selftest_mfma16(const void* A, const void* B, void* D, void* stream) {
    hipLaunchKernelGGL(k_mfma16, dim3(1), dim3(64), 0, (hipStream_t)stream, (const uint16_t*)A,
                       (const uint16_t*)B, (float*)D);
    return hipGetLastError() == hipSuccess ? 0 : 6;
}
int mr_selftest_mfma32(const void* A, const void* B, void* D, void* stream) {
    hipLaunchKernelGGL(k_mfma32, dim3(1), dim3(64), 0, (hipStream_t)stream, (const uint16_t*)A,
                       (const uint16_t*)B, (float*)D);
    return hipGetLastError() == hipSuccess ? 0 : 6;
}
int mr_selftest_permlane32(const void* d_in, void* d_out, void* stream) {
    hipLaunchKernelGGL(k_permlane32, dim3(1), dim3(64), 0, (hipStream_t)stream, (const uint32_t*)d_in,
                       (uint32_t*)d_out);
    return hipGetLastError() == hipSuccess ? 0 : 6;
}
int mr_selftest_permlane16(const void* d_in, void* d_out, void* stream) {
    hipLaunchKernelGGL(k_permlane16, dim3(1), dim3(64), 0, (hipStream_t)stream, (const uint32_t*)d_in,
                       (uint32_t*)d_out);
    return hipGetLastError() == hipSuccess ? 0 : 6;
}
int mr_selftest_permlane16_pair(const void* d_in, void* d_out, void* stream) {
    hipLaunchKernelGGL(k_permlane16_pair, dim3(1), dim3(64), 0, (hipStream_t)stream, (const uint32_t*)d_in,
                       (uint32_t*)d_out);
    return hipGetLastError() == hipSuccess ? 0 : 6;
}
int mr_selftest_tr16(const int32_t* host_offsets, const void* d_offsets, void* d_out, void* stream) {
    for (int i = 0; i < 64; ++i)
        if (host_offsets[i] < 0 || host_offsets[i] > 4096 - 8 || (host_offsets[i] % 8) != 0) return 1;
    hipLaunchKernelGGL(k_tr16, dim3(1), dim3(64), 0, (hipStream_t)stream, (const int32_t*)d_offsets,
                       (uint16_t*)d_out);
    return hipGetLastError() == hipSuccess ? 0 : 6;
}
// sink: blocks * 256 floats, stamps: 2 * blocks uint64 (device)
int mr_selftest_mfma_rate(int blocks, int iters, void* sink, void* stamps, void* stream) {
    if (blocks <= 0 || iters <= 0) return 1;
    hipLaunchKernelGGL(k_mfma_rate, dim3(blocks), dim3(256), 0, (hipStream_t)stream, iters, (float*)sink,
                       (uint64_t*)stamps);
    return hipGetLastError() == hipSuccess ? 0 : 6;
}
}
