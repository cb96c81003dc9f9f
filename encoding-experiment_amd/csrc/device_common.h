// Device-side helpers shared by the matvec, KNN, prefill and decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace larql {

// IEEE binary16 -> binary32 (exact; subnormal inputs are decoded, as the
// reference decoders LC/src/cpu/ops/q4_common.rs:426-442 and q4_dot.c:9-35 do).
// Workgroup barrier for data exchanged through LDS only: the wave's LDS accesses complete,
// then s_barrier.  __syncthreads() is also a workgroup-scope release, which waits for every
// global load in flight (vmcnt(0)): in a kernel that keeps loads in flight across its
// barriers (prefetch, or operands used after later LDS phases) that exposes their latency.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(bits16 & 0xFFFFu)));
}

__device__ __forceinline__ float ubyte0(uint32_t v) { return static_cast<float>(v & 0xFFu); }
__device__ __forceinline__ float ubyte1(uint32_t v) { return static_cast<float>((v >> 8) & 0xFFu); }
__device__ __forceinline__ float ubyte2(uint32_t v) { return static_cast<float>((v >> 16) & 0xFFu); }
__device__ __forceinline__ float ubyte3(uint32_t v) { return static_cast<float>(v >> 24); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Row statistics of one token row for the f32-accuracy GEMMs, by a 256-thread workgroup
// (all threads call it; it synchronises the workgroup): *e = the power of two that puts
// max |row| in [2^14, 2^15) (0 for a row of zeros or a non-finite maximum) and, with xs,
// xs[j] = 2^(e - 5) times the sum of the 32 elements of sub-block j, summed in f64 and
// rounded once (|xs| < 2^15).  K a multiple of 4 (of 32 with xs); row 16-byte aligned.
__device__ __forceinline__ void gemm_row_stats(const float* __restrict__ row, int K, int* __restrict__ e,
                                               float* __restrict__ xs) {
    __shared__ float wm[4];
    __shared__ int es;
    float m = 0.f;
    for (int i = 4 * static_cast<int>(threadIdx.x); i < K; i += 4 * 256) {
        const float4 v = *reinterpret_cast<const float4*>(row + i);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
        const int ev = (m > 0.f && m <= 3.4e38f) ? min(120, max(-120, 14 - ilogbf(m))) : 0;
        *e = ev;
        es = ev;
    }
    if (!xs) return;  // (uniform)
    __syncthreads();
    const double sc = ldexp(1.0, es - 5);
    const int nsb = K / 32;
    for (int j = static_cast<int>(threadIdx.x); j < nsb; j += 256) {
        const float4* p = reinterpret_cast<const float4*>(row + 32 * j);
        double sum[2] = {0.0, 0.0};  // f64: the sum is rounded once, to f32
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = p[k];
            sum[k & 1] += (static_cast<double>(v.x) + static_cast<double>(v.y)) +
                          (static_cast<double>(v.z) + static_cast<double>(v.w));
        }
        xs[j] = static_cast<float>((sum[0] + sum[1]) * sc);
    }
}

}  // namespace larql
