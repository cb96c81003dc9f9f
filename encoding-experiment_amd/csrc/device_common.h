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

}  // namespace larql
