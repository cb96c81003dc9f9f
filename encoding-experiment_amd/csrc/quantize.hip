// Weight quantizers on the device, byte-identical to the reference's host quantizers
// (LC/src/cpu/ops/q4_common.rs):
//   quantize_q4_0 (:50-81)   -> 18 B / 32
//   quantize_q4_k (:104-170) -> 148 B / 256
//   quantize_q6_k (:179-239) -> 210 B / 256
//   quantize_weights_q8 (LC/src/cpu/ops/q8_matvec.rs:11-34) -> i8 + f32 scales
// Numerics follow the Rust source: IEEE division (hipcc's default correctly
// rounded f32 divide), round-half-away-from-zero (roundf), clamps before the
// integer cast, f16 stored by truncation with subnormals flushed (q4_common.rs:83-95).
// One thread per block / super-block; each thread reads its elements once.
#include "device_common.h"
#include "larql_hip_internal.h"

#pragma clang fp contract(off)

namespace larql {

__device__ __forceinline__ uint16_t f32_to_f16_trunc(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int exp = static_cast<int>((bits >> 23) & 0xFFu);
    const uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0) return static_cast<uint16_t>(sign);
    if (exp == 255) return static_cast<uint16_t>(sign | 0x7C00u | (mant >> 13));
    const int ne = exp - 127 + 15;
    if (ne >= 31) return static_cast<uint16_t>(sign | 0x7C00u);
    if (ne <= 0) return static_cast<uint16_t>(sign);
    return static_cast<uint16_t>(sign | (static_cast<uint32_t>(ne) << 10) | (mant >> 13));
}

__device__ __forceinline__ float clampf(float v, float lo, float hi) {
    v = v < lo ? lo : v;
    return v > hi ? hi : v;
}

// Rust `f as u8` / `as i8` of an already clamped value (NaN -> 0).
__device__ __forceinline__ uint32_t to_u8(float f) { return isnan(f) ? 0u : static_cast<uint32_t>(f); }
__device__ __forceinline__ int to_i8(float f) { return isnan(f) ? 0 : static_cast<int>(f); }

// Rust `f as i32` (saturating, NaN -> 0).
__device__ __forceinline__ int sat_i32(float f) {
    if (isnan(f)) return 0;
    if (f >= 2147483647.0f) return 2147483647;
    if (f <= -2147483648.0f) return -2147483647 - 1;
    return static_cast<int>(f);
}

__global__ void quantize_q4_0_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, size_t nblocks) {
    const size_t b = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (b >= nblocks) return;
    const float* blk = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i]));
    const float scale = amax / 7.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    uint8_t* o = out + b * 18;
    const uint16_t h = f32_to_f16_trunc(scale);
    o[0] = static_cast<uint8_t>(h & 0xFF);
    o[1] = static_cast<uint8_t>(h >> 8);
    for (int j = 0; j < 16; j++) {
        int lo = sat_i32(roundf(blk[2 * j] * inv)) + 8;
        int hi = sat_i32(roundf(blk[2 * j + 1] * inv)) + 8;
        lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
        hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
        o[2 + j] = static_cast<uint8_t>(lo | (hi << 4));
    }
}

__global__ void quantize_q4_k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, size_t nsb) {
    const size_t sb = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (sb >= nsb) return;
    const float* blk = x + sb * 256;
    uint8_t* o = out + sb * 148;
    float smin[8], smax[8];
    for (int j = 0; j < 8; j++) {
        float mn = INFINITY, mx = -INFINITY;
        for (int i = 0; i < 32; i++) {
            mn = fminf(mn, blk[j * 32 + i]);
            mx = fmaxf(mx, blk[j * 32 + i]);
        }
        smin[j] = mn;
        smax[j] = mx;
    }
    float gmr = 0.0f, gmin = INFINITY;
    for (int j = 0; j < 8; j++) gmr = fmaxf(gmr, smax[j] - smin[j]);
    for (int j = 0; j < 8; j++) gmin = fminf(gmin, smin[j]);
    const float d = gmr > 0.0f ? gmr / 63.0f : 0.0f;
    const float dmin = gmin < 0.0f ? -gmin / 15.0f : 0.0f;
    const uint16_t hd = f32_to_f16_trunc(d), hm = f32_to_f16_trunc(dmin);
    o[0] = hd & 0xFF; o[1] = hd >> 8; o[2] = hm & 0xFF; o[3] = hm >> 8;
    uint32_t qs[8], qm[8];
    for (int j = 0; j < 8; j++) {
        const float range = smax[j] - smin[j];
        qs[j] = d > 0.0f ? to_u8(clampf(roundf(range / d), 0.0f, 63.0f)) : 0u;
        qm[j] = dmin > 0.0f ? to_u8(clampf(roundf(-smin[j] / dmin), 0.0f, 15.0f)) : 0u;
    }
    for (int j = 0; j < 8; j++) o[4 + j] = static_cast<uint8_t>(qs[j] & 0x3F);
    for (int j = 8; j < 12; j++) o[4 + j] = 0;
    for (int j = 0; j < 4; j++) o[16 + j] = static_cast<uint8_t>((qm[j] & 0xF) | ((qm[j + 4] & 0xF) << 4));
    for (int j = 0; j < 8; j++) {
        const float sc = d * static_cast<float>(qs[j]);
        const float mn = dmin * static_cast<float>(qm[j]);
        const float inv_sc = sc > 0.0f ? 1.0f / sc : 0.0f;
        const float* sub = blk + j * 32;
        for (int i = 0; i < 16; i++) {
            const uint32_t v0 = to_u8(clampf(roundf((sub[2 * i] + mn) * inv_sc), 0.0f, 15.0f));
            const uint32_t v1 = to_u8(clampf(roundf((sub[2 * i + 1] + mn) * inv_sc), 0.0f, 15.0f));
            o[20 + j * 16 + i] = static_cast<uint8_t>(v0 | (v1 << 4));
        }
    }
}

__global__ void quantize_q6_k_kernel(const float* __restrict__ x, uint8_t* __restrict__ out, size_t nsb) {
    const size_t sb = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (sb >= nsb) return;
    const float* blk = x + sb * 256;
    uint8_t* o = out + sb * 210;
    float amax = 0.0f;
    for (int i = 0; i < 256; i++) amax = fmaxf(amax, fabsf(blk[i]));
    const float d = amax / 32.0f;
    int ssc[16];
    for (int j = 0; j < 16; j++) {
        float smx = 0.0f;
        for (int i = 0; i < 16; i++) smx = fmaxf(smx, fabsf(blk[j * 16 + i]));
        const float sc = d > 0.0f ? smx / d : 0.0f;
        ssc[j] = to_i8(clampf(roundf(sc), -128.0f, 127.0f));
    }
    uint32_t qhw[16];
#pragma unroll
    for (int w = 0; w < 16; w++) qhw[w] = 0u;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float sc = d * static_cast<float>(ssc[j]);
        const float inv_sc = fabsf(sc) > 1e-10f ? 1.0f / sc : 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            const int idx = j * 16 + i;
            const int q0 = to_i8(clampf(roundf(blk[idx] * inv_sc), -32.0f, 31.0f)) + 32;
            const int q1 = to_i8(clampf(roundf(blk[idx + 1] * inv_sc), -32.0f, 31.0f)) + 32;
            o[idx / 2] = static_cast<uint8_t>((q0 & 0xF) | ((q1 & 0xF) << 4));
            // element e's two high bits live at qh byte e/4, shift 2*(e%4): bit 2*(e%16) of word e/16
            qhw[idx / 16] |= static_cast<uint32_t>((q0 >> 4) & 3) << (2 * (idx % 16));
            qhw[idx / 16] |= static_cast<uint32_t>((q1 >> 4) & 3) << (2 * ((idx + 1) % 16));
        }
    }
#pragma unroll
    for (int w = 0; w < 16; w++)
#pragma unroll
        for (int k = 0; k < 4; k++) o[128 + 4 * w + k] = static_cast<uint8_t>(qhw[w] >> (8 * k));
    for (int j = 0; j < 16; j++) o[192 + j] = static_cast<uint8_t>(static_cast<int8_t>(ssc[j]));
    const uint16_t hd = f32_to_f16_trunc(d);
    o[208] = hd & 0xFF;
    o[209] = hd >> 8;
}

__global__ void quantize_weights_q8_kernel(const float* __restrict__ x, int8_t* __restrict__ q,
                                           float* __restrict__ scales, size_t nblocks) {
    const size_t b = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (b >= nblocks) return;
    const float* blk = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(blk[i]));
    const float scale = amax / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    scales[b] = scale;
    for (int i = 0; i < 32; i++) q[b * 32 + i] = static_cast<int8_t>(to_i8(clampf(roundf(blk[i] * inv), -128.0f, 127.0f)));
}

void launch_quantize_weights(int format, const float* x, size_t n, void* out, float* q8_scales, hipStream_t s) {
    const int T = 256;
    switch (format) {
        case LARQL_Q4_0: {
            const size_t nb = n / 32;
            quantize_q4_0_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(x, static_cast<uint8_t*>(out), nb);
            break;
        }
        case LARQL_Q4_K: {
            const size_t nb = n / 256;
            quantize_q4_k_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(x, static_cast<uint8_t*>(out), nb);
            break;
        }
        case LARQL_Q6_K: {
            const size_t nb = n / 256;
            quantize_q6_k_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(x, static_cast<uint8_t*>(out), nb);
            break;
        }
        case LARQL_Q8_0: {
            const size_t nb = n / 32;
            quantize_weights_q8_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(x, static_cast<int8_t*>(out),
                                                                                  q8_scales, nb);
            break;
        }
        default: fail(LARQL_HIP_ERR_UNSUPPORTED, "quantize: unsupported format");
    }
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
