// x fixed-point levels for the K-quant matvecs: one 32-element sub-block of the
// (normalised) activation as two byte planes laid out for v_dot4 against 4-bit and
// 6-bit weight codes.
#pragma once

#include "device_common.h"

namespace larql {

// Three-level byte image of one 32-element x sub-block, laid out for v_dot4 against
// nibble dwords: word w of a level holds elements {8w+0, 8w+2, 8w+4, 8w+6} (even) or
// {8w+1, 8w+3, 8w+5, 8w+7} (odd), one per byte.  x is held in 23-bit fixed point
//   T = rint(x * (2^22 - 1) / amax) = 65536 a + 256 b + c,   |T| < 2^22,
// level 0 = a (signed byte 2 of T, in [-64, 63]), levels 1, 2 = b, c (unsigned bytes
// 1, 0).  |x - s' T| <= s'/2 = 1.2e-7 amax with s' = amax / (2^22 - 1): the size of
// an f32 rounding of the block's largest element.  (Sixteen-bit T was tried: over a
// 32-layer decode its error is amplified past the 1e-3 bar on the logits.)
struct XLevels {
    uint32_t ev[3][4], od[3][4];
    float sp;           // s'
    float xs;           // f32 sum of the 32 elements (Q4_K min term)
    float xs0, xs1;     // f32 sums of elements 0..15 and 16..31 (Q6_K -32 offset)
};

constexpr float kLevelScale = 4194303.0f;  // 2^22 - 1

// Byte `b` of each of four dwords, packed low to high.
__device__ __forceinline__ uint32_t gather_byte(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3, int b) {
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, 0x0C0C0400u + 0x0101u * b);  // t0.b, t1.b
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, 0x04000C0Cu + 0x01010000u * b);  // t2.b, t3.b
    return lo | hi;
}

// T_k is taken from the bit pattern of fma(x_k, inv, 1.5 * 2^23): the sum lies in
// [2^23, 2^24), where the f32 spacing is 1, so the single rounding of the fma gives
// 1.5 * 2^23 + rint(x_k * inv) and the low 16 bits of its encoding are T_k in two's
// complement (|T_k| <= 32513 < 2^22).  One VALU op per element instead of three.
// Pairwise (tree) reductions: VALU results are ~32 cycles away from a dependent use on
// gfx950, so a 32-long serial chain costs ~1000 cycles where a tree costs ~160.
template <int N>
__device__ __forceinline__ float tree_max_abs(const float* v) {
    if constexpr (N == 1) {
        return fabsf(v[0]);
    } else {
        return fmaxf(tree_max_abs<N / 2>(v), tree_max_abs<N / 2>(v + N / 2));
    }
}
template <int N>
__device__ __forceinline__ float tree_sum(const float* v) {
    if constexpr (N == 1) {
        return v[0];
    } else {
        return tree_sum<N / 2>(v) + tree_sum<N / 2>(v + N / 2);
    }
}

// T_k comes from the encoding of fma(x_k, inv, 1.5 * 2^23): the sum lies in
// [2^23, 2^24), where the f32 spacing is 1, so the single rounding of the fma gives
// 1.5 * 2^23 + rint(x_k * inv), whose bits minus those of 1.5 * 2^23 are T_k.
__device__ __forceinline__ void make_levels(const float (&x)[32], XLevels& L) {
    const float amax = tree_max_abs<32>(x);
    const float s0 = tree_sum<16>(x);
    const float s1 = tree_sum<16>(x + 16);
    const float inv = amax > 0.f ? kLevelScale / amax : 0.f;
    const float sp = amax / kLevelScale;
    uint32_t T[32];
#pragma unroll
    for (int k = 0; k < 32; k++) T[k] = __float_as_uint(fmaf(x[k], inv, 12582912.0f)) - 0x4B400000u;
#pragma unroll
    for (int l = 0; l < 3; l++)
#pragma unroll
        for (int w = 0; w < 4; w++) {
            L.ev[l][w] = gather_byte(T[8 * w + 0], T[8 * w + 2], T[8 * w + 4], T[8 * w + 6], 2 - l);
            L.od[l][w] = gather_byte(T[8 * w + 1], T[8 * w + 3], T[8 * w + 5], T[8 * w + 7], 2 - l);
        }
    L.sp = sp;
    L.xs = s0 + s1;
    L.xs0 = s0;
    L.xs1 = s1;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

__device__ __forceinline__ uint32_t udot4(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_udot4(a, b, c, false);
}

// s' * sum(q * T) = s' * (65536 ia + 256 ib + ic).  256 ib + ic is formed in int32
// (< 2^31 for Q4_K and Q6_K blocks) and the float result rounds at most twice (2^-24).
__device__ __forceinline__ float combine(int ia, uint32_t ib, uint32_t ic, float sp) {
    const float lo = static_cast<float>(static_cast<int>((ib << 8) + ic));
    return fmaf(static_cast<float>(ia), sp * 65536.0f, sp * lo);
}

}  // namespace larql
