// Helpers shared by the matrix-core K-quant matvecs (matvec_q4k_mfma.hip,
// matvec_q6k_mfma.hip): the x digit planes and the non-temporal weight loads.
//
// x digit planes: per 32-element sub-block, T = rint(x * (2^22 - 1) / max|x|) is split
// into balanced signed bytes T = 65536 a + 256 b + c (a, b, c in [-128, 127]) taken from
// the bytes of T + 0x808080 with their top bits flipped.  |x - s' T| <= s'/2 with
// s' = max|x| / (2^22 - 1): the size of one f32 rounding of the sub-block's largest
// element.  Plane p holds digit p (c, b, a for p = 0, 1, 2) of every element; within a
// 16-element half the bytes are ordered as the weight codes unpack: elements 0, 2, 4, 6,
// then 1, 3, 5, 7, then 8 .. 14 and 9 .. 15 alike.
#pragma once

#include <cstdint>

namespace larql {

// One sub-block's planes in LDS: [half m][plane p] x 16 bytes, then a float4 of
// per-sub-block values (s' and the sums of x the kernel's offset terms use).
struct PlSlot {
    uint4 pl[2][3];
    float4 s;
};
static_assert(sizeof(PlSlot) == 112, "LDS plane slot");

// Byte b (b = 0, 1, 2) of each of u0..u3 -> dword b, top bits flipped: the signed digit
// planes of four elements, low to high.
__device__ __forceinline__ void pack_planes(uint32_t u0, uint32_t u1, uint32_t u2, uint32_t u3, uint32_t (&pl)[3]) {
    const uint32_t p01 = __builtin_amdgcn_perm(u1, u0, 0x05010400u);  // u0.b0 u1.b0 u0.b1 u1.b1
    const uint32_t q01 = __builtin_amdgcn_perm(u1, u0, 0x0C0C0602u);  // u0.b2 u1.b2 0 0
    const uint32_t p23 = __builtin_amdgcn_perm(u3, u2, 0x05010400u);
    const uint32_t q23 = __builtin_amdgcn_perm(u3, u2, 0x0C0C0602u);
    pl[0] = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;
    pl[1] = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;
    pl[2] = __builtin_amdgcn_perm(q23, q01, 0x05040100u) ^ 0x80808080u;
}

// Weight bytes are read exactly once: non-temporal loads keep them from displacing x and
// the planes in the caches (measured: 8.4 -> 7.9 us on a [14336 x 4096] Q4_K matvec).
__device__ __forceinline__ uint4 load_nt(const void* p) {
    typedef unsigned int v4u __attribute__((ext_vector_type(4)));
    const v4u v = __builtin_nontemporal_load(static_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace larql
