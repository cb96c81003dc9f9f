// x fixed point for the K-quant matvecs (matvec_q4k_mfma.hip, matvec_q6k_mfma.hip): the
// level scale and the pairwise reductions the digit-plane build uses.
#pragma once

#include "device_common.h"

namespace larql {

// x is held in 23-bit fixed point per 32-element sub-block:
//   T = rint(x * (2^22 - 1) / amax),   |T| < 2^22,
// |x - s' T| <= s'/2 = 1.2e-7 amax with s' = amax / (2^22 - 1): the size of an f32
// rounding of the block's largest element.  (Sixteen-bit T was tried: over a 32-layer
// decode its error is amplified past the 1e-3 bar on the logits.)  T_k comes from the bit
// pattern of fma(x_k, inv, 1.5 * 2^23): the sum lies in [2^23, 2^24), where the f32
// spacing is 1, so the single rounding of the fma gives 1.5 * 2^23 + rint(x_k * inv).
constexpr float kLevelScale = 4194303.0f;  // 2^22 - 1

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

}  // namespace larql
