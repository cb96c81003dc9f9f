// Shared pieces of the Q4_K / Q6_K matvec kernels: launch arguments, the fused
// RMSNorm prologue, the multi-row wave reduction and the epilogues.
#pragma once

#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

enum MvEpi : int {
    EPI_STORE = 0,      // out[n] = dot
    EPI_RESID = 1,      // out[n] = resid[n] + dot              (residual add, LI/src/forward/layer.rs:88-92)
    EPI_SILU_PAIR = 2,  // rows interleaved gate/up: out[n/2] = silu(gate) * up  (LI/src/ffn/mod.rs:87-94)
};

struct MvArgs {
    // weight (device layout)
    const uint8_t* qs = nullptr;   // Q4_K nibbles / Q6_K ql
    const uint4* hdr = nullptr;    // Q4_K headers
    const uint8_t* qh = nullptr;   // Q6_K high bits
    const int8_t* sc = nullptr;    // Q6_K scales
    const uint16_t* d = nullptr;   // Q6_K f16 super-block scales
    int rows = 0, cols = 0;
    // activation / output
    const float* x = nullptr;
    float* out = nullptr;
    // fused RMSNorm of x (LI/src/residual.rs:17-33): x / rms * (offset + w)
    const float* norm_w = nullptr;  // null = no norm
    float norm_offset = 0.f;
    double eps = 1e-6;
    // epilogue
    int epi = EPI_STORE;
    const float* resid = nullptr;
    // launch shape: waves per row slot, row tiles, tiles per workgroup, CUs on the device
    int wpr = 1, tiles = 0, steps = 1, num_cus = 256;
};

// Reduce RB per-lane partials over the 64 lanes of a wave; on return lane
// (r << (6 - log2 RB)) holds the total of row r.
template <int RB>
__device__ __forceinline__ float multi_row_reduce(float (&v)[RB], int lane) {
    int n = RB;
    int mask = 32;
#pragma unroll
    for (int step = 0; step < 6; step++) {
        if (n > 1) {
            const bool upper = (lane & mask) != 0;
            const int half = n >> 1;
#pragma unroll
            for (int i = 0; i < RB / 2; i++) {
                if (i < half) {
                    float keep = upper ? v[i + half] : v[i];
                    float send = upper ? v[i] : v[i + half];
                    v[i] = keep + __shfl_xor(send, mask, 64);
                }
            }
            n = half;
        } else {
            v[0] += __shfl_xor(v[0], mask, 64);
        }
        mask >>= 1;
    }
    return v[0];
}

template <int RB>
__device__ __forceinline__ constexpr int rb_shift() {
    return RB == 1 ? 6 : RB == 2 ? 5 : RB == 4 ? 4 : 3;
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sig = 1.0f / (1.0f + expf(-g));
    return (g * sig) * u;
}

// Sum over the wpr waves of one row slot through LDS (scratch of >= nwaves doubles).
__device__ __forceinline__ double slot_sum_d(double v, double* scratch, int wave, int slot, int wpr, int lane) {
    v = wave_sum_d(v);
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    double s = 0.0;
    for (int w = 0; w < wpr; w++) s += scratch[slot * wpr + w];
    __syncthreads();
    return s;
}

// Epilogue for a totals vector after the wave reduction.  `tot` is valid in lane
// (r << rsh) for row row0 + r.  Used when the slot is a single wave.
template <int RB>
__device__ __forceinline__ void epilogue_wave(const MvArgs& a, float tot, int lane, int row0) {
    constexpr int rsh = rb_shift<RB>();
    const int r = lane >> rsh;
    const bool owner = (lane & ((1 << rsh) - 1)) == 0;
    const int row = row0 + r;
    if (a.epi == EPI_SILU_PAIR) {
        const float up = __shfl_down(tot, 1 << rsh, 64);
        if (owner && (r & 1) == 0 && row < a.rows) a.out[row >> 1] = silu_mul(tot, up);
    } else if (owner && row < a.rows) {
        a.out[row] = a.epi == EPI_RESID ? a.resid[row] + tot : tot;
    }
}

// Epilogue when lanes 0..RB-1 hold rows row0 + lane (multi-wave slots).
__device__ __forceinline__ void epilogue_lanes(const MvArgs& a, float tot, int lane, int row0, int rb) {
    const int row = row0 + lane;
    if (a.epi == EPI_SILU_PAIR) {
        const float up = __shfl_down(tot, 1, 64);
        if (lane < rb && (lane & 1) == 0 && row < a.rows) a.out[row >> 1] = silu_mul(tot, up);
    } else if (lane < rb && row < a.rows) {
        a.out[row] = a.epi == EPI_RESID ? a.resid[row] + tot : tot;
    }
}

// Load N floats starting at base[c0] (N % 4 == 0, 16-byte aligned); zeros when !valid.
template <int N>
__device__ __forceinline__ void load_slice(const float* __restrict__ base, int c0, bool valid, float (&v)[N]) {
    const float4* xp = reinterpret_cast<const float4*>(base + static_cast<size_t>(c0));
#pragma unroll
    for (int k = 0; k < N / 4; k++) {
        float4 t = valid ? xp[k] : make_float4(0.f, 0.f, 0.f, 0.f);
        v[4 * k + 0] = t.x;
        v[4 * k + 1] = t.y;
        v[4 * k + 2] = t.z;
        v[4 * k + 3] = t.w;
    }
}

void launch_mv(const DevWeight& w, MvArgs a, hipStream_t s);

}  // namespace larql
