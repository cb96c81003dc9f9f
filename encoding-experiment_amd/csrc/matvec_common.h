// Shared pieces of the Q4_K / Q6_K matvec kernels: launch arguments, the wave reductions
// and the epilogues.
#pragma once

#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

enum MvEpi : int {
    EPI_STORE = 0,      // out[n] = dot
    EPI_RESID = 1,      // out[n] = resid[n] + dot              (residual add, LI/src/forward/layer.rs:88-92)
    EPI_GATED_PAIR = 2,  // rows interleaved gate/up: out[n/2] = act(gate) * up  (LI/src/ffn/mod.rs:87-103)
    EPI_GATED_MUL = 3,   // out[n] = act(resid[n]) * dot: the up projection after a separate gate
};

struct MvArgs {
    // weight (device layout)
    const uint8_t* qs = nullptr;   // Q4_K nibbles / Q6_K tile-major blocks
    const uint4* hdr = nullptr;    // Q4_K headers
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
    int act = 0;             // gated epilogues: 0 = SiLU, 1 = GELU-tanh (Activation, LC/src/pipeline.rs:48-54)
    float out_scale = 1.0f;  // EPI_RESID: (resid + dot) * out_scale, the layer scalar (LC/src/metal/decode.rs:717-728)
    // Q4_K MFMA kernel only.  Producer (EPI_RESID): also out2[n] = out[n] * (out2_off +
    // out2_w[n]), the next matvec's norm-weighted input, and psum[workgroup] = sum of
    // out[n]^2 over the workgroup's rows (f64).  Consumer: x already carries the norm
    // weight; x_psum[0 .. x_npsum) are its producer's partial sums of squares, and the row
    // totals are scaled by 1 / sqrt(sum / cols + eps) (an RMSNorm whose statistics come
    // with its input).
    float* out2 = nullptr;
    const float* out2_w = nullptr;
    float out2_off = 0.f;
    double* psum = nullptr;
    const double* x_psum = nullptr;
    int x_npsum = 0;
    // launch shape: rounds per wave, CUs on the device, device rows (a multiple of 64;
    // rows past `rows` decode to zero)
    int steps = 1, num_cus = 0, rows_pad = 0;
};

// Transposing reduction across 32- and 16-lane halves (gfx950 permlane swaps): after
// swap(A, B) and A + B, the lower half of the result holds A's pair sums and the upper
// half B's.  With A == B it is a plain butterfly step.
__device__ __forceinline__ float swap32_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap16_add(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_1032 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;  // quad_perm [2,3,0,1]

__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sig = 1.0f / (1.0f + expf(-g));
    return (g * sig) * u;
}

// gelu_tanh(g) * u, gelu_tanh(x) = 0.5 x (1 + tanh(0.7978846 (x + 0.044715 x^3)))
// (LI/src/ffn/mod.rs:96-103).
__device__ __forceinline__ float gelu_tanh_mul(float g, float u) {
    const float inner = 0.7978846f * (g + 0.044715f * g * g * g);
    return (0.5f * g * (1.0f + tanhf(inner))) * u;
}

__device__ __forceinline__ float gated_act(int act, float g, float u) {
    return act == 1 ? gelu_tanh_mul(g, u) : silu_mul(g, u);
}

// Output of a non-pair epilogue for a row whose dot is `tot` and resid value `rv`.
__device__ __forceinline__ float epi_value(const MvArgs& a, float rv, float tot) {
    if (a.epi == EPI_RESID) return (rv + tot) * a.out_scale;
    if (a.epi == EPI_GATED_MUL) return gated_act(a.act, rv, tot);
    return tot;
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
void launch_q4k_mfma(const DevWeight& w, MvArgs a, hipStream_t s);
// Q6_K on the matrix cores (matvec_q6k_mfma.hip); no prenormed input or second output.
bool q6k_mfma_supported(const DevWeight& w);
void launch_q6k_mfma(const DevWeight& w, MvArgs a, hipStream_t s);
// Workgroups of launch_q4k_mfma for this weight (the partial sums a producer writes), and
// the most partial sums its launch can take as a consumer (two per thread).
int q4k_mfma_groups(const DevWeight& w, int num_cus);
int q4k_mfma_max_psum(const DevWeight& w, int num_cus);
// The launch split of the weight's m = 1 matvec (pick_q4k_split) and its grid.
struct Q4kShape {
    int ur, tiles, pre, xb, rounds;
    unsigned groups, threads;
};
Q4kShape q4k_mfma_shape(const DevWeight& w, int num_cus);

}  // namespace larql
