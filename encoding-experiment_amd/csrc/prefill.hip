// Quantized prefill: Y[M x N] = X[M x K] . deq(W)^T for a Q4_K weight W [N x K],
// M tokens at once (M = 512 in the prefill workload).
//
// Reference semantics: the trait's prefill (LC/src/backend.rs:143-152) runs, per token,
// the Q4_K matvec (LC/src/cpu/ops/q4k_matvec.rs:31-90; the Metal prefill is that matvec
// in a loop over positions, LC/src/metal/prefill.rs:21-110).  Here the M matvecs are one
// GEMM on the matrix cores:
//   * the loaders dequantize each 32-element sub-block of W (d * sc_j * q - dmin * m_j in
//     f32, then fp16) and convert X to fp16, straight into LDS (double-buffered);
//   * v_mfma_f32_16x16x32_f16 accumulates in f32.
// fp16 operands carry 11 significant bits: over K = 2560 random terms the error is
// ~1e-4 of max|Y|, inside the 1e-3 bar.
#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kMt = 128, kNt = 128, kKs = 32;
constexpr int kRow = kKs + 8;  // LDS row pitch in halves (80 bytes: conflict-free 16-lane reads)

__device__ __forceinline__ half8 to_half8(float4 a, float4 b) {
    half8 h;
    h[0] = static_cast<_Float16>(a.x); h[1] = static_cast<_Float16>(a.y);
    h[2] = static_cast<_Float16>(a.z); h[3] = static_cast<_Float16>(a.w);
    h[4] = static_cast<_Float16>(b.x); h[5] = static_cast<_Float16>(b.y);
    h[6] = static_cast<_Float16>(b.z); h[7] = static_cast<_Float16>(b.w);
    return h;
}

// Eight weights from four nibble bytes: byte i holds elements 2i (low) and 2i+1 (high).
__device__ __forceinline__ half8 deq8(uint32_t bytes, float sc, float mn) {
    half8 h;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t b = (bytes >> (8 * i)) & 0xFFu;
        h[2 * i] = static_cast<_Float16>(fmaf(sc, static_cast<float>(b & 0xFu), -mn));
        h[2 * i + 1] = static_cast<_Float16>(fmaf(sc, static_cast<float>(b >> 4), -mn));
    }
    return h;
}

// Grid (ceil(N / 128), ceil(M / 128)); four waves, each a 64 x 64 block of Y as 4 x 4
// MFMA tiles of 16 x 16.
__global__ __launch_bounds__(kThreads, 2) void q4k_gemm_kernel(const uint8_t* __restrict__ qs,
                                                               const uint4* __restrict__ hdr,
                                                               const float* __restrict__ X, float* __restrict__ Y,
                                                               int M, int N, int K) {
    __shared__ _Float16 Xs[2][kMt][kRow];
    __shared__ _Float16 Ws[2][kNt][kRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * kNt, m0 = blockIdx.y * kMt;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * 64;

    // loaders: two threads per row, 16 consecutive k each
    const int lr = tid >> 1, lh = (tid & 1) * 16;
    const float* xp = X + static_cast<size_t>(min(m0 + lr, M - 1)) * K + lh;
    const size_t wrow = static_cast<size_t>(min(n0 + lr, N - 1));
    const size_t S = static_cast<size_t>(K / 256);
    float4 xr[4];
    uint2 wqv;
    uint4 whv;
    auto gload = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; i++) xr[i] = *reinterpret_cast<const float4*>(xp + k0 + 4 * i);
        wqv = *reinterpret_cast<const uint2*>(qs + q4k_sub_offset(wrow, k0 >> 8, (k0 >> 5) & 7, S) + lh / 2);
        whv = hdr[q4k_hdr_index(wrow, k0 >> 8, S)];
    };
    auto lstore = [&](int b, int k0) __attribute__((always_inline)) {
        *reinterpret_cast<half8*>(&Xs[b][lr][lh]) = to_half8(xr[0], xr[1]);
        *reinterpret_cast<half8*>(&Xs[b][lr][lh + 8]) = to_half8(xr[2], xr[3]);
        const int j = (k0 >> 5) & 7;  // sub-block within the super-block
        const float d = h2f(whv.x), dmin = h2f(whv.x >> 16);
        const uint32_t scw = j < 4 ? whv.y : whv.z;
        const float sc = d * static_cast<float>((scw >> (8 * (j & 3))) & 0x3Fu);
        const float mn = dmin * static_cast<float>((whv.w >> (8 * (j & 3) + (j < 4 ? 0 : 4))) & 0xFu);
        *reinterpret_cast<half8*>(&Ws[b][lr][lh]) = deq8(wqv.x, sc, mn);
        *reinterpret_cast<half8*>(&Ws[b][lr][lh + 8]) = deq8(wqv.y, sc, mn);
    };

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int nk = K / kKs;
    const int fr = lane & 15, fk = 8 * (lane >> 4);
    gload(0);
    lstore(0, 0);
    __syncthreads();
    for (int s = 0; s < nk; s++) {
        const int b = s & 1;
        if (s + 1 < nk) gload((s + 1) * kKs);
        half8 a[4], w[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            a[t] = *reinterpret_cast<const half8*>(&Xs[b][wm + 16 * t + fr][fk]);
            w[t] = *reinterpret_cast<const half8*>(&Ws[b][wn + 16 * t + fr][fk]);
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], w[j], acc[i][j], 0, 0, 0);
        // buffer b ^ 1 was last read in step s - 1, before that step's barrier
        if (s + 1 < nk) lstore(b ^ 1, (s + 1) * kKs);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + wn + 16 * j + fr;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm + 16 * i + 4 * (lane >> 4) + r;
                if (m < M && n < N) Y[static_cast<size_t>(m) * N + n] = acc[i][j][r];
            }
        }
}

}  // namespace

void launch_q4k_gemm(const DevWeight& w, const float* X, float* Y, size_t m, hipStream_t s) {
    if (w.format != LARQL_Q4_K) fail(LARQL_HIP_ERR_UNSUPPORTED, "prefill GEMM: Q4_K weights only");
    if (m == 0) return;
    if (m > 0x7FFFFFFF / w.cols) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: too many tokens");
    const dim3 grid(static_cast<unsigned>((w.rows + kNt - 1) / kNt), static_cast<unsigned>((m + kMt - 1) / kMt));
    q4k_gemm_kernel<<<grid, dim3(kThreads), 0, s>>>(w.qs, w.hdr, X, Y, static_cast<int>(m), static_cast<int>(w.rows),
                                                     static_cast<int>(w.cols));
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
