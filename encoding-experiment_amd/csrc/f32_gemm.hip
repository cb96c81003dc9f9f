// f32 matrix products of the trait: ComputeBackend::matmul (C = A . B) and matmul_transb
// (C = A . B^T), LC/src/backend.rs:27-31 (the Metal backend runs both as tiled sgemm
// kernels, LC/src/metal/f32_ops.rs:93-140).
//
// Every element of C is one f32 fma chain over k = 0 .. K-1 starting from +0, the
// canonical order of the gate-score kernel, so a product is reproducible bit for bit and
// equals the oracle's chain; the reference CPU path (matrixmultiply's blocked sgemm) sums in
// its own order, within f32 rounding of this one.
//
// Workgroup tile: 256 "rows" (operand R) x 64 "columns" (operand C), thread tile 8 x 8,
// K in LDS stages of 16 (double-buffered, the next stage's global loads held in registers
// while the current one is consumed).  Each operand may be k-minor in memory (a row of K
// floats per row / column) or k-major (a row of the other dimension per k); the LDS tiles
// are k-major either way.  The launcher puts the larger of m and n on the 256 side and
// stores C transposed when it swaps them.  Loads are scalar and predicated (any K, any
// alignment); rows and columns past the matrix are clamped duplicates, never stored.
#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

namespace {

constexpr int kGThreads = 256;
constexpr int kGTileR = 256, kGTileC = 64, kGKs = 16;

template <bool R_KMAJOR, bool C_KMAJOR, bool OUT_T>
__global__ __launch_bounds__(kGThreads) void f32_gemm_kernel(const float* __restrict__ R, size_t ldr,
                                                             const float* __restrict__ Cm, size_t ldc,
                                                             float* __restrict__ out, size_t ldo, int Rn, int Cn,
                                                             int K) {
    __shared__ float Rs[2][kGKs][kGTileR];
    __shared__ float Cs[2][kGKs][kGTileC];
    const int tid = threadIdx.x;
    const int r0 = blockIdx.y * kGTileR, c0 = blockIdx.x * kGTileC;
    const int tr = tid & 31, tc = tid >> 5;  // rows r0 + 8 tr .., columns c0 + 8 tc ..

    // R stage: k-minor, thread = row r0 + tid, 16 consecutive k; k-major, thread =
    // (rows r0 + 4 (tid & 63) .. + 3, k 4 (tid >> 6) .. + 3)
    float rv[16];
    auto rload = [&](int k0) __attribute__((always_inline)) {
        if constexpr (!R_KMAJOR) {
            const float* p = R + static_cast<size_t>(min(r0 + tid, Rn - 1)) * ldr;
#pragma unroll
            for (int i = 0; i < 16; i++) rv[i] = k0 + i < K ? p[k0 + i] : 0.f;
        } else {
            const int rr = 4 * (tid & 63), kk = 4 * (tid >> 6);
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const int k = k0 + kk + a;
                    rv[4 * a + b] = k < K ? R[static_cast<size_t>(k) * ldr + min(r0 + rr + b, Rn - 1)] : 0.f;
                }
        }
    };
    auto rstore = [&](int buf) __attribute__((always_inline)) {
        if constexpr (!R_KMAJOR) {
#pragma unroll
            for (int i = 0; i < 16; i++) Rs[buf][i][tid] = rv[i];
        } else {
            const int rr = 4 * (tid & 63), kk = 4 * (tid >> 6);
#pragma unroll
            for (int a = 0; a < 4; a++)
                *reinterpret_cast<float4*>(&Rs[buf][kk + a][rr]) =
                    make_float4(rv[4 * a], rv[4 * a + 1], rv[4 * a + 2], rv[4 * a + 3]);
        }
    };
    // C stage: k-minor, thread = (column c0 + (tid & 63), k 4 (tid >> 6) .. + 3); k-major,
    // thread = (columns c0 + 4 (tid & 15) .. + 3, k tid >> 4)
    float cv[4];
    auto cload = [&](int k0) __attribute__((always_inline)) {
        if constexpr (!C_KMAJOR) {
            const float* p = Cm + static_cast<size_t>(min(c0 + (tid & 63), Cn - 1)) * ldc;
            const int kk = k0 + 4 * (tid >> 6);
#pragma unroll
            for (int i = 0; i < 4; i++) cv[i] = kk + i < K ? p[kk + i] : 0.f;
        } else {
            const int k = k0 + (tid >> 4), cc = 4 * (tid & 15);
#pragma unroll
            for (int i = 0; i < 4; i++)
                cv[i] = k < K ? Cm[static_cast<size_t>(k) * ldc + min(c0 + cc + i, Cn - 1)] : 0.f;
        }
    };
    auto cstore = [&](int buf) __attribute__((always_inline)) {
        if constexpr (!C_KMAJOR) {
            const int kk = 4 * (tid >> 6);
#pragma unroll
            for (int i = 0; i < 4; i++) Cs[buf][kk + i][tid & 63] = cv[i];
        } else {
            *reinterpret_cast<float4*>(&Cs[buf][tid >> 4][4 * (tid & 15)]) = make_float4(cv[0], cv[1], cv[2], cv[3]);
        }
    };

    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = 0.f;

    const int nk = (K + kGKs - 1) / kGKs;
    if (nk > 0) {
        rload(0);
        cload(0);
        rstore(0);
        cstore(0);
    }
    __syncthreads();
    for (int s = 0; s < nk; s++) {
        const int b = s & 1;
        if (s + 1 < nk) {
            rload((s + 1) * kGKs);
            cload((s + 1) * kGKs);
        }
        // the last stage runs only its real k: no padded term enters a chain
        const int kend = min(kGKs, K - s * kGKs);
#pragma unroll 2
        for (int k = 0; k < kend; k++) {
            const float4 ra = *reinterpret_cast<const float4*>(&Rs[b][k][tr * 8]);
            const float4 rb = *reinterpret_cast<const float4*>(&Rs[b][k][tr * 8 + 4]);
            const float4 ca = *reinterpret_cast<const float4*>(&Cs[b][k][tc * 8]);
            const float4 cb = *reinterpret_cast<const float4*>(&Cs[b][k][tc * 8 + 4]);
            const float rw[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
            const float cw[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc[i][j] = fmaf(cw[j], rw[i], acc[i][j]);
        }
        // buffer b ^ 1 was last read in stage s - 1, before that stage's barrier
        if (s + 1 < nk) {
            rstore(b ^ 1);
            cstore(b ^ 1);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = r0 + tr * 8 + i;
        if (r >= Rn) continue;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int c = c0 + tc * 8 + j;
            if (c >= Cn) continue;
            if constexpr (OUT_T) out[static_cast<size_t>(c) * ldo + r] = acc[i][j];
            else out[static_cast<size_t>(r) * ldo + c] = acc[i][j];
        }
    }
}

template <bool RK, bool CK, bool OT>
void launch_gemm(const float* R, size_t ldr, const float* Cm, size_t ldc, float* out, size_t ldo, size_t Rn,
                 size_t Cn, size_t K, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>((Cn + kGTileC - 1) / kGTileC),
                    static_cast<unsigned>((Rn + kGTileR - 1) / kGTileR));
    f32_gemm_kernel<RK, CK, OT><<<grid, dim3(kGThreads), 0, s>>>(R, ldr, Cm, ldc, out, ldo, static_cast<int>(Rn),
                                                                 static_cast<int>(Cn), static_cast<int>(K));
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace

void launch_f32_matmul(const float* A, const float* B, float* C, size_t m, size_t k, size_t n, bool transpose_b,
                       hipStream_t s) {
    if (m == 0 || n == 0) return;
    if (m > 0x7FFFFFFFu || n > 0x7FFFFFFFu || k > 0x7FFFFFFFu || (m + kGTileR - 1) / kGTileR > 65535 ||
        (n + kGTileR - 1) / kGTileR > 65535)
        fail(LARQL_HIP_ERR_INVALID, "matmul: dimensions too large");
    // A [m][k] is k-minor; B is [n][k] (k-minor, transpose_b) or [k][n] (k-major).  The
    // larger of m and n goes on the 256 side; C [m][n] is stored transposed when n is there.
    if (transpose_b) {
        if (m >= n) launch_gemm<false, false, false>(A, k, B, k, C, n, m, n, k, s);
        else launch_gemm<false, false, true>(B, k, A, k, C, n, n, m, k, s);
    } else {
        if (m >= n) launch_gemm<false, true, false>(A, k, B, n, C, n, m, n, k, s);
        else launch_gemm<true, false, true>(B, n, A, k, C, n, n, m, k, s);
    }
}

}  // namespace larql
