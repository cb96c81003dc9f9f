// Row kernels of the batched prompt pass (prefill_q4, LC/src/backend.rs:139-152): the
// per-position operations of a Llama layer applied to all M positions of a prompt at
// once, around the Q4_K GEMMs (prefill.hip) and the prompt-mode attention (decode.hip).
// Each follows the decode step's arithmetic for one position:
//   * RMSNorm  (LI/src/residual.rs:17-33): rms = sqrt(sum(x^2) in f64 / n + eps) rounded
//     to f32, y = (x * (1 / rms)) * w — the fused-norm prologue of the matvecs;
//   * RoPE of K (LI/src/attention/rope.rs:22-55) with the cos/sin table, K and V rounded
//     to fp16 (RNE) into the cache rows of their positions;
//   * residual add (LI/src/forward/layer.rs:88-92) and act(gate) * up
//     (LI/src/ffn/mod.rs:87-103) over gate/up rows interleaved as the fused weight emits them;
//   * the layer variants of FullPipelineLayer (LC/src/pipeline.rs:76-115): norm weight
//     offset, the post-norm residual h + norm(v) (LI/src/attention/block.rs:139-150,
//     LI/src/forward/layer.rs:76-87), the parameter-free per-head V-norm
//     (LI/src/residual.rs:86-110) and the layer scalar.  These kernels also serve the
//     decode step (one row).
#include "decode.h"
#include "matvec_common.h"

namespace larql {

namespace {

// sum(x^2) of n floats in f64 by a 256-thread workgroup -> rms as the CPU path rounds it
// (LI/src/residual.rs:24).
__device__ __forceinline__ float row_rms(const float* __restrict__ x, int n, double eps, double* red) {
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) ss += static_cast<double>(x[i]) * x[i];
    ss = wave_sum_d(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    return static_cast<float>(sqrt(tot / static_cast<double>(n) + eps));
}

// Grid M rows; 256 threads.  y = (x * (1 / rms)) * (off + w), or without a weight
// (w == null) y = x * (1 / rms) (LI/src/residual.rs:25-29: weight None -> 1.0).
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float* __restrict__ X, const float* __restrict__ w,
                                                           float off, float* __restrict__ Y, int n, double eps) {
    __shared__ double red[4];
    const float* x = X + static_cast<size_t>(blockIdx.x) * n;
    float* y = Y + static_cast<size_t>(blockIdx.x) * n;
    const float inv = 1.0f / row_rms(x, n, eps, red);
    if (w) {
        for (int i = threadIdx.x; i < n; i += 256) y[i] = (x[i] * inv) * (off + w[i]);
    } else {
        for (int i = threadIdx.x; i < n; i += 256) y[i] = x[i] * inv;
    }
}

// Post-norm residual, grid M rows: out = (h + norm(v, w)) * scale (scale 1 = none).
__global__ __launch_bounds__(256) void resid_norm_rows_kernel(const float* __restrict__ H, const float* __restrict__ V,
                                                              const float* __restrict__ w, float off, float scale,
                                                              float* __restrict__ OUT, int n, double eps) {
    __shared__ double red[4];
    const size_t r = static_cast<size_t>(blockIdx.x) * n;
    const float* v = V + r;
    const float inv = 1.0f / row_rms(v, n, eps, red);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float nv = w ? (v[i] * inv) * (off + w[i]) : v[i] * inv;
        OUT[r + i] = (H[r + i] + nv) * scale;
    }
}

// Parameter-free RMS norm of each V head in place: grid (M rows, num_kv heads), one wave;
// head h of row p starts at X + p * ld + h * hd.
__global__ __launch_bounds__(64) void vnorm_rows_kernel(float* __restrict__ X, int ld, int hd, double eps) {
    float* v = X + static_cast<size_t>(blockIdx.x) * ld + static_cast<size_t>(blockIdx.y) * hd;
    double ss = 0.0;
    for (int i = threadIdx.x; i < hd; i += 64) ss += static_cast<double>(v[i]) * v[i];
    ss = wave_sum_d(ss);
    const float rms = static_cast<float>(sqrt(ss / static_cast<double>(hd) + eps));
    for (int i = threadIdx.x; i < hd; i += 64) v[i] = v[i] / rms;
}

// Thread per (position p, kv element j): K RoPE'd at p, K and V to fp16 in the cache.
__global__ void rope_kv_rows_kernel(const float* __restrict__ QKV, int M, int p0, int ld, int q_dim, int kv_dim,
                                    int hd, int half, const float2* __restrict__ rope, __half* __restrict__ kc,
                                    __half* __restrict__ vc, int num_kv) {
    const size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (t >= static_cast<size_t>(M) * kv_dim) return;
    const int p = static_cast<int>(t / kv_dim), j = static_cast<int>(t - static_cast<size_t>(p) * kv_dim);
    const int kvh = j / hd, d = j - kvh * hd, pos = p0 + p;
    const float* row = QKV + static_cast<size_t>(p) * ld;
    const float* k = row + q_dim + kvh * hd;
    const float2* cs = rope + static_cast<size_t>(pos) * half;
    float kr = k[d];
    if (d < half) kr = k[d] * cs[d].x - k[d + half] * cs[d].y;
    else if (d < 2 * half) kr = k[d - half] * cs[d - half].y + k[d] * cs[d - half].x;
    kc[(static_cast<size_t>(pos) * num_kv + kvh) * hd + d] = __float2half_rn(kr);
    vc[((static_cast<size_t>(pos >> 3) * num_kv + kvh) * hd + d) * 8 + (pos & 7)] =
        __float2half_rn(row[q_dim + kv_dim + j]);
}

__global__ void add_rows_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                                size_t n, float scale) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i < n) out[i] = (a[i] + b[i]) * scale;
}

// GU rows [M][2 inter] with gate and up interleaved (2i, 2i + 1) -> act [M][inter].
__global__ void gated_pair_rows_kernel(const float* __restrict__ GU, float* __restrict__ act, size_t n, int kind) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i < n) act[i] = gated_act(kind, GU[2 * i], GU[2 * i + 1]);
}

// act[i] = act(G[i]) * U[i] (gate and up in separate buffers).
__global__ void gated_mul_kernel(const float* __restrict__ G, const float* __restrict__ U, float* __restrict__ act,
                                 size_t n, int kind) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i < n) act[i] = gated_act(kind, G[i], U[i]);
}

// ── Fused row kernels of the prompt pass ─────────────────────────────────
// One workgroup per row; the row stays in LDS (kFusedRowMax floats at most) between the
// steps, and each thread's loads of a chunk are issued together (indices clamped into
// the row, so no load sits under a branch), so a row costs one round trip to memory per
// chunk and two workgroup barriers instead of a dependent load per element.
constexpr int kRowChunk = 16;  // elements per thread per chunk

// The row's exponent (every thread gets it; thread 0 stores it) and, with xs, its scaled
// sub-block sums from the row in LDS: the arithmetic of gemm_row_stats, whose maximum is
// order-free and whose sums run per sub-block in one thread.  m: this thread's max |x|;
// wm: one float per wave.
template <int NT>
__device__ __forceinline__ void lds_row_stats(const float* row, int n, float m, float* wm, int* __restrict__ e,
                                              float* __restrict__ xs) {
    const int t = threadIdx.x;
    m = wave_max(m);
    if ((t & 63) == 0) wm[t >> 6] = m;
    __syncthreads();
    m = wm[0];
#pragma unroll
    for (int k = 1; k < NT / 64; k++) m = fmaxf(m, wm[k]);
    const int ev = (m > 0.f && m <= 3.4e38f) ? min(120, max(-120, 14 - ilogbf(m))) : 0;
    if (t == 0) *e = ev;
    if (!xs) return;
    const double sc = ldexp(1.0, ev - 5);
    for (int j = t; j < n / 32; j += NT) {
        const float4* p = reinterpret_cast<const float4*>(row + 32 * j);
        double sum[2] = {0.0, 0.0};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = p[k];
            sum[k & 1] += (static_cast<double>(v.x) + static_cast<double>(v.y)) +
                          (static_cast<double>(v.z) + static_cast<double>(v.w));
        }
        xs[j] = static_cast<float>((sum[0] + sum[1]) * sc);
    }
}

// Grid M rows; 256 threads.  The residual step after a projection and the next
// projection's input, per row of n floats, in the arithmetic of the separate kernels:
//   y = the projection row, its `splits` partial products summed in split order (split z
//       at P + z pstride; splits 1: P is the row itself)             (sum_splits_kernel);
//   hout = (hin + y) * scale                                          (add_rows_kernel);
//   and with xn: xn = (hout * (1 / rms(hout))) * (off + w)            (rmsnorm_rows_kernel,
//   the f64 sum of squares over the same 256 threads, element i in thread i % 256, in the
//   same order) with its row statistics for the next GEMM             (gemm_row_stats).
__global__ __launch_bounds__(256) void resid_norm_stats_rows_kernel(
    const float* __restrict__ P, size_t pstride, int splits, const float* __restrict__ hin, float scale,
    float* __restrict__ hout, const float* __restrict__ w, float off, float* __restrict__ xn, int n, double eps,
    int* __restrict__ xe, float* __restrict__ xs) {
    __shared__ __align__(16) float row[kFusedRowMax];
    __shared__ double red[4];
    __shared__ float wm[4];
    const int t = threadIdx.x;
    const size_t r = static_cast<size_t>(blockIdx.x) * n;
    double ss = 0.0;
    float w0[kRowChunk];  // the norm weights of the first chunk, requested with its rows
    for (int c0 = 0; c0 < n; c0 += 256 * kRowChunk) {
        float a[kRowChunk], h[kRowChunk];
#pragma unroll
        for (int q = 0; q < kRowChunk; q++) {
            const size_t i = r + min(c0 + t + 256 * q, n - 1);
            a[q] = P[i];
            h[q] = hin[i];
        }
        if (c0 == 0) {
#pragma unroll
            for (int q = 0; q < kRowChunk; q++) w0[q] = w && xn ? w[min(t + 256 * q, n - 1)] : 0.f;
        }
        for (int z = 1; z < splits; z++) {
#pragma unroll
            for (int q = 0; q < kRowChunk; q++) a[q] += P[z * pstride + r + min(c0 + t + 256 * q, n - 1)];
        }
#pragma unroll
        for (int q = 0; q < kRowChunk; q++) {
            const int i = c0 + t + 256 * q;
            if (i < n) {
                const float hv = (h[q] + a[q]) * scale;
                hout[r + i] = hv;
                row[i] = hv;
                ss += static_cast<double>(hv) * hv;
            }
        }
    }
    if (!xn) return;  // (uniform)
    ss = wave_sum_d(ss);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / static_cast<float>(sqrt(tot / static_cast<double>(n) + eps));
    float m = 0.f;
    for (int c0 = 0; c0 < n; c0 += 256 * kRowChunk) {
        float wv[kRowChunk];
#pragma unroll
        for (int q = 0; q < kRowChunk; q++) wv[q] = c0 == 0 ? w0[q] : (w ? w[min(c0 + t + 256 * q, n - 1)] : 0.f);
#pragma unroll
        for (int q = 0; q < kRowChunk; q++) {
            const int i = c0 + t + 256 * q;
            if (i < n) {  // (the thread's own elements of `row`: no barrier needed)
                const float x = w ? (row[i] * inv) * (off + wv[q]) : row[i] * inv;
                xn[r + i] = x;
                row[i] = x;
                m = fmaxf(m, fabsf(x));
            }
        }
    }
    lds_row_stats<256>(row, n, m, wm, xe + blockIdx.x, xs ? xs + static_cast<size_t>(blockIdx.x) * (n / 32) : nullptr);
}

// Grid M rows; 1024 threads.  act = act(gate) * up over a row of n outputs from the
// gate/up row (pairs interleaved, as gated_pair_rows_kernel), with act's row statistics
// for the down GEMM.
__global__ __launch_bounds__(1024) void gated_pair_stats_rows_kernel(const float* __restrict__ GU,
                                                                     float* __restrict__ act, int n, int kind,
                                                                     int* __restrict__ xe, float* __restrict__ xs) {
    __shared__ __align__(16) float row[kFusedRowMax];
    __shared__ float wm[16];
    const int t = threadIdx.x;
    const size_t r = static_cast<size_t>(blockIdx.x) * n;
    const float2* gu = reinterpret_cast<const float2*>(GU) + r;
    float m = 0.f;
    for (int c0 = 0; c0 < n; c0 += 1024 * kRowChunk) {
        float2 v[kRowChunk];
#pragma unroll
        for (int q = 0; q < kRowChunk; q++) v[q] = gu[min(c0 + t + 1024 * q, n - 1)];
#pragma unroll
        for (int q = 0; q < kRowChunk; q++) {
            const int i = c0 + t + 1024 * q;
            if (i < n) {
                const float a = gated_act(kind, v[q].x, v[q].y);
                act[r + i] = a;
                row[i] = a;
                m = fmaxf(m, fabsf(a));
            }
        }
    }
    lds_row_stats<1024>(row, n, m, wm, xe + blockIdx.x, xs ? xs + static_cast<size_t>(blockIdx.x) * (n / 32) : nullptr);
}

unsigned blocks(size_t n) { return static_cast<unsigned>((n + 255) / 256); }

}  // namespace

void launch_rmsnorm_rows(const float* X, const float* w, float off, float* Y, size_t m, size_t n, double eps,
                         hipStream_t s) {
    if (m == 0) return;
    rmsnorm_rows_kernel<<<dim3(static_cast<unsigned>(m)), dim3(256), 0, s>>>(X, w, off, Y, static_cast<int>(n), eps);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_resid_norm_rows(const float* H, const float* V, const float* w, float off, float scale, float* out,
                            size_t m, size_t n, double eps, hipStream_t s) {
    if (m == 0) return;
    resid_norm_rows_kernel<<<dim3(static_cast<unsigned>(m)), dim3(256), 0, s>>>(H, V, w, off, scale, out,
                                                                                static_cast<int>(n), eps);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_vnorm_rows(float* X, size_t m, size_t ld, int num_heads, int hd, double eps, hipStream_t s) {
    if (m == 0 || num_heads == 0) return;
    vnorm_rows_kernel<<<dim3(static_cast<unsigned>(m), static_cast<unsigned>(num_heads)), dim3(64), 0, s>>>(
        X, static_cast<int>(ld), hd, eps);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_rope_kv_rows(const float* QKV, size_t m, size_t p0, size_t q_dim, size_t kv_dim, int hd, int rdim,
                         const float2* rope, __half* kc, __half* vc, int num_kv, hipStream_t s) {
    const size_t n = m * kv_dim;
    if (n == 0) return;
    rope_kv_rows_kernel<<<dim3(blocks(n)), dim3(256), 0, s>>>(
        QKV, static_cast<int>(m), static_cast<int>(p0), static_cast<int>(q_dim + 2 * kv_dim), static_cast<int>(q_dim),
        static_cast<int>(kv_dim), hd, rdim / 2, rope, kc, vc, num_kv);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_add_rows(const float* a, const float* b, float* out, size_t n, hipStream_t s, float scale) {
    if (n == 0) return;
    add_rows_kernel<<<dim3(blocks(n)), dim3(256), 0, s>>>(a, b, out, n, scale);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_gated_mul(const float* G, const float* U, float* act, size_t n, int kind, hipStream_t s) {
    if (n == 0) return;
    gated_mul_kernel<<<dim3(blocks(n)), dim3(256), 0, s>>>(G, U, act, n, kind);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_resid_norm_stats_rows(const float* P, size_t pstride, int splits, const float* hin, float scale,
                                  float* hout, const float* w, float off, float* xn, size_t m, size_t n, double eps,
                                  const GemmRowStats& st, hipStream_t s) {
    if (m == 0) return;
    if (splits < 1 || n % 32 != 0 || n > static_cast<size_t>(kFusedRowMax) || (xn && !st.xe))
        fail(LARQL_HIP_ERR_INVALID, "fused residual and norm rows: bad arguments");
    resid_norm_stats_rows_kernel<<<dim3(static_cast<unsigned>(m)), dim3(256), 0, s>>>(
        P, pstride, splits, hin, scale, hout, w, off, xn, static_cast<int>(n), eps, st.xe, st.xs);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_gated_pair_stats_rows(const float* GU, float* act, size_t m, size_t n, int kind, const GemmRowStats& st,
                                  hipStream_t s) {
    if (m == 0) return;
    if (n % 32 != 0 || n > static_cast<size_t>(kFusedRowMax) || !st.xe)
        fail(LARQL_HIP_ERR_INVALID, "fused gated rows: bad arguments");
    gated_pair_stats_rows_kernel<<<dim3(static_cast<unsigned>(m)), dim3(1024), 0, s>>>(GU, act, static_cast<int>(n),
                                                                                       kind, st.xe, st.xs);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_gated_pair_rows(const float* GU, float* act, size_t n, int kind, hipStream_t s) {
    if (n == 0) return;
    gated_pair_rows_kernel<<<dim3(blocks(n)), dim3(256), 0, s>>>(GU, act, n, kind);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
