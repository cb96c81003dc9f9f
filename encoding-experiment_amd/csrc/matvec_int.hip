// Integer-dot matvecs with the reference's exact float accumulation order.
//
//   Q4_0 x Q8 : ComputeBackend::q4_matvec (LC/src/backend.rs:49-53).  The C kernel's
//               ARM path and the Metal q4_matvec_v4 kernel form an exact int32 dot per
//               32-element block and accumulate  acc += (float)isum_b * (f16(s_b) * q8s_b)
//               over blocks in order (LC/csrc/q4_dot.c:58-89).
//   Q8_0 x Q8 : q8_matvec::dispatch (LC/src/cpu/ops/q8_matvec.rs:36-62), same structure
//               with an int8 weight block and a separate f32 weight scale.
//
// Both kernels reproduce that order bit for bit: a tile of (row, block) pairs is
// mapped flat onto the workgroup (consecutive threads read consecutive 16/32-byte
// blocks, so a tile is one contiguous stream), each pair's product
// (float)isum * scale is written to LDS, and one thread per row then sums its
// products in block order.  The activation (int8 values, re-ordered into even/odd
// element dwords for v_dot4_i32_i8, plus its f32 block scales) is staged in LDS
// once per workgroup.
//
// quantize_to_q8 (LC/src/cpu/ops/q4_common.rs:28-44) is reproduced bit for bit:
// IEEE division for amax/127 and 1/scale, round-half-away-from-zero, clamp.
#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

// ── activation quantizer ───────────────────────────────────────────────
// 32 threads per 32-element block; 8 blocks per 256-thread workgroup.
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x,
                                                          int8_t* __restrict__ q8,
                                                          float* __restrict__ scales,
                                                          size_t nblocks) {
    const size_t b = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    if (b >= nblocks) return;  // whole 32-lane group exits together
    const float v = x[b * 32 + j];
    float amax = fabsf(v);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    const float scale = amax / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    float q = roundf(v * inv);
    q = fminf(fmaxf(q, -128.0f), 127.0f);
    q8[b * 32 + j] = static_cast<int8_t>(isnan(q) ? 0.0f : q);
    if (j == 0) scales[b] = scale;
}

void launch_quantize_q8(const float* x, size_t n, size_t m, int8_t* q8, float* scales, hipStream_t s) {
    const size_t nb = n / 32 * m;
    if (nb == 0) return;
    quantize_q8_kernel<<<dim3((nb + 7) / 8), dim3(256), 0, s>>>(x, q8, scales, nb);
    LARQL_HIP_CHECK(hipGetLastError());
}

// ── staging helpers ────────────────────────────────────────────────────
// LDS image of one Q8 activation row: per block b, 16 bytes of even-index values,
// 16 bytes of odd-index values, their integer sum, and the f32 scale.
struct Q8Lds {
    uint32_t* xe;   // [nb][4]
    uint32_t* xo;   // [nb][4]
    int* xsum;      // [nb]
    float* xs;      // [nb]
};

__device__ __forceinline__ void stage_q8_row(const int8_t* __restrict__ xq, const float* __restrict__ xsc,
                                             int nb, Q8Lds L) {
    for (int b = threadIdx.x; b < nb; b += blockDim.x) {
        const uint4* p = reinterpret_cast<const uint4*>(xq + static_cast<size_t>(b) * 32);
        const uint4 a = p[0], c = p[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        int s = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // dword t of the nibble block covers elements 8t..8t+7: bytes 2t, 2t+1 of x.
            const uint32_t e0 = w[2 * t], e1 = w[2 * t + 1];
            // even elements 8t+0,2,4,6 -> bytes 0,2 of e0 and 0,2 of e1
            const uint32_t ev = __builtin_amdgcn_perm(e1, e0, 0x06040200u);
            const uint32_t od = __builtin_amdgcn_perm(e1, e0, 0x07050301u);
            L.xe[b * 4 + t] = ev;
            L.xo[b * 4 + t] = od;
            s += __builtin_amdgcn_sdot4(static_cast<int>(e0), 0x01010101, 0, false);
            s += __builtin_amdgcn_sdot4(static_cast<int>(e1), 0x01010101, 0, false);
        }
        L.xsum[b] = s;
        L.xs[b] = xsc[b];
    }
}

// ── Q4_0 x Q8 ──────────────────────────────────────────────────────────
__global__ __launch_bounds__(256) void q4_0_matvec_kernel(const uint8_t* __restrict__ qs,
                                                          const uint16_t* __restrict__ dsc,
                                                          const int8_t* __restrict__ xq,
                                                          const float* __restrict__ xsc,
                                                          float* __restrict__ out, int rows, int cols,
                                                          int rw, int tiles) {
    extern __shared__ uint32_t lds[];
    const int nb = cols >> 5;
    Q8Lds L;
    L.xe = lds;
    L.xo = L.xe + nb * 4;
    L.xsum = reinterpret_cast<int*>(L.xo + nb * 4);
    L.xs = reinterpret_cast<float*>(L.xsum + nb);
    float* p = L.xs + nb;  // [rw][nb]
    stage_q8_row(xq, xsc, nb, L);
    __syncthreads();

    const int pairs = rw * nb;
    for (int tile = 0; tile < tiles; tile++) {
        const int row0 = (blockIdx.x * tiles + tile) * rw;
        int rl = threadIdx.x / nb;
        int b = threadIdx.x - rl * nb;
        for (int f = threadIdx.x; f < pairs; f += blockDim.x) {
            const int row = row0 + rl;
            if (row < rows) {
                const size_t blk = static_cast<size_t>(row) * nb + b;
                const uint4 q = reinterpret_cast<const uint4*>(qs)[blk];
                const float cs = h2f(dsc[blk]) * L.xs[b];
                const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                int isum = -8 * L.xsum[b];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    isum = __builtin_amdgcn_sdot4(static_cast<int>(qw[t] & 0x0F0F0F0Fu),
                                                  static_cast<int>(L.xe[b * 4 + t]), isum, false);
                    isum = __builtin_amdgcn_sdot4(static_cast<int>((qw[t] >> 4) & 0x0F0F0F0Fu),
                                                  static_cast<int>(L.xo[b * 4 + t]), isum, false);
                }
                p[f] = static_cast<float>(isum) * cs;
            }
            b += blockDim.x;
            while (b >= nb) { b -= nb; rl++; }
        }
        __syncthreads();
        for (int r = threadIdx.x; r < rw; r += blockDim.x) {
            const int row = row0 + r;
            if (row < rows) {
                float acc = 0.0f;
                const float* pr = p + r * nb;
                for (int k = 0; k < nb; k++) acc += pr[k];
                out[row] = acc;
            }
        }
        __syncthreads();
    }
}

// Rows per tile: enough tiles for ~4 workgroups per CU (the per-row block sums are
// serial, so parallelism comes from tiles), a power of two in [4, 64].  Measured on
// [10240 x 2560] Q4_0: 64 rows 15.8 us, 8 rows 7.8 us.
static int tile_rows(size_t rows) {
    const size_t want = rows / (4 * static_cast<size_t>(current_device_cus()));
    int rw = 4;
    while (rw < 64 && static_cast<size_t>(rw) * 2 <= want) rw *= 2;
    return rw;
}

void launch_q4_0_matvec(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, size_t m,
                        hipStream_t s) {
    if (m != 1) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_matvec: batch > 1 not supported");
    const int nb = static_cast<int>(w.cols / 32);
    int rw = tile_rows(w.rows);
    const size_t fixed = static_cast<size_t>(nb) * (16 + 16 + 4 + 4);
    while (rw > 1 && fixed + static_cast<size_t>(rw) * nb * 4 > 60 * 1024) rw >>= 1;
    if (fixed + static_cast<size_t>(rw) * nb * 4 > 60 * 1024)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_matvec: hidden too large for LDS staging");
    const size_t ntiles = (w.rows + rw - 1) / rw;
    const size_t target = 2048;
    const int tiles = static_cast<int>((ntiles + target - 1) / target);
    const size_t grid = (ntiles + tiles - 1) / tiles;
    const size_t shmem = fixed + static_cast<size_t>(rw) * nb * 4;
    q4_0_matvec_kernel<<<dim3(grid), dim3(256), shmem, s>>>(
        w.qs, static_cast<const uint16_t*>(w.d), q8x, q8s, out, static_cast<int>(w.rows),
        static_cast<int>(w.cols), rw, tiles);
    LARQL_HIP_CHECK(hipGetLastError());
}

// ── Q8_0 x Q8, batched over M activation rows ──────────────────────────
template <int M>
__global__ __launch_bounds__(256) void q8_matvec_kernel(const int8_t* __restrict__ wq,
                                                        const float* __restrict__ wsc,
                                                        const int8_t* __restrict__ xq,
                                                        const float* __restrict__ xsc,
                                                        float* __restrict__ out, int rows, int cols,
                                                        int rw, int tiles) {
    extern __shared__ uint32_t lds[];
    const int nb = cols >> 5;
    uint32_t* xw = lds;                                                  // [M][nb*8] raw int8 dwords
    float* xs = reinterpret_cast<float*>(xw + M * nb * 8);              // [M][nb]
    float* p = xs + M * nb;                                              // [M][rw*nb]
    for (int i = threadIdx.x; i < M * nb * 8; i += blockDim.x)
        xw[i] = reinterpret_cast<const uint32_t*>(xq)[i];
    for (int i = threadIdx.x; i < M * nb; i += blockDim.x) xs[i] = xsc[i];
    __syncthreads();

    const int pairs = rw * nb;
    for (int tile = 0; tile < tiles; tile++) {
        const int row0 = (blockIdx.x * tiles + tile) * rw;
        int rl = threadIdx.x / nb;
        int b = threadIdx.x - rl * nb;
        for (int f = threadIdx.x; f < pairs; f += blockDim.x) {
            const int row = row0 + rl;
            if (row < rows) {
                const size_t blk = static_cast<size_t>(row) * nb + b;
                const uint4* wp = reinterpret_cast<const uint4*>(wq + blk * 32);
                const uint4 a = wp[0], c = wp[1];
                const uint32_t ww[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
                const float ws = wsc[blk];
#pragma unroll
                for (int mi = 0; mi < M; mi++) {
                    const uint32_t* xr = xw + (mi * nb + b) * 8;
                    int isum = 0;
#pragma unroll
                    for (int t = 0; t < 8; t++)
                        isum = __builtin_amdgcn_sdot4(static_cast<int>(ww[t]), static_cast<int>(xr[t]), isum, false);
                    const float cs = ws * xs[mi * nb + b];
                    p[mi * pairs + f] = static_cast<float>(isum) * cs;
                }
            }
            b += blockDim.x;
            while (b >= nb) { b -= nb; rl++; }
        }
        __syncthreads();
        for (int q = threadIdx.x; q < M * rw; q += blockDim.x) {
            const int mi = q / rw;
            const int r = q - mi * rw;
            const int row = row0 + r;
            if (row < rows) {
                float acc = 0.0f;
                const float* pr = p + mi * pairs + r * nb;
                for (int k = 0; k < nb; k++) acc += pr[k];
                out[static_cast<size_t>(mi) * rows + row] = acc;
            }
        }
        __syncthreads();
    }
}

void launch_q8_matvec(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, size_t m,
                      hipStream_t s) {
    const int nb = static_cast<int>(w.cols / 32);
    auto go = [&](auto mtag) {
        constexpr int M = decltype(mtag)::value;
        const size_t fixed = static_cast<size_t>(M) * nb * (32 + 4);
        int rw = tile_rows(w.rows);
        while (rw > 1 && fixed + static_cast<size_t>(M) * rw * nb * 4 > 64 * 1024) rw >>= 1;
        if (fixed + static_cast<size_t>(M) * rw * nb * 4 > 64 * 1024)
            fail(LARQL_HIP_ERR_UNSUPPORTED, "q8_matvec: hidden too large for LDS staging");
        const size_t ntiles = (w.rows + rw - 1) / rw;
        const size_t target = 2048;
        const int tiles = static_cast<int>((ntiles + target - 1) / target);
        const size_t grid = (ntiles + tiles - 1) / tiles;
        const size_t shmem = fixed + static_cast<size_t>(M) * rw * nb * 4;
        q8_matvec_kernel<M><<<dim3(grid), dim3(256), shmem, s>>>(
            reinterpret_cast<const int8_t*>(w.qs), static_cast<const float*>(w.d), q8x, q8s, out,
            static_cast<int>(w.rows), static_cast<int>(w.cols), rw, tiles);
    };
    switch (m) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        case 8: go(std::integral_constant<int, 8>{}); break;
        default: {
            // Arbitrary M: run in chunks of 8/4/2/1 rows of activations.
            size_t done = 0;
            while (done < m) {
                size_t left = m - done, take = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
                launch_q8_matvec(w, q8x + done * w.cols, q8s + done * nb, out + done * w.rows, take, s);
                done += take;
            }
            return;
        }
    }
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
