// Integer-dot matvecs with the reference's exact float accumulation order.
//
//   Q4_0 x Q8 : ComputeBackend::q4_matvec (LC/src/backend.rs:49-53).  The C kernel's
//               ARM path and the Metal q4_matvec_v4 kernel form an exact int32 dot per
//               32-element block and accumulate  acc += (float)isum_b * (f16(s_b) * q8s_b)
//               over blocks in order (LC/csrc/q4_dot.c:58-89).
//   Q8_0 x Q8 : q8_matvec::dispatch (LC/src/cpu/ops/q8_matvec.rs:36-62), same structure
//               with an int8 weight block and a separate f32 weight scale.
//
// Both reproduce that order bit for bit, for 1..8 activation rows at once (the
// weights are read once for all of them):
//   * int_mv_kernel: a group of G (4 or 16) consecutive lanes owns one weight row; at
//     step s lane j holds block s*G + j, so a step reads G contiguous blocks of the
//     row, and the block products (float)isum * scale are added to the row's running
//     sum in block order by G v_add_f32 with a DPP broadcast of lane 0, 1, ..., G-1
//     (every lane of the group carries the same sum; lane 0 stores it).  Lanes of a
//     step that fall past the last block contribute +0, which leaves a sum that starts
//     at +0 unchanged.
//   * q8_mfma_kernel (Q8_0, 5..8 activation rows): the int32 block dots on the matrix
//     cores, the products and sums per lane (described at the kernel).
// Weight blocks stream through a register ring several steps deep.  The activation
// rows (int8 values, for Q4_0 re-ordered into even/odd element dwords for
// v_dot4_i32_i8 with the block's integer sum; f32 block scales) are staged in LDS
// once per workgroup.
//
// quantize_to_q8 (LC/src/cpu/ops/q4_common.rs:28-44) is reproduced bit for bit:
// IEEE division for amax/127 and 1/scale, round-half-away-from-zero, clamp.
#include <algorithm>
#include <utility>

#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

// ── activation quantizer ───────────────────────────────────────────────
// Block scale from the block's largest |x| (a fold of fmaxf from 0, which skips NaNs, so
// any order gives it), the inverse used for the codes, and one code: round half away from
// zero, clamp, NaN -> 0 (Rust's `as i8`: v * inv is NaN for a NaN v, or an infinite v in a
// block whose scale is infinite).  Shared by the quantizer and the Q4_0 matrix-core kernel
// that quantizes its own activation rows.
__device__ __forceinline__ float q8_block_scale(float amax) { return amax / 127.0f; }
__device__ __forceinline__ float q8_block_inv(float scale) { return scale > 0.0f ? 1.0f / scale : 0.0f; }
__device__ __forceinline__ int q8_code(float v, float inv) {
    const float q = roundf(v * inv);
    return isnan(q) ? 0 : static_cast<int>(fminf(fmaxf(q, -128.0f), 127.0f));
}

// 32 threads per 32-element block; 8 blocks per 256-thread workgroup.
__global__ __launch_bounds__(256) void quantize_q8_kernel(const float* __restrict__ x,
                                                          int8_t* __restrict__ q8,
                                                          float* __restrict__ scales,
                                                          size_t nblocks) {
    const size_t b = blockIdx.x * 8 + (threadIdx.x >> 5);
    const int j = threadIdx.x & 31;
    if (b >= nblocks) return;  // whole 32-lane group exits together
    const float v = x[b * 32 + j];
    float amax = fmaxf(0.0f, fabsf(v));
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    const float scale = q8_block_scale(amax);
    q8[b * 32 + j] = static_cast<int8_t>(q8_code(v, q8_block_inv(scale)));
    if (j == 0) scales[b] = scale;
}

void launch_quantize_q8(const float* x, size_t n, size_t m, int8_t* q8, float* scales, hipStream_t s) {
    const size_t nb = n / 32 * m;
    if (nb == 0) return;
    quantize_q8_kernel<<<dim3((nb + 7) / 8), dim3(256), 0, s>>>(x, q8, scales, nb);
    LARQL_HIP_CHECK(hipGetLastError());
}

// ── the kernel ─────────────────────────────────────────────────────────
#pragma clang fp contract(off)

namespace {

constexpr int kThreads = 256;

template <int C>
__device__ __forceinline__ float dpp_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), C, 0xF, 0xF, true));
}

// acc[m] + p[m](lane 0) + p[m](lane 1) + ... + p[m](lane G-1) of the lane's G-lane group,
// left to right for every m: G = 16 broadcasts with row_newbcast:J (lane J of each
// 16-lane row), G = 4 with quad_perm:[J,J,J,J].  The M sums advance together, so
// consecutive adds are independent (no read-after-write stall between them).
template <int G, int M, int J>
__device__ __forceinline__ void chain_step(float (&acc)[M], const float (&p)[M]) {
    static_assert(G == 16 || G == 4, "lane group of 4 or 16");
#pragma unroll
    for (int mi = 0; mi < M; mi++) acc[mi] = acc[mi] + dpp_bcast<G == 16 ? 0x150 + J : J * 0x55>(p[mi]);
}

template <int G, int M, int... J>
__device__ __forceinline__ void chain_add(float (&acc)[M], const float (&p)[M], std::integer_sequence<int, J...>) {
    (chain_step<G, M, J>(acc, p), ...);
}

// One raw Q8 activation block: 32 int8 values and the f32 scale.
struct XRaw {
    uint4 a, c;
    float s;
    __device__ __forceinline__ void load(const int8_t* xq, const float* xsc, int i) {
        const uint4* p = reinterpret_cast<const uint4*>(xq + static_cast<size_t>(i) * 32);
        a = p[0];
        c = p[1];
        s = xsc[i];
    }
};

template <int FMT>
struct Blk;

// Q4_0: 16 nibble bytes + the f16 scale.  LDS image per (activation row, block):
// 8 dwords (even-element, odd-element dwords) and {-8 * sum(x_q), x scale}.
template <>
struct Blk<LARQL_Q4_0> {
    uint4 q;
    uint32_t d;
    static constexpr int kXAux = 2;
    __device__ __forceinline__ void load(const uint8_t* qs, const void* dsc, int row, int b, int nb) {
        const size_t blk = static_cast<size_t>(row) * nb + b;
        q = reinterpret_cast<const uint4*>(qs)[blk];
        d = static_cast<const uint16_t*>(dsc)[blk];
    }
    __device__ __forceinline__ float product(const uint4* x0, const uint4* x1, const uint32_t* xa) const {
        const uint4 e0 = *x0;
        const uint4 e1 = *x1;
        const uint2 a = *reinterpret_cast<const uint2*>(xa);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        const uint32_t xe[4] = {e0.x, e0.y, e0.z, e0.w};
        const uint32_t xo[4] = {e1.x, e1.y, e1.z, e1.w};
        int isum = static_cast<int>(a.x);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            isum = __builtin_amdgcn_sdot4(static_cast<int>(qw[t] & 0x0F0F0F0Fu), static_cast<int>(xe[t]), isum, false);
            isum = __builtin_amdgcn_sdot4(static_cast<int>((qw[t] >> 4) & 0x0F0F0F0Fu), static_cast<int>(xo[t]), isum,
                                          false);
        }
        const float cs = h2f(d) * __uint_as_float(a.y);
        return static_cast<float>(isum) * cs;
    }
    // one x block (flat index i over [M][nb]) -> LDS image
    __device__ static void put_x(const XRaw& r, uint4* x0, uint4* x1, uint32_t* xa) {
        const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.c.x, r.c.y, r.c.z, r.c.w};
        uint32_t ev[4], od[4];
        int s = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            // nibble dword t covers elements 8t..8t+7 (byte i: elements 2i low, 2i+1 high),
            // i.e. x dwords 2t and 2t+1: even elements go with the low nibbles.
            const uint32_t e0 = w[2 * t], e1 = w[2 * t + 1];
            ev[t] = __builtin_amdgcn_perm(e1, e0, 0x06040200u);
            od[t] = __builtin_amdgcn_perm(e1, e0, 0x07050301u);
            s = __builtin_amdgcn_sdot4(static_cast<int>(e0), 0x01010101, s, false);
            s = __builtin_amdgcn_sdot4(static_cast<int>(e1), 0x01010101, s, false);
        }
        *x0 = make_uint4(ev[0], ev[1], ev[2], ev[3]);
        *x1 = make_uint4(od[0], od[1], od[2], od[3]);
        xa[0] = static_cast<uint32_t>(-8 * s);
        xa[1] = __float_as_uint(r.s);
    }
};

// Q8_0: 32 int8 + an f32 scale, tile-major (q8_piece: a 16-row tile's pieces of one
// block are 256 contiguous bytes).  LDS image: the 8 raw x dwords and the x scale.
template <>
struct Blk<LARQL_Q8_0> {
    uint4 a, c;
    float ws;
    static constexpr int kXAux = 1;
    __device__ __forceinline__ void load(const uint8_t* qs, const void* dsc, int row, int b, int nb) {
        const size_t P = q8_pairs(nb), off = q8_piece(row, b, 0, P);
        a = *reinterpret_cast<const uint4*>(qs + off);
        c = *reinterpret_cast<const uint4*>(qs + off + 256);
        ws = static_cast<const float*>(dsc)[q8_scale_index(row, b, P)];
    }
    __device__ __forceinline__ float product(const uint4* xp0, const uint4* xp1, const uint32_t* xa) const {
        const uint4 x0 = *xp0;
        const uint4 x1 = *xp1;
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
        const uint32_t x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int isum = 0;
#pragma unroll
        for (int t = 0; t < 8; t++) isum = __builtin_amdgcn_sdot4(static_cast<int>(w[t]), static_cast<int>(x[t]), isum, false);
        const float cs = ws * __uint_as_float(xa[0]);
        return static_cast<float>(isum) * cs;
    }
    __device__ static void put_x(const XRaw& r, uint4* x0, uint4* x1, uint32_t* xa) {
        *x0 = r.a;
        *x1 = r.c;
        xa[0] = __float_as_uint(r.s);
    }
};

template <int FMT>
constexpr size_t x_lds_bytes(int m, int nb) {
    return static_cast<size_t>(m) * nb * (32 + Blk<FMT>::kXAux * 4);
}

// A second weight matrix of the same shape, multiplied by the same activation rows in the
// same launch (gate and up of a walk FFN): workgroups nwg1 .. 2 nwg1 - 1 take it.
struct IntMvPair {
    const uint8_t* qs;
    const void* dsc;
    float* out;
    int nwg1;  // workgroups of the first matrix
};

// Grid: one workgroup per 256 / G rows (of each matrix).  x: m <= M activation rows of Q8
// values (cols int8 each) and their scales (nb each); out: m rows of `rows` floats.  Rows
// m..M-1 of the x image are left unset: their sums are formed and discarded.
template <int FMT, int M, int G, int D, int NT>
__device__ __forceinline__ void int_mv_body(const uint8_t* __restrict__ qs, const void* __restrict__ dsc,
                                            const int8_t* __restrict__ xq, const float* __restrict__ xsc,
                                            float* __restrict__ out, int rows, int nb, int m, int wg) {
    using B = Blk<FMT>;
    // x image: first and second 16 bytes of every block in separate arrays, so the 16
    // lanes of a group read 256 contiguous bytes (no bank conflicts)
    extern __shared__ uint4 lds4[];
    uint4* xw0 = lds4;                                             // [M][nb]
    uint4* xw1 = lds4 + M * nb;                                    // [M][nb]
    uint32_t* xa = reinterpret_cast<uint32_t*>(lds4 + 2 * M * nb);  // [M][nb][kXAux]
    const int j = threadIdx.x & (G - 1);
    const int row = wg * (NT / G) + threadIdx.x / G;
    const int rowc = min(row, rows - 1);
    const int steps = (nb + G - 1) / G;
    const int nx = m * nb;

    // x loads first (the staging wait then covers them only), kXBatch blocks per thread
    // in flight together, then the first D steps of weights, which stay in flight
    // through the staging and the barrier
    constexpr int kXBatch = (M * 128 + NT - 1) / NT;  // all of x for hidden <= 4096
    XRaw xr[kXBatch];
#pragma unroll
    for (int k = 0; k < kXBatch; k++) xr[k].load(xq, xsc, min(static_cast<int>(threadIdx.x) + k * NT, nx - 1));
    B ring[D];
#pragma unroll
    for (int u = 0; u < D; u++) ring[u].load(qs, dsc, rowc, min(u * G + j, nb - 1), nb);
#pragma unroll
    for (int k = 0; k < kXBatch; k++) {
        const int i = threadIdx.x + k * NT;
        if (i < nx) B::put_x(xr[k], xw0 + i, xw1 + i, xa + i * B::kXAux);
    }
    for (int i0 = threadIdx.x + kXBatch * NT; i0 < nx; i0 += kXBatch * NT) {
#pragma unroll
        for (int k = 0; k < kXBatch; k++) xr[k].load(xq, xsc, min(i0 + k * NT, nx - 1));
#pragma unroll
        for (int k = 0; k < kXBatch; k++) {
            const int i = i0 + k * NT;
            if (i < nx) B::put_x(xr[k], xw0 + i, xw1 + i, xa + i * B::kXAux);
        }
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int mi = 0; mi < M; mi++) acc[mi] = 0.0f;
    auto consume = [&](const B& blk, int s) __attribute__((always_inline)) {
        const int b = s * G + j;
        const int bc = min(b, nb - 1);
        float p[M];
#pragma unroll
        for (int mi = 0; mi < M; mi++) {
            const int xi = mi * nb + bc;
            p[mi] = blk.product(xw0 + xi, xw1 + xi, xa + xi * B::kXAux);
            p[mi] = b < nb ? p[mi] : 0.0f;
        }
        chain_add<G, M>(acc, p, std::make_integer_sequence<int, G>{});
    };
    int s0 = 0;
    for (; s0 + D <= steps; s0 += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            // consume, then refill the same registers (a copy of a slot whose load is
            // still in flight would wait for it)
            consume(ring[u], s0 + u);
            ring[u].load(qs, dsc, rowc, min((s0 + u + D) * G + j, nb - 1), nb);
            // keep the refills in ring order: the wait for the next step then leaves the
            // younger steps in flight
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int u = 0; u < D; u++)
        if (s0 + u < steps) consume(ring[u], s0 + u);

    if (j == 0 && row < rows) {
#pragma unroll
        for (int mi = 0; mi < M; mi++)
            if (mi < m) out[static_cast<size_t>(mi) * rows + row] = acc[mi];
    }
}

template <int FMT, int M, int G, int D, int NT>
__global__ __launch_bounds__(NT) void int_mv_kernel(const uint8_t* __restrict__ qs,
                                                          const void* __restrict__ dsc,
                                                          const int8_t* __restrict__ xq,
                                                          const float* __restrict__ xsc,
                                                          float* __restrict__ out, int rows, int nb, int m) {
    int_mv_body<FMT, M, G, D, NT>(qs, dsc, xq, xsc, out, rows, nb, m, blockIdx.x);
}

template <int FMT, int M, int G, int D, int NT>
__global__ __launch_bounds__(NT) void int_mv_pair_kernel(const uint8_t* __restrict__ qs,
                                                               const void* __restrict__ dsc,
                                                               const int8_t* __restrict__ xq,
                                                               const float* __restrict__ xsc,
                                                               float* __restrict__ out, int rows, int nb, int m,
                                                               IntMvPair second) {
    if (static_cast<int>(blockIdx.x) >= second.nwg1)  // workgroup-uniform
        int_mv_body<FMT, M, G, D, NT>(second.qs, second.dsc, xq, xsc, second.out, rows, nb, m,
                                  blockIdx.x - second.nwg1);
    else
        int_mv_body<FMT, M, G, D, NT>(qs, dsc, xq, xsc, out, rows, nb, m, blockIdx.x);
}

// ── Q8_0 x Q8 for 2..8 activation rows on the matrix cores ─────────────
// v_mfma_i32_16x16x64_i8 gives exact int32 block dots for 16 weight rows x 8
// activation rows x one block pair at once:
//   B (64 x 16): the lane with column c and k-group g (l = 16 g + c) holds weight row
//     c, bytes 16 g .. 16 g + 15 of the pair, i.e. block 2bp + g/2, half g % 2;
//   A (16 x 64): row i = 2 mi + h holds x_mi's block 2bp + h in the two k-groups of
//     that block and zeros in the other two,
// so D[2 mi + h][c] is exactly the int32 dot of block 2bp + h of weight row c with
// x_mi.  D lane l holds rows 4 g + t (t = 0..3): activation rows 2g and 2g + 1, both
// blocks of the pair, for weight row c — the lane forms the four products
// (float)isum * (ws * xs) and adds them to its two running sums in block order,
// exactly as the serial loop does.  Requires an even block count (hidden % 64 == 0).
// Weights stream through buffer loads (a prefetch past the end of the array reads 0);
// weight scales through clamped global loads.
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kMfmaMaxM = 8;
constexpr int kBufDword3 = 0x00020000;  // raw buffer descriptor word 3 (32-bit data format)

constexpr size_t mfma_lds_bytes(int nb) {
    return (static_cast<size_t>(nb) * 16 + 1) * 16 + static_cast<size_t>(nb) * 8 * 4;
}

template <int D, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void q8_mfma_kernel(const uint8_t* __restrict__ wq,
                                                              const float* __restrict__ wsc,
                                                              const int8_t* __restrict__ xq,
                                                              const float* __restrict__ xsc,
                                                              float* __restrict__ out, int rows, int nb, int m) {
    constexpr int kT = 64 * WAVES;
    extern __shared__ uint4 lds4[];
    const int npair = nb >> 1;
    const int nchunk = nb * 16;
    uint4* xl = lds4;                                           // [npair][16 A rows][2 halves], then a zero chunk
    float* xsl = reinterpret_cast<float*>(lds4 + nchunk + 1);   // [npair][8 mi][2 blocks]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int rbase = (blockIdx.x * WAVES + wave) * 16;  // one 16-row tile per wave

    // x image item j: pair j >> 5, A row i = (j >> 1) & 15 (mi = i >> 1, block 2bp + (i & 1)),
    // half j & 1 of the block; zero for mi >= m
    auto xchunk = [&](int j) __attribute__((always_inline)) {
        const int mi = min((j >> 2) & 7, m - 1);
        const int blk = 2 * (j >> 5) + ((j >> 1) & 1);
        return reinterpret_cast<const uint4*>(xq + (static_cast<size_t>(mi) * nb + blk) * 32)[j & 1];
    };
    // x scale item j: pair j >> 4, mi (j >> 1) & 7, block 2bp + (j & 1)
    auto xscale = [&](int j) __attribute__((always_inline)) {
        const int mi = min((j >> 1) & 7, m - 1);
        return xsc[static_cast<size_t>(mi) * nb + 2 * (j >> 4) + (j & 1)];
    };

    // x loads first, all in flight together (the staging wait then covers them only),
    // then the first D steps of weights
    constexpr int kXB = 2048 / kT, kSB = 1024 / kT;  // one batch covers x for hidden <= 4096
    const uint4 zero = make_uint4(0, 0, 0, 0);
    auto put_chunk = [&](int j, uint4 v) __attribute__((always_inline)) {
        if (((j >> 2) & 7) >= m) v = make_uint4(0, 0, 0, 0);
        if (j < nchunk) xl[j] = v;
    };
    auto put_scale = [&](int j, float v) __attribute__((always_inline)) {
        if (j < nb * 8) xsl[j] = ((j >> 1) & 7) < m ? v : 0.0f;
    };
    const int t0 = threadIdx.x;
    uint4 x0[kXB];
    float s0[kSB];
#pragma unroll
    for (int k = 0; k < kXB; k++) x0[k] = xchunk(min(t0 + k * kT, nchunk - 1));
#pragma unroll
    for (int k = 0; k < kSB; k++) s0[k] = xscale(min(t0 + k * kT, nb * 8 - 1));

    // tile-major weights (q8_piece): the chunk of pair bp is 1 KB, lane 16 g + c's piece at
    // 16 lane, so one load per pair reads the wave's 16 rows contiguously; tiles past the
    // last row (the workgroup's last waves) read zeros past the descriptor's end, and their
    // rows are not stored
    const uint32_t tile = static_cast<uint32_t>(rbase >> 4);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(wq), 0, static_cast<int>(static_cast<uint32_t>((rows + 15) / 16) * npair * 1024u), kBufDword3);
    const uint32_t voff_w = tile * static_cast<uint32_t>(npair) * 1024u + 16u * lane;
    const int tiles = (rows + 15) / 16;
    const float2* wsrow = reinterpret_cast<const float2*>(wsc) +
                          static_cast<size_t>(min(static_cast<int>(tile), tiles - 1)) * npair * 16 + c;
    v4i wv[D];
    float2 ws[D];
    auto refill = [&](int u, int bp) __attribute__((always_inline)) {
        wv[u] = __builtin_amdgcn_raw_buffer_load_b128(rw, voff_w + 1024u * bp, 0, 0);
        ws[u] = wsrow[static_cast<size_t>(min(bp, npair - 1)) * 16];
    };
#pragma unroll
    for (int u = 0; u < D; u++) refill(u, u);

#pragma unroll
    for (int k = 0; k < kXB; k++) put_chunk(t0 + k * kT, x0[k]);
#pragma unroll
    for (int k = 0; k < kSB; k++) put_scale(t0 + k * kT, s0[k]);
    // hidden > 4096: further batches, each loaded whole before it is stored
    for (int j0 = t0 + kXB * kT; j0 < nchunk; j0 += kXB * kT) {
        uint4 xb[kXB];
#pragma unroll
        for (int k = 0; k < kXB; k++) xb[k] = xchunk(min(j0 + k * kT, nchunk - 1));
#pragma unroll
        for (int k = 0; k < kXB; k++) put_chunk(j0 + k * kT, xb[k]);
    }
    for (int j0 = t0 + kSB * kT; j0 < nb * 8; j0 += kSB * kT) {
        float sb[kSB];
#pragma unroll
        for (int k = 0; k < kSB; k++) sb[k] = xscale(min(j0 + k * kT, nb * 8 - 1));
#pragma unroll
        for (int k = 0; k < kSB; k++) put_scale(j0 + k * kT, sb[k]);
    }
    if (threadIdx.x == 0) xl[nchunk] = zero;
    __syncthreads();

    // A operand of this lane: row c (mi = c >> 1, block half c & 1) at k-group g; the
    // k-groups of the other block of the pair read the zero chunk
    const bool a_on = (c & 1) == (g >> 1) && (c >> 1) < m;
    const uint4* abase = a_on ? xl + c * 2 + (g & 1) : xl + nchunk;
    const int astride = a_on ? 32 : 0;
    const float* xsbase = xsl + 4 * g;

    float acc[2] = {0.0f, 0.0f};
    auto dots = [&](const v4i& w, int bp, v4i& d, float4& xs4) __attribute__((always_inline)) {
        const uint4 av = abase[bp * astride];
        const v4i a = {static_cast<int>(av.x), static_cast<int>(av.y), static_cast<int>(av.z), static_cast<int>(av.w)};
        d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, w, v4i{0, 0, 0, 0}, 0, 0, 0);
        xs4 = *reinterpret_cast<const float4*>(xsbase + bp * 16);
    };
    auto chain = [&](const v4i& d, const float4& xs4, const float2& w2) __attribute__((always_inline)) {
        // d[2j + h] = block 2bp + h of activation row 2g + j
        const float p0 = static_cast<float>(d[0]) * (w2.x * xs4.x);
        const float p1 = static_cast<float>(d[1]) * (w2.y * xs4.y);
        const float p2 = static_cast<float>(d[2]) * (w2.x * xs4.z);
        const float p3 = static_cast<float>(d[3]) * (w2.y * xs4.w);
        acc[0] = acc[0] + p0;
        acc[0] = acc[0] + p1;
        acc[1] = acc[1] + p2;
        acc[1] = acc[1] + p3;
    };
    // the ring is processed in halves of DB steps: all dots of a half, then its sums,
    // then its refill, while the other half's loads are in flight
    constexpr int DB = D / 2;
    int bp0 = 0;
    for (; bp0 + D <= npair; bp0 += D) {
#pragma unroll
        for (int h = 0; h < D; h += DB) {
            v4i dd[DB];
            float4 xx[DB];
#pragma unroll
            for (int k = 0; k < DB; k++) dots(wv[h + k], bp0 + h + k, dd[k], xx[k]);
#pragma unroll
            for (int k = 0; k < DB; k++) chain(dd[k], xx[k], ws[h + k]);
#pragma unroll
            for (int k = 0; k < DB; k++) refill(h + k, bp0 + h + k + D);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int u = 0; u < D; u++)
        if (bp0 + u < npair) {
            v4i d;
            float4 xs4;
            dots(wv[u], bp0 + u, d, xs4);
            chain(d, xs4, ws[u]);
        }

    const int row = rbase + c;
    if (row < rows) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int mi = 2 * g + j;
            if (mi < m) out[static_cast<size_t>(mi) * rows + row] = acc[j];
        }
    }
}

// ── Q4_0 x Q8 on the matrix cores, 2 .. 8 activation rows ───────────────
// Same exact int32 block dots and in-order f32 accumulation as int_mv_kernel (per block b
// in order: cs = f16(d_b) * xs_b; acc += (float)isum_b * cs, LC/csrc/q4_dot.c:58-89), over
// the row-major Q4_0 layout.  One wave owns a 16-row tile and walks the row in quads of
// four blocks; per quad and group of four activation rows (TG groups), two
// v_mfma_i32_16x16x64_i8 (block halves 0 and 1, the second accumulating onto the first)
// with A row i = 4 t + j = activation row t of the group, block 4 q + j, live only in
// k-group j, and B column c = weight row c, k-group g = half of block 4 q + g.  D lane
// (g, c) then holds, in registers r = 0 .. 3, the exact int32 dots of blocks 4 q + r of
// activation row g with weight row c: four consecutive blocks of one chain, added in order
// in the lane (no cross-lane traffic).  The weights are loaded two quads at a time (below)
// so that each load instruction reads whole 128-byte lines.  The B operands are the raw
// nibble codes 0 .. 15 (one mask per byte group); the -8 offset enters as the first
// MFMA's accumulator input, -8 sum(x) of the block for each activation row, staged with
// the x image, so D is still exactly sum((code - 8) x).  The activation bytes are staged
// in LDS in the order the nibbles unpack (even elements, then odd, per 16).  Requires
// hidden % 128 == 0.  The
// weight loads are plain (cached): with one quad per load a wave read half of a 128-byte
// line of each row and the next quad the other half, which a nontemporal load fetched
// from HBM twice (pair batch [10240 x 2560] x 6: 15.4 against 19.6 us with the
// quantization launch).  W tiles per workgroup, chosen per shape
// so the busiest CU holds the fewest tiles (640 + 640 tiles on 256 CUs: five per
// workgroup, one workgroup per CU; with four, 64 CUs hold two).
constexpr int kQ40MfmaD = 4;  // quads of weights in flight per wave (2, 4, 6, 8 tried: 4 is fastest; 6 equal)

// zero chunks after the x image: the A operand reads of lanes outside their k-group land
// there (offsets up to one activation-row group + one half: 32 + 1 chunks past the base)
constexpr int kQ40Zero = 34;

constexpr size_t q40_mfma_lds_bytes(int nb) {
    return (static_cast<size_t>(nb / 4) * 64 + kQ40Zero) * 16 + static_cast<size_t>(nb / 4) * 32 * 4 * 2;
}

// keep in the lanes outside BANKS, the DPP row_ror:8 partner's `from` in those inside
template <int BANKS>
__device__ __forceinline__ uint32_t swap_half(uint32_t keep, uint32_t from) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(keep), static_cast<int>(from), 0x128, 0xF, BANKS, false));
}

template <int TG, int W>
__global__ __launch_bounds__(64 * W) void q4_0_mfma_kernel(const uint8_t* __restrict__ qs,
                                                           const uint16_t* __restrict__ dsc,
                                                           const int8_t* __restrict__ xq,
                                                           const float* __restrict__ xsc,
                                                           float* __restrict__ out, int rows, int nb, int m,
                                                           IntMvPair second) {
    constexpr int kT = 64 * W, D = kQ40MfmaD;
    extern __shared__ uint4 lds4[];
    int wg = blockIdx.x;
    if (second.nwg1 > 0 && wg >= second.nwg1) {  // workgroup-uniform: the second matrix
        qs = second.qs;
        dsc = static_cast<const uint16_t*>(second.dsc);
        out = second.out;
        wg -= second.nwg1;
    }
    const int nq = nb >> 2;
    const int nchunk = nq * 64;
    uint4* xl = lds4;  // [nq][8 t][4 j][2 h], then kQ40Zero zero chunks
    float* xsl = reinterpret_cast<float*>(lds4 + nchunk + kQ40Zero);  // [nq][8 t][4 j]
    int* xcl = reinterpret_cast<int*>(xsl + nq * 32);          // [nq][8 t][4 j]: -8 sum of the codes
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int rbase = (wg * W + wave) * 16;  // < rows_pad: the grid covers rows_pad / 16 tiles exactly

    // x image: job bj = (q, t, j) stages activation row t, block 4 q + j: chunks 2 bj + h
    // (bytes 16 h .. of its 32 codes in the unpack order, even elements of the 16, then odd)
    // and its scale xsl[bj]; zero for t >= m.  Loads return in issue order, so the x of the
    // first PX passes is requested before the weights (a pass requested after them would
    // wait an HBM round trip); any further pass loads and stages in turn.
    constexpr int PX = 2, XV = 3;  // 16-byte values per job: 32 codes + the scale
    const int njob = nq * 32;
    auto xload = [&](int bj, uint4(&v)[XV]) __attribute__((always_inline)) {
        const int q = bj >> 5, t = (bj >> 2) & 7, j = bj & 3;
        const size_t blk = static_cast<size_t>(min(t, m - 1)) * nb + 4 * q + j;
        const uint4* src = reinterpret_cast<const uint4*>(xq + blk * 32);
        v[0] = src[0];
        v[1] = src[1];
        v[2].x = __float_as_uint(xsc[blk]);
    };
    auto xstage = [&](int bj, const uint4(&v)[XV]) __attribute__((always_inline)) {
        const bool live = ((bj >> 2) & 7) < m;
        int cs = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            cs = __builtin_amdgcn_sdot4(static_cast<int>(v[h].x), 0x01010101, cs, false);
            cs = __builtin_amdgcn_sdot4(static_cast<int>(v[h].y), 0x01010101, cs, false);
            cs = __builtin_amdgcn_sdot4(static_cast<int>(v[h].z), 0x01010101, cs, false);
            cs = __builtin_amdgcn_sdot4(static_cast<int>(v[h].w), 0x01010101, cs, false);
        }
        xcl[bj] = live ? -8 * cs : 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint4 r = v[h];
            const uint4 cv = make_uint4(__builtin_amdgcn_perm(r.y, r.x, 0x06040200u), __builtin_amdgcn_perm(r.w, r.z, 0x06040200u),
                                        __builtin_amdgcn_perm(r.y, r.x, 0x07050301u), __builtin_amdgcn_perm(r.w, r.z, 0x07050301u));
            xl[2 * bj + h] = live ? cv : make_uint4(0u, 0u, 0u, 0u);
        }
        xsl[bj] = live ? __uint_as_float(v[2].x) : 0.0f;
    };
    uint4 xv[PX][XV];
#pragma unroll
    for (int p = 0; p < PX; p++)
        if (static_cast<int>(threadIdx.x) + p * kT < njob) xload(threadIdx.x + p * kT, xv[p]);

    // then the weights, two quads (2 p, 2 p + 1) at a time: lane (g, c) loads block g of
    // quad 2 p + (c >> 3) of rows c & 7 (wa) and 8 + (c & 7) (wb), so each load instruction
    // reads 128 contiguous bytes of each of 8 rows (whole cache lines when the row length is
    // a multiple of 128 bytes); one DPP rotation by 8 lanes then gives every lane both quads
    // of its own row c.  Block scales: row c's four of each quad.  Both through buffer
    // descriptors over the padded matrix (rows_pad = the tiles of the grid x 16): the pair
    // index is a uniform offset, and a load past the matrix's end (a prefetch past the last
    // pair of the last row) reads 0; past a row's end it reads the next row's bytes, never
    // used.
    constexpr int DP = D / 2;  // pairs of quads in flight
    const int np = (nq + 1) >> 1, qh = c >> 3;
    const uint32_t rows_pad = static_cast<uint32_t>(second.nwg1 > 0 ? second.nwg1 : gridDim.x) * W * 16;
    const uint32_t rowb = static_cast<uint32_t>(nb) * 16;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(qs), 0,
                                                                        static_cast<int>(rows_pad * rowb), kBufDword3);
    const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(dsc), 0, static_cast<int>(rows_pad * static_cast<uint32_t>(nb) * 2), kBufDword3);
    const uint32_t wa_off = static_cast<uint32_t>(rbase + (c & 7)) * rowb + g * 16 + qh * 64;
    const uint32_t wb_off = wa_off + 8 * rowb;
    const uint32_t s_off = static_cast<uint32_t>(rbase + c) * static_cast<uint32_t>(nb) * 2;
    uint4 wa[DP], wb[DP];
    uint2 sa[DP], sb[DP];
    // The three loads of a pair are issued in one fixed order everywhere (scheduling
    // barriers around each): the wait counts at the loop head merge the order of the loads
    // before the loop with that of the loop body, and with the prologue's loads interleaved
    // the compiler waited for the next pair's data while the current pair was computed.
    auto refill = [&](int u, int p) __attribute__((always_inline)) {
        const int po = p * 128;
        __builtin_amdgcn_sched_barrier(0);
        wa[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, wa_off, po, 0));
        __builtin_amdgcn_sched_barrier(0);
        wb[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, wb_off, po, 0));
        __builtin_amdgcn_sched_barrier(0);
        const uint4 s4 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rd, s_off, p * 16, 0));
        __builtin_amdgcn_sched_barrier(0);
        sa[u] = make_uint2(s4.x, s4.y);
        sb[u] = make_uint2(s4.z, s4.w);
    };
#pragma unroll
    for (int u = 0; u < DP; u++) refill(u, u);

#pragma unroll
    for (int p = 0; p < PX; p++)
        if (static_cast<int>(threadIdx.x) + p * kT < njob) xstage(threadIdx.x + p * kT, xv[p]);
    for (int bj = threadIdx.x + PX * kT; bj < njob; bj += kT) {
        uint4 v[XV];
        xload(bj, v);
        xstage(bj, v);
    }
    if (static_cast<int>(threadIdx.x) < kQ40Zero) xl[nchunk + threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
    __syncthreads();

    // A operand of this lane for group tg, half h: row c = 4 t + j live in k-group j only.
    // A live lane reads chunk ((q 8 + t) 4 + g) 2 + h, i.e. its base + 64 q + 32 tg + h; the
    // others read the zero chunks (stride 0), so one multiply-add per quad gives the address.
    const bool a_on = (c & 3) == g;
    const uint32_t a_base = a_on ? static_cast<uint32_t>(((c >> 2) * 4 + g) * 2) * 16u : static_cast<uint32_t>(nchunk) * 16u;
    const uint32_t a_step = a_on ? 1024u : 0u;
    auto a_of = [&](uint32_t qa, int tg, int h) __attribute__((always_inline)) {
        const uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(xl) + qa + tg * 512 + h * 16);
        return v4i{static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
    };
    float acc[TG];
#pragma unroll
    for (int tg = 0; tg < TG; tg++) acc[tg] = 0.0f;
    auto quad = [&](int q, const uint4& w, const uint2& s2) __attribute__((always_inline)) {
        const v4i b0 = {static_cast<int>(w.x & 0x0F0F0F0Fu), static_cast<int>(w.y & 0x0F0F0F0Fu),
                        static_cast<int>((w.x >> 4) & 0x0F0F0F0Fu), static_cast<int>((w.y >> 4) & 0x0F0F0F0Fu)};
        const v4i b1 = {static_cast<int>(w.z & 0x0F0F0F0Fu), static_cast<int>(w.w & 0x0F0F0F0Fu),
                        static_cast<int>((w.z >> 4) & 0x0F0F0F0Fu), static_cast<int>((w.w >> 4) & 0x0F0F0F0Fu)};
        const float wsc[4] = {h2f(s2.x), h2f(s2.x >> 16), h2f(s2.y), h2f(s2.y >> 16)};
        const uint32_t qa = a_base + static_cast<uint32_t>(q) * a_step;
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const int4 c4 = *reinterpret_cast<const int4*>(xcl + (q * 8 + 4 * tg + g) * 4);
            v4i d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_of(qa, tg, 0), b0, v4i{c4.x, c4.y, c4.z, c4.w}, 0, 0, 0);
            d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a_of(qa, tg, 1), b1, d, 0, 0, 0);
            const float4 xs4 = *reinterpret_cast<const float4*>(xsl + (q * 8 + 4 * tg + g) * 4);
            const float xs[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
#pragma unroll
            for (int r = 0; r < 4; r++) {  // blocks 4 q + r in order
                const float cs = wsc[r] * xs[r];
                const float p = static_cast<float>(d[r]) * cs;
                acc[tg] = acc[tg] + p;
            }
        }
    };
    // lane c < 8 holds (row c, quad 2 p) in wa and passes wb (row c + 8, quad 2 p) to lane
    // c + 8; lane c >= 8 holds (row c, quad 2 p + 1) in wb and passes wa (row c - 8,
    // quad 2 p + 1) to lane c - 8.  DPP row_ror:8 swaps the two halves of each 16-lane row;
    // its bank mask writes only the receiving half (lanes 0-7: banks 0-1, lanes 8-15: banks
    // 2-3), the other half keeping the old value, its own quad.
    auto pair = [&](int p, int u) __attribute__((always_inline)) {
        const uint4 a = wa[u], b = wb[u];
        const uint4 x0 = {swap_half<0xC>(a.x, b.x), swap_half<0xC>(a.y, b.y), swap_half<0xC>(a.z, b.z),
                          swap_half<0xC>(a.w, b.w)};
        const uint4 x1 = {swap_half<0x3>(b.x, a.x), swap_half<0x3>(b.y, a.y), swap_half<0x3>(b.z, a.z),
                          swap_half<0x3>(b.w, a.w)};
        quad(2 * p, x0, sa[u]);
        if (2 * p + 1 < nq) quad(2 * p + 1, x1, sb[u]);
    };
    int p0 = 0;
    for (; p0 + DP <= np; p0 += DP) {
#pragma unroll
        for (int u = 0; u < DP; u++) {
            pair(p0 + u, u);
            refill(u, p0 + u + DP);
        }
    }
#pragma unroll
    for (int u = 0; u < DP; u++)
        if (p0 + u < np) pair(p0 + u, u);

    const int row = rbase + c;
    if (row < rows) {
#pragma unroll
        for (int tg = 0; tg < TG; tg++) {
            const int t = 4 * tg + g;
            if (t < m) out[static_cast<size_t>(t) * rows + row] = acc[tg];
        }
    }
}

// Q4_0 with up to 8 activation rows (w2 / out2: a second matrix of the same shape in the
// same grid).
template <int W>
void launch_q4_0_mfma_w(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, int m, hipStream_t s,
                        const DevWeight* w2, float* out2) {
    const int nb = static_cast<int>(w.cols / 32);
    const unsigned grid1 = static_cast<unsigned>(w.rows_pad / 16 / W);
    IntMvPair second{};
    unsigned grid = grid1;
    if (w2) {
        second.qs = w2->qs;
        second.dsc = w2->d;
        second.out = out2;
        second.nwg1 = static_cast<int>(grid1);
        grid = 2 * grid1;
    }
    const size_t lds = q40_mfma_lds_bytes(nb);
    if (m <= 4)
        q4_0_mfma_kernel<1, W><<<dim3(grid), dim3(64 * W), lds, s>>>(
            w.qs, static_cast<const uint16_t*>(w.d), q8x, q8s, out, static_cast<int>(w.rows), nb, m, second);
    else
        q4_0_mfma_kernel<2, W><<<dim3(grid), dim3(64 * W), lds, s>>>(
            w.qs, static_cast<const uint16_t*>(w.d), q8x, q8s, out, static_cast<int>(w.rows), nb, m, second);
    LARQL_HIP_CHECK(hipGetLastError());
}

// m (2 .. 8) rows through the matrix-core kernel; false when the weight does not fit it
// (hidden % 128, the x image in LDS, rows padded to 64).
bool launch_q4_0_mfma(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, int m, hipStream_t s,
                      const DevWeight* w2, float* out2) {
    const int nb = static_cast<int>(w.cols / 32);
    if (m < 2 || m > 8 || nb % 4 != 0 || q40_mfma_lds_bytes(nb) > 64 * 1024 || w.rows_pad % 64 != 0 ||
        w.rows_pad * w.cols / 2 > 0x7FFFFFFF)  // buffer descriptors: byte offsets below 2^31
        return false;
    // tiles per workgroup: of those that divide the tile count (so every wave owns a tile
    // in the allocation), the one whose busiest CU holds the fewest tiles; ties to the
    // larger workgroup (fewer x images staged)
    const size_t tiles = w.rows_pad / 16, mats = w2 ? 2 : 1, cus = static_cast<size_t>(current_device_cus());
    int best = 4;
    size_t best_cost = ~size_t{0};
    for (int W : {8, 5, 4}) {
        if (tiles % W != 0) continue;
        const size_t cost = (mats * tiles / W + cus - 1) / cus * W;
        if (cost < best_cost) best = W, best_cost = cost;
    }
    switch (best) {
        case 8: launch_q4_0_mfma_w<8>(w, q8x, q8s, out, m, s, w2, out2); break;
        case 5: launch_q4_0_mfma_w<5>(w, q8x, q8s, out, m, s, w2, out2); break;
        default: launch_q4_0_mfma_w<4>(w, q8x, q8s, out, m, s, w2, out2); break;
    }
    return true;
}

template <int D, int WAVES>
void launch_q8_mfma_t(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, int m, hipStream_t s) {
    const int nb = static_cast<int>(w.cols / 32);
    const size_t rows_per_wg = 16 * WAVES;
    const size_t grid = (w.rows + rows_per_wg - 1) / rows_per_wg;
    q8_mfma_kernel<D, WAVES><<<dim3(static_cast<unsigned>(grid)), dim3(64 * WAVES), mfma_lds_bytes(nb), s>>>(
        w.qs, static_cast<const float*>(w.d), q8x, q8s, out, static_cast<int>(w.rows), nb, m);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_q8_mfma(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, int m, hipStream_t s) {
    launch_q8_mfma_t<8, 4>(w, q8x, q8s, out, m, s);
}

constexpr size_t kLdsLimit = 64 * 1024;

// w2 / out2: the optional second matrix of the same shape (one grid over both).
template <int FMT, int M, int G, int D, int NT = kThreads>
void launch_int_mv_g(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, int m, hipStream_t s,
                     const DevWeight* w2, float* out2) {
    const int nb = static_cast<int>(w.cols / 32);
    const size_t rows_per_wg = NT / G;
    const size_t grid = (w.rows + rows_per_wg - 1) / rows_per_wg;
    if (w2) {
        IntMvPair second;
        second.qs = w2->qs;
        second.dsc = w2->d;
        second.out = out2;
        second.nwg1 = static_cast<int>(grid);
        int_mv_pair_kernel<FMT, M, G, D, NT>
            <<<dim3(static_cast<unsigned>(2 * grid)), dim3(NT), x_lds_bytes<FMT>(M, nb), s>>>(
                w.qs, w.d, q8x, q8s, out, static_cast<int>(w.rows), nb, m, second);
    } else {
        int_mv_kernel<FMT, M, G, D, NT><<<dim3(static_cast<unsigned>(grid)), dim3(NT), x_lds_bytes<FMT>(M, nb), s>>>(
            w.qs, w.d, q8x, q8s, out, static_cast<int>(w.rows), nb, m);
    }
    LARQL_HIP_CHECK(hipGetLastError());
}

// Lane groups of 4 when the launch has enough 64-row workgroups to cover the chip
// (fewer DPP adds per block), else of 16 (four times the workgroups).  Measured on
// Q8_0 [14336 x 4096]: 16.1 us (G = 4) vs 17.2 us (G = 16); on Q4_0 [10240 x 2560]:
// 5.2 us (G = 16) vs 5.3 us (G = 4).
template <int FMT, int M>
void launch_int_mv(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, int m, hipStream_t s,
                   const DevWeight* w2, float* out2) {
    const size_t nmat = w2 ? 2 : 1;
    // Q4_0 always takes 16-lane groups: a step of 4 lanes reads 64 bytes of a row, half a
    // cache line (the lm-head [128256 x 4096] 78.7 -> 52 us, the pair [10240 x 2560] x 2
    // 8.9 -> 7.7 us with 16).  A Q8_0 block is 32 bytes, so 4 lanes read a whole line.
    if (FMT != LARQL_Q4_0 && nmat * (w.rows + 63) / 64 * 4 >= static_cast<size_t>(current_device_cus()) * 3) {
        // one activation row: 32 rows per 128-thread workgroup (twice the workgroups; the x
        // image each stages is small).  Q8_0 [14336 x 4096]: 13.6 us against 14.6 with 64
        // rows per 256 threads; with 4 rows the doubled staging costs more (17.3 vs 15.1 us).
        if constexpr (M == 1)
            launch_int_mv_g<FMT, M, 4, 4, 128>(w, q8x, q8s, out, m, s, w2, out2);
        else
            launch_int_mv_g<FMT, M, 4, 4>(w, q8x, q8s, out, m, s, w2, out2);
    } else
        launch_int_mv_g<FMT, M, 16, 4>(w, q8x, q8s, out, m, s, w2, out2);
}

// M activation rows in passes of up to 8 (one pass over the weights per pass): each pass
// takes the kernel with 1, 2, 4 or 8 x rows that holds the rows left, or the largest
// whose x image fits LDS.  With w2, every pass multiplies both matrices in one launch.
template <int FMT>
void launch_int_mv_batched(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, size_t m,
                           hipStream_t s, const DevWeight* w2 = nullptr, float* out2 = nullptr) {
    const int nb = static_cast<int>(w.cols / 32);
    if (x_lds_bytes<FMT>(1, nb) > kLdsLimit) fail(LARQL_HIP_ERR_UNSUPPORTED, "int matvec: hidden too large for LDS staging");
    size_t done = 0;
    while (done < m) {
        const size_t left = m - done;
        if constexpr (FMT == LARQL_Q4_0) {  // 2 .. 8 rows of a pass on the matrix cores
            const int take = static_cast<int>(std::min<size_t>(left, 8));
            if (launch_q4_0_mfma(w, q8x + done * w.cols, q8s + done * nb, out + done * w.rows, take, s, w2,
                                 w2 ? out2 + done * w.rows : nullptr)) {
                done += take;
                continue;
            }
        }
        int cap = 1;  // the largest kernel whose x image fits
        for (int c : {8, 4, 2})
            if (x_lds_bytes<FMT>(c, nb) <= kLdsLimit) { cap = c; break; }
        int kern = 1;
        while (kern < cap && static_cast<size_t>(kern) < left) kern *= 2;
        const int take = static_cast<int>(std::min<size_t>(left, kern));
        const int8_t* xq = q8x + done * w.cols;
        const float* xs = q8s + done * nb;
        float* o = out + done * w.rows;
        float* o2 = w2 ? out2 + done * w.rows : nullptr;
        switch (kern) {
            case 8: launch_int_mv<FMT, 8>(w, xq, xs, o, take, s, w2, o2); break;
            case 4: launch_int_mv<FMT, 4>(w, xq, xs, o, take, s, w2, o2); break;
            case 2: launch_int_mv<FMT, 2>(w, xq, xs, o, take, s, w2, o2); break;
            default: launch_int_mv<FMT, 1>(w, xq, xs, o, take, s, w2, o2); break;
        }
        done += take;
    }
}

}  // namespace

void launch_q4_0_matvec(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, size_t m,
                        hipStream_t s) {
    launch_int_mv_batched<LARQL_Q4_0>(w, q8x, q8s, out, m, s);
}

void launch_q4_0_matvec_pair(const DevWeight& w1, const DevWeight& w2, const int8_t* q8x, const float* q8s,
                             float* out1, float* out2, size_t m, hipStream_t s) {
    if (w1.format != LARQL_Q4_0 || w2.format != LARQL_Q4_0 || w1.rows != w2.rows || w1.cols != w2.cols)
        fail(LARQL_HIP_ERR_INVALID, "q4_0 matvec pair: two Q4_0 matrices of one shape");
    launch_int_mv_batched<LARQL_Q4_0>(w1, q8x, q8s, out1, m, s, &w2, out2);
}

// ── Q4_0 weights x f32 activation ─────────────────────────────────────────
// The reference GPU's down projection of a Q4_0 FFN (q4_f32_matvec,
// LC/src/metal/shaders/q4_f32_matvec.rs:10-38): per block, block_sum = sum over the 16
// nibble bytes of (lo - 8) x[2j] + (hi - 8) x[2j+1], then acc += block_sum * f16(scale).
// Workgroup = kQfRows rows x the whole row: wave w covers blocks 64 w .. 64 w + 63, lane l
// block 64 w + l of each of the rows, so the lane loads its 32 x values once for all
// kQfRows rows (x crosses the caches once per workgroup, not once per row: 40 KB per
// [.. x 10240] row otherwise).  The lanes' and then the waves' partial sums are added in a
// tree, an order within f32 rounding of the reference's serial one.  [2560 x 10240]: 16.5
// us with one row per wave; 10.3 / 11.8 / 10.4 / 13.2 us with 4 / 8 / 10 / 16 rows per
// workgroup.
namespace {
constexpr int kQfRows = 4;

__global__ __launch_bounds__(1024) void q4_0_f32_mv_kernel(const uint8_t* __restrict__ qs,
                                                           const uint16_t* __restrict__ d, const float* __restrict__ x,
                                                           float* __restrict__ out, int rows, int nb) {
    __shared__ float part[16][kQfRows];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int r0 = blockIdx.x * kQfRows;
    const int b = 64 * wave + lane;
    const bool on = b < nb;
    const int bc = on ? b : nb - 1;  // past the row's end: a real block, contributing 0
    float xs[32];
    {
        const float4* xb = reinterpret_cast<const float4*>(x + 32 * static_cast<size_t>(bc));
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = xb[k];
            xs[4 * k] = v.x, xs[4 * k + 1] = v.y, xs[4 * k + 2] = v.z, xs[4 * k + 3] = v.w;
        }
    }
    uint4 w[kQfRows];
    uint32_t dv[kQfRows];
#pragma unroll
    for (int r = 0; r < kQfRows; r++) {
        const size_t row = static_cast<size_t>(min(r0 + r, rows - 1));
        w[r] = reinterpret_cast<const uint4*>(qs + row * nb * 16)[bc];
        dv[r] = d[row * nb + bc];
    }
    // sum((nib - 8) x) as sum(nib x) - 8 sum(x): sum(x) once per block for all the rows,
    // then one byte conversion and one fma per weight
    float xsum = 0.f;
#pragma unroll
    for (int k = 0; k < 32; k++) xsum += xs[k];
    float acc[kQfRows];
#pragma unroll
    for (int r = 0; r < kQfRows; r++) {
        const uint32_t wd[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
        float bs = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t lo4 = wd[k] & 0x0F0F0F0Fu, hi4 = (wd[k] >> 4) & 0x0F0F0F0Fu;
            asm volatile("" : "+v"(lo4), "+v"(hi4));  // byte conversions, not field extracts
            bs = __builtin_fmaf(ubyte0(lo4), xs[8 * k + 0], bs);
            bs = __builtin_fmaf(ubyte0(hi4), xs[8 * k + 1], bs);
            bs = __builtin_fmaf(ubyte1(lo4), xs[8 * k + 2], bs);
            bs = __builtin_fmaf(ubyte1(hi4), xs[8 * k + 3], bs);
            bs = __builtin_fmaf(ubyte2(lo4), xs[8 * k + 4], bs);
            bs = __builtin_fmaf(ubyte2(hi4), xs[8 * k + 5], bs);
            bs = __builtin_fmaf(ubyte3(lo4), xs[8 * k + 6], bs);
            bs = __builtin_fmaf(ubyte3(hi4), xs[8 * k + 7], bs);
        }
        acc[r] = on ? __builtin_fmaf(-8.0f, xsum, bs) * h2f(dv[r]) : 0.f;
    }
#pragma unroll
    for (int r = 0; r < kQfRows; r++)
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) acc[r] += __shfl_xor(acc[r], off, 64);
    if (lane == 0)
#pragma unroll
        for (int r = 0; r < kQfRows; r++) part[wave][r] = acc[r];
    __syncthreads();
    if (threadIdx.x < kQfRows && r0 + static_cast<int>(threadIdx.x) < rows) {
        float v = part[0][threadIdx.x];
        for (int i = 1; i < nw; i++) v += part[i][threadIdx.x];
        out[r0 + threadIdx.x] = v;
    }
}
}  // namespace

void launch_q4_0_f32_matvec(const DevWeight& w, const float* x, float* out, hipStream_t s) {
    if (w.format != LARQL_Q4_0) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_0 f32 matvec: Q4_0 weights only");
    if (w.rows == 0) return;
    const int nb = static_cast<int>(w.cols / 32);
    if (nb > 16 * 64) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_0 f32 matvec: rows longer than 32768");
    const dim3 grid(static_cast<unsigned>((w.rows + kQfRows - 1) / kQfRows)), block(64 * ((nb + 63) / 64));
    q4_0_f32_mv_kernel<<<grid, block, 0, s>>>(w.qs, static_cast<const uint16_t*>(w.d), x, out,
                                             static_cast<int>(w.rows), nb);
    LARQL_HIP_CHECK(hipGetLastError());
}

// 1..4 activation rows: the lane-group kernel (one pass over the weights); 5..8: the
// matrix-core kernel; more: chunks of 8 (a single leftover row takes the one-row
// kernel).  Measured on Q8_0 [14336 x 4096]: M = 4 16.9 us (lane groups) vs 20.1 us
// (matrix cores); M = 8 27.1 us vs 20.1 us.
void launch_q8_matvec(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out, size_t m,
                      hipStream_t s) {
    const int nb = static_cast<int>(w.cols / 32);
    const bool mfma_ok = nb % 2 == 0 && mfma_lds_bytes(nb) <= kLdsLimit && w.rows * w.cols < (size_t{1} << 31);
    if (m <= 4 || !mfma_ok) {
        launch_int_mv_batched<LARQL_Q8_0>(w, q8x, q8s, out, m, s);
        return;
    }
    size_t done = 0;
    while (done < m) {
        const size_t take = std::min<size_t>(m - done, kMfmaMaxM);
        if (take == 1)
            launch_int_mv_batched<LARQL_Q8_0>(w, q8x + done * w.cols, q8s + done * nb, out + done * w.rows, 1, s);
        else
            launch_q8_mfma(w, q8x + done * w.cols, q8s + done * nb, out + done * w.rows, static_cast<int>(take), s);
        done += take;
    }
}

}  // namespace larql
