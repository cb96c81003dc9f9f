// Quantized prefill: Y[M x N] = X[M x K] . deq(W)^T for a Q4_K weight W [N x K],
// M tokens at once (M = 512 in the prefill workload).
//
// Reference semantics: the trait's prefill (LC/src/backend.rs:143-152) runs, per token,
// the Q4_K matvec (LC/src/cpu/ops/q4k_matvec.rs:31-90; the Metal prefill is that matvec
// in a loop over positions, LC/src/metal/prefill.rs:21-110).  Here the M matvecs are one
// GEMM on the matrix cores, v_mfma_f32_16x16x32_f16 with f32 accumulation:
//   * x16_pack_kernel converts X to fp16 once, laid out as ready-made A operands:
//     one 1 KB block (64 lanes x 8 halves) per (16 tokens, super-block, half, step);
//   * the GEMM streams the tile-major Q4_K weights (one coalesced 1 KB load per 16 rows
//     and half super-block) and dequantizes them in registers into B operands,
//     w = (1024 + q) * (d sc_j) - (1024 d sc_j + dmin m_j) in one f32 fma per element,
//     rounded to fp16 (the same value as d sc_j q - dmin m_j, to ~2^-14 d sc_j);
//   * the A blocks of a workgroup's 64 tokens go through LDS, double-buffered, and are
//     shared by its four waves; each wave owns 80 weight rows.
// The MFMA k order within a step is free as long as A and B agree: lane (g, c) of step s
// in half h supplies elements 8s + {0,4,1,5,2,6,3,7} of sub-block 4h + g (the order in
// which the nibble bytes unpack), and x16_pack_kernel writes X in that order.
// fp16 operands carry 11 significant bits: over K = 2560 random terms the error is
// ~1e-4 of max|Y|, inside the 1e-3 bar.
#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kMt = 4;                 // 16-token tiles per workgroup (64 tokens)
constexpr int kNT = 5;                 // 16-row weight tiles per wave (80 rows)
constexpr int kWaves = 4;              // waves per workgroup, side by side along N
constexpr int kThreads = 64 * kWaves;
constexpr int kNwg = 16 * kNT * kWaves;  // 320 weight rows per workgroup
constexpr int kXUnit = kMt * 4 * 64;     // uint4 of A operands per unit (16 KB)

// X [M x K] f32 -> XP[mt][sb][h][s][lane] (uint4 = 8 halves); rows >= M are zeros.
// Workgroup (sb, mt): the 16 x 256 block of X, read row-major into LDS, written out as
// its 512 operand uint4 in order.
__global__ __launch_bounds__(256) void x16_pack_kernel(const float* __restrict__ X, v4u* __restrict__ XP, int M,
                                                       int K) {
    __shared__ float xs[16][256 + 4];
    const int sb = blockIdx.x, S = gridDim.x, mt = blockIdx.y, tid = threadIdx.x;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int idx = tid + 256 * r, row = idx >> 6, c4 = idx & 63;
        const size_t m = static_cast<size_t>(mt) * 16 + row;
        const float4 v = m < static_cast<size_t>(M)
                             ? *reinterpret_cast<const float4*>(X + m * K + 256 * sb + 4 * c4)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(&xs[row][4 * c4]) = v;
    }
    __syncthreads();
    auto pk = [](float lo, float hi) __attribute__((always_inline)) {
        return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(lo))) |
               (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(hi))) << 16);
    };
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int t = tid + 256 * q, h = t >> 8, s = (t >> 6) & 3, lane = t & 63;
        const int g = lane >> 4, i = lane & 15;
        const float* p = &xs[i][32 * (4 * h + g) + 8 * s];
        const float4 a = *reinterpret_cast<const float4*>(p);
        const float4 b = *reinterpret_cast<const float4*>(p + 4);
        // element order 0, 4, 1, 5, 2, 6, 3, 7
        const v4u out = {pk(a.x, b.x), pk(a.y, b.y), pk(a.z, b.z), pk(a.w, b.w)};
        XP[(static_cast<size_t>(mt) * S + sb) * 512 + t] = out;
    }
}

// Two weights from a dword holding two fp16 values v: (v * sc + c) in f32, each rounded
// to fp16 (v_fma_mix, fp16 source operand with f32 scale and offset).
__device__ __forceinline__ uint32_t mix2(uint32_t p, float sc, float c) {
    uint32_t r;
    asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=&v"(r) : "v"(p), "v"(sc), "v"(c));
    asm("v_fma_mixhi_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(r) : "v"(p), "v"(sc), "v"(c));
    return r;
}

// (m & x) | magic for a magic with no bits under m.
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t x, uint32_t magic) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(x), "s"(magic));
    return r;
}

// Scale and offsets of one sub-block for the two nibble positions of a byte: the low
// nibble q becomes the fp16 1024 + q, the high nibble (left in place) 1024 + 16 q, so
//   w = (1024 + q) sc - (1024 sc + mn) = (1024 + 16 q) (sc / 16) - (64 sc + mn).
struct SubScale {
    float sc, c_lo, sc16, c_hi;
};

// Eight weights (elements 8s + 0, 4, 1, 5, 2, 6, 3, 7) from the nibble dword of step s;
// byte i holds elements 2i (low nibble) and 2i + 1 (high nibble).
__device__ __forceinline__ half8 deq8(uint32_t u, const SubScale& k, uint32_t m_lo, uint32_t m_hi) {
    constexpr uint32_t kMagic = 0x64006400u;  // fp16 1024 in both halves
    const uint32_t u8 = u >> 8;
    v4u r;
    r.x = mix2(bfi(m_lo, u, kMagic), k.sc, k.c_lo);     // elements 0, 4
    r.y = mix2(bfi(m_hi, u, kMagic), k.sc16, k.c_hi);   // 1, 5
    r.z = mix2(bfi(m_lo, u8, kMagic), k.sc, k.c_lo);    // 2, 6
    r.w = mix2(bfi(m_hi, u8, kMagic), k.sc16, k.c_hi);  // 3, 7
    return __builtin_bit_cast(half8, r);
}

// Grid (ceil(N / 320), ceil(M / 64)): workgroups that share weight rows are 8 apart in
// launch order when gridDim.x is a multiple of 8, i.e. on one XCD.  One wave per SIMD
// (the accumulators, three units of staged weights and the operands take ~410 registers).
__global__ __launch_bounds__(kThreads) void q4k_gemm_kernel(const uint8_t* __restrict__ qs,
                                                            const v4u* __restrict__ hdr,
                                                            const v4u* __restrict__ XP, float* __restrict__ Y,
                                                            int M, int N, int K, int ntiles) {
    __shared__ v4u As[3 * kXUnit];  // A operands of three units
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int S = K / 256;
    const int n = 2 * S;  // units: (super-block u / 2, half u % 2)
    const int mt0 = blockIdx.y * kMt;
    const int nt0 = (blockIdx.x * kWaves + wave) * kNT;  // first 16-row weight tile of this wave

    // wave-uniform byte offsets of tile j's qs block (sb 0, half 0) and header block;
    // the lane adds its 16-byte slot (qs) or header row c
    uint32_t qo[kNT], ho[kNT];
#pragma unroll
    for (int j = 0; j < kNT; j++) {
        const uint32_t t = static_cast<uint32_t>(min(nt0 + j, ntiles - 1));
        qo[j] = __builtin_amdgcn_readfirstlane(t * S * 2048u);
        ho[j] = __builtin_amdgcn_readfirstlane(t * S * 256u);
    }
    const v4u* xb = XP + static_cast<size_t>(mt0) * S * 512 + tid;

    // A: 1024 uint4 per unit, four per thread: idx = tid + 256 r -> (tile r, step, lane)
    struct Xu {
        v4u v[4];
    };
    auto load_x = [&](int u, Xu& x) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 4; r++) x.v[r] = xb[static_cast<size_t>(r) * S * 512 + u * 256];
    };
    auto store_x = [&](int b, const Xu& x) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < 4; r++) As[b * kXUnit + r * 256 + tid] = x.v[r];
    };
    // nibbles and super-block header of the unit (the half's scale word is chosen when
    // the unit is consumed: selecting at load time would wait for the load)
    struct Wu {
        v4u q[kNT], hd[kNT];
    };
    const uint8_t* hdrb = reinterpret_cast<const uint8_t*>(hdr) + c * 16;
    auto load_w = [&](int u, Wu& w) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            w.q[j] = __builtin_nontemporal_load(
                reinterpret_cast<const v4u*>(qs + qo[j] + static_cast<uint32_t>(u) * 1024u) + lane);
            w.hd[j] = *reinterpret_cast<const v4u*>(hdrb + ho[j] + static_cast<uint32_t>(u >> 1) * 256u);
        }
    };

    floatx4 acc[kMt][kNT];
#pragma unroll
    for (int i = 0; i < kMt; i++)
#pragma unroll
        for (int j = 0; j < kNT; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u;
    asm volatile("" : "+v"(m_lo), "+v"(m_hi));  // keep the masks in VGPRs
    auto compute = [&](int b, int u, const Wu& w) __attribute__((always_inline)) {
        const int h = u & 1;
        SubScale k[kNT];
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const float d = h2f(w.hd[j].x & 0xFFFFu), dmin = h2f(w.hd[j].x >> 16);
            const uint32_t scw = h ? w.hd[j].z : w.hd[j].y;
            const float sc = d * static_cast<float>((scw >> (8 * g)) & 0x3Fu);
            const float mn = dmin * static_cast<float>((w.hd[j].w >> (8 * g + 4 * h)) & 0xFu);
            k[j].sc = sc;
            k[j].c_lo = -__builtin_fmaf(1024.f, sc, mn);
            k[j].sc16 = sc * 0.0625f;
            k[j].c_hi = -__builtin_fmaf(64.f, sc, mn);
        }
        const v4u* Ab = As + b * kXUnit;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            half8 bq[kNT], aq[kMt];
#pragma unroll
            for (int j = 0; j < kNT; j++) bq[j] = deq8(w.q[j][s], k[j], m_lo, m_hi);
#pragma unroll
            for (int i = 0; i < kMt; i++) aq[i] = __builtin_bit_cast(half8, Ab[(i * 4 + s) * 64 + lane]);
#pragma unroll
            for (int i = 0; i < kMt; i++)
#pragma unroll
                for (int j = 0; j < kNT; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[i], bq[j], acc[i][j], 0, 0, 0);
        }
    };

    // Three-stage ring: unit u uses LDS buffer u % 3 and register sets u % 3.  After unit
    // u is consumed, X of unit u + 1 goes to LDS and X and W of unit u + 3 are requested,
    // so every load has two units of compute to arrive.  Loads past the last unit re-read
    // it (unused), keeping the count of loads in flight the same in every stage.
    Wu w0, w1, w2;
    Xu x0, x1, x2;
    load_x(0, x0);
    load_w(0, w0);
    load_x(min(1, n - 1), x1);
    load_w(min(1, n - 1), w1);
    load_x(min(2, n - 1), x2);
    load_w(min(2, n - 1), w2);
    store_x(0, x0);
    __syncthreads();
    auto stage = [&](int u, int b, Wu& w, Xu& xnext, Xu& xload) __attribute__((always_inline)) {
        compute(b, u, w);
        store_x(b == 2 ? 0 : b + 1, xnext);
        load_x(min(u + 3, n - 1), xload);
        load_w(min(u + 3, n - 1), w);
        __syncthreads();
    };
    int u = 0;
    for (; u + 3 <= n; u += 3) {
        stage(u, 0, w0, x1, x0);
        stage(u + 1, 1, w1, x2, x1);
        stage(u + 2, 2, w2, x0, x2);
    }
    if (u < n) stage(u, 0, w0, x1, x0);
    if (u + 1 < n) stage(u + 1, 1, w1, x2, x1);

    // D lane (g, c) holds rows 4g .. 4g + 3 of column c of each 16 x 16 tile
#pragma unroll
    for (int i = 0; i < kMt; i++)
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const int col = (nt0 + j) * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = (mt0 + i) * 16 + 4 * g + r;
                if (m < M && col < N) Y[static_cast<size_t>(m) * N + col] = acc[i][j][r];
            }
        }
}

// ── f32 operands: the accurate variant for chains of projections ────────
// Same tiling (64 tokens x 320 weight rows per workgroup, 80 rows per wave), with
// v_mfma_f32_16x16x4f32: weights dequantized to f32 (`fma(q, d sc_j, -dmin m_j)`, one
// rounding) and X read in f32, so each product is exact and the error is the f32
// accumulation's (~1e-6) instead of the fp16 operands' (~1e-4 per projection), which
// compounds through a model's layers.  A k-step of 4 takes element e of the lane's
// sub-block 4h + g for lane group g, so a lane's 16 nibble bytes feed 32 steps and its A
// operands are the matching 32 consecutive elements of its token's row of X.
constexpr int kF32Pitch = 36;  // floats per lane slot in LDS (32 + 4: spread the banks)

__global__ __launch_bounds__(kThreads) void q4k_gemm_f32_kernel(const uint8_t* __restrict__ qs,
                                                                const v4u* __restrict__ hdr,
                                                                const float* __restrict__ X, float* __restrict__ Y,
                                                                int M, int N, int K, int ntiles, int sb_per, int ldy) {
    __shared__ float As[2][kMt][64][kF32Pitch];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int S = K / 256;
    const int mt0 = blockIdx.y * kMt;
    const int nt0 = (blockIdx.x * kWaves + wave) * kNT;
    // split blockIdx.z of K: super-blocks [z sb_per, (z + 1) sb_per), partial sums to Y[z]
    // (rows ldy apart; the dense partials of a split launch have ldy = N)
    const int u0 = 2 * static_cast<int>(blockIdx.z) * sb_per, u1 = min(2 * S, u0 + 2 * sb_per), last = u1 - 1;
    Y += static_cast<size_t>(blockIdx.z) * M * ldy;
    uint32_t qo[kNT], ho[kNT];
#pragma unroll
    for (int j = 0; j < kNT; j++) {
        const uint32_t t = static_cast<uint32_t>(min(nt0 + j, ntiles - 1));
        qo[j] = __builtin_amdgcn_readfirstlane(t * S * 2048u);
        ho[j] = __builtin_amdgcn_readfirstlane(t * S * 256u);
    }
    // X staging: thread (tile r = tid / 64, slot l = tid % 64) loads token 16 (mt0 + r) + l % 16,
    // elements 32 (4h + l / 16) .. + 31 of super-block sb; zeros for tokens past M.
    const int xr_row = (mt0 + (tid >> 6)) * 16 + (lane & 15);
    const bool xr_ok = xr_row < M;  // (the select also keeps the compiler from a stack copy of Xu)
    const float* xrow = X + static_cast<size_t>(min(xr_row, M - 1)) * K + 32 * g;
    struct Xu {
        float4 v[8];
    };
    auto load_x = [&](int u, Xu& x) __attribute__((always_inline)) {
        const float4* p = reinterpret_cast<const float4*>(xrow + 256 * (u >> 1) + 128 * (u & 1));
#pragma unroll
        for (int k = 0; k < 8; k++) x.v[k] = xr_ok ? p[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto store_x = [&](int b, const Xu& x) __attribute__((always_inline)) {
        float4* d = reinterpret_cast<float4*>(&As[b][tid >> 6][lane][0]);
#pragma unroll
        for (int k = 0; k < 8; k++) d[k] = x.v[k];
    };
    struct Wu {
        v4u q[kNT], hd[kNT];
    };
    const uint8_t* hdrb = reinterpret_cast<const uint8_t*>(hdr) + c * 16;
    auto load_w = [&](int u, Wu& w) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            w.q[j] = __builtin_nontemporal_load(
                reinterpret_cast<const v4u*>(qs + qo[j] + static_cast<uint32_t>(u) * 1024u) + lane);
            w.hd[j] = *reinterpret_cast<const v4u*>(hdrb + ho[j] + static_cast<uint32_t>(u >> 1) * 256u);
        }
    };
    floatx4 acc[kMt][kNT];
#pragma unroll
    for (int i = 0; i < kMt; i++)
#pragma unroll
        for (int j = 0; j < kNT; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int b, int u, const Wu& w) __attribute__((always_inline)) {
        const int h = u & 1;
        float sc[kNT], nmn[kNT];
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const float d = h2f(w.hd[j].x & 0xFFFFu), dmin = h2f(w.hd[j].x >> 16);
            const uint32_t scw = h ? w.hd[j].z : w.hd[j].y;
            sc[j] = d * static_cast<float>((scw >> (8 * g)) & 0x3Fu);
            nmn[j] = -(dmin * static_cast<float>((w.hd[j].w >> (8 * g + 4 * h)) & 0xFu));
        }
#pragma unroll
        for (int e4 = 0; e4 < 8; e4++) {  // elements 4 e4 .. 4 e4 + 3 of the lane's sub-block
            float4 a[kMt];
#pragma unroll
            for (int i = 0; i < kMt; i++) a[i] = *reinterpret_cast<const float4*>(&As[b][i][lane][4 * e4]);
#pragma unroll
            for (int j = 0; j < kNT; j++) {
                // byte i of the 16 holds element 2i (low nibble) and 2i + 1 (high): split into
                // low and high nibble bytes once per dword, then one byte convert per weight
                const uint32_t word = w.q[j][e4 >> 1];
                uint32_t lo = word & 0x0F0F0F0Fu, hi = (word >> 4) & 0x0F0F0F0Fu;
                asm("" : "+v"(lo), "+v"(hi));  // opaque: keeps v_cvt_f32_ubyteN, not bfe + convert
                const int b0 = 16 * (e4 & 1);
                float wt[4];
                wt[0] = __builtin_fmaf(static_cast<float>((lo >> b0) & 0xFFu), sc[j], nmn[j]);
                wt[1] = __builtin_fmaf(static_cast<float>((hi >> b0) & 0xFFu), sc[j], nmn[j]);
                wt[2] = __builtin_fmaf(static_cast<float>((lo >> (b0 + 8)) & 0xFFu), sc[j], nmn[j]);
                wt[3] = __builtin_fmaf(static_cast<float>((hi >> (b0 + 8)) & 0xFFu), sc[j], nmn[j]);
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < kMt; i++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][t], wt[t], acc[i][j], 0, 0, 0);
            }
        }
    };

    // two-unit ring: unit u in LDS buffer u % 2; X and W of unit u + 1 in flight meanwhile
    Wu w0, w1;
    Xu x0, x1;
    // (u1 - u0 is even: the range is whole super-blocks)
    load_x(u0, x0);
    load_w(u0, w0);
    load_x(u0 + 1, x1);
    load_w(u0 + 1, w1);
    store_x(0, x0);
    __syncthreads();
    for (int u = u0; u < u1; u += 2) {
        store_x(1, x1);
        load_x(min(u + 2, last), x0);
        compute(0, u, w0);
        load_w(min(u + 2, last), w0);
        __syncthreads();
        store_x(0, x0);
        load_x(min(u + 3, last), x1);
        compute(1, u + 1, w1);
        load_w(min(u + 3, last), w1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kMt; i++)
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const int col = (nt0 + j) * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = (mt0 + i) * 16 + 4 * g + r;
                if (m < M && col < N) Y[static_cast<size_t>(m) * ldy + col] = acc[i][j][r];
            }
        }
}

// Q6_K weights (ql nibble of element e at byte e / 2, its two high bits regrouped per
// 16-element group G: element 16 G + 8 w + 2 j + p at bits 8 j + 4 w + 2 p of word G; int8
// scale per group; f16 d per block) with the f32 kernel's X staging and tiling: lane (g, c)
// of unit (sb, h) takes elements 32 (4h + g) .. + 31 of row c of each tile, i.e. 16 ql
// bytes, two high-bit words and two scales; w = fma(q, d sc, -32 d sc) = d sc (q - 32).
__global__ __launch_bounds__(kThreads) void q6k_gemm_f32_kernel(const uint8_t* __restrict__ ql,
                                                                const uint8_t* __restrict__ qh,
                                                                const int8_t* __restrict__ scl,
                                                                const uint16_t* __restrict__ dd,
                                                                const float* __restrict__ X, float* __restrict__ Y,
                                                                int M, int N, int K, int sb_per, int ldy) {
    __shared__ float As[2][kMt][64][kF32Pitch];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int S = K / 256;
    const int mt0 = blockIdx.y * kMt;
    const int nt0 = (blockIdx.x * kWaves + wave) * kNT;
    const int u0 = 2 * static_cast<int>(blockIdx.z) * sb_per, u1 = min(2 * S, u0 + 2 * sb_per), last = u1 - 1;
    Y += static_cast<size_t>(blockIdx.z) * M * ldy;
    size_t blk[kNT];  // first block of the lane's row in tile j (rows past N re-read row N - 1)
#pragma unroll
    for (int j = 0; j < kNT; j++) blk[j] = static_cast<size_t>(min((nt0 + j) * 16 + c, N - 1)) * S;
    const int xr_row = (mt0 + (tid >> 6)) * 16 + (lane & 15);
    const bool xr_ok = xr_row < M;
    const float* xrow = X + static_cast<size_t>(min(xr_row, M - 1)) * K + 32 * g;
    struct Xu {
        float4 v[8];
    };
    auto load_x = [&](int u, Xu& x) __attribute__((always_inline)) {
        const float4* p = reinterpret_cast<const float4*>(xrow + 256 * (u >> 1) + 128 * (u & 1));
#pragma unroll
        for (int k = 0; k < 8; k++) x.v[k] = xr_ok ? p[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto store_x = [&](int b, const Xu& x) __attribute__((always_inline)) {
        float4* d = reinterpret_cast<float4*>(&As[b][tid >> 6][lane][0]);
#pragma unroll
        for (int k = 0; k < 8; k++) d[k] = x.v[k];
    };
    struct Wu {
        v4u l[kNT];
        uint2 h[kNT];
        uint32_t sd[kNT];  // scales of groups G0, G0 + 1 | d << 16
    };
    auto load_w = [&](int u, Wu& w) __attribute__((always_inline)) {
        const int G0 = 8 * (u & 1) + 2 * g;
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const size_t o = blk[j] + (u >> 1);
            w.l[j] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(ql + o * 128 + 64 * (u & 1) + 16 * g));
            w.h[j] = *reinterpret_cast<const uint2*>(qh + o * 64 + 4 * G0);
            w.sd[j] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(scl + o * 16 + G0)) |
                      (static_cast<uint32_t>(dd[o]) << 16);
        }
    };
    floatx4 acc[kMt][kNT];
#pragma unroll
    for (int i = 0; i < kMt; i++)
#pragma unroll
        for (int j = 0; j < kNT; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int b, const Wu& w) __attribute__((always_inline)) {
        float ds[kNT][2];
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const float d = h2f(w.sd[j] >> 16);
            ds[j][0] = d * static_cast<float>(static_cast<int8_t>(w.sd[j] & 0xFFu));
            ds[j][1] = d * static_cast<float>(static_cast<int8_t>((w.sd[j] >> 8) & 0xFFu));
        }
#pragma unroll
        for (int e4 = 0; e4 < 8; e4++) {  // elements 4 e4 .. 4 e4 + 3 of the lane's 32
            float4 a[kMt];
#pragma unroll
            for (int i = 0; i < kMt; i++) a[i] = *reinterpret_cast<const float4*>(&As[b][i][lane][4 * e4]);
#pragma unroll
            for (int j = 0; j < kNT; j++) {
                const float sc = ds[j][e4 >> 2], nb = -32.f * sc;
                const uint32_t lo = w.l[j][e4 >> 1], hi = (e4 >> 2) ? w.h[j].y : w.h[j].x;
                float wt[4];
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const uint32_t q4 = (lo >> (16 * (e4 & 1) + 4 * t)) & 0xFu;
                    const uint32_t q2 =
                        (hi >> (16 * (e4 & 1) + 8 * (t >> 1) + 4 * ((e4 >> 1) & 1) + 2 * (t & 1))) & 3u;
                    wt[t] = __builtin_fmaf(static_cast<float>(q4 | (q2 << 4)), sc, nb);
                }
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int i = 0; i < kMt; i++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i][t], wt[t], acc[i][j], 0, 0, 0);
            }
        }
    };

    Wu w0, w1;
    Xu x0, x1;
    load_x(u0, x0);
    load_w(u0, w0);
    load_x(u0 + 1, x1);
    load_w(u0 + 1, w1);
    store_x(0, x0);
    __syncthreads();
    for (int u = u0; u < u1; u += 2) {
        store_x(1, x1);
        load_x(min(u + 2, last), x0);
        compute(0, w0);
        load_w(min(u + 2, last), w0);
        __syncthreads();
        store_x(0, x0);
        load_x(min(u + 3, last), x1);
        compute(1, w1);
        load_w(min(u + 3, last), w1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kMt; i++)
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const int col = (nt0 + j) * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = (mt0 + i) * 16 + 4 * g + r;
                if (m < M && col < N) Y[static_cast<size_t>(m) * ldy + col] = acc[i][j][r];
            }
        }
}

// Y = sum over the splits of the partial products, in split order (deterministic).
__global__ void sum_splits_kernel(const float* __restrict__ P, float* __restrict__ Y, size_t n, int splits, int N,
                                  int ldy) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i >= n) return;
    float a = P[i];
    for (int z = 1; z < splits; z++) a += P[z * n + i];
    Y[(i / N) * ldy + i % N] = a;
}

// K-splits for the f32 GEMM: the count (1..4, whole super-blocks each) that minimises
// rounds of workgroups over the CUs x units per workgroup (one workgroup per CU at a time).
struct F32Split {
    int splits, sb_per;
};
F32Split f32_split(const DevWeight& w, size_t m) {
    const int S = static_cast<int>(w.cols / 256);
    const long wgs = static_cast<long>((w.rows + kNwg - 1) / kNwg) * static_cast<long>((m + 16 * kMt - 1) / (16 * kMt));
    const long cus = current_device_cus();
    F32Split best{1, S};
    long best_cost = -1;
    for (int s = 1; s <= 4 && s <= S; s++) {
        const int per = (S + s - 1) / s, eff = (S + per - 1) / per;
        const long cost = ((wgs * eff + cus - 1) / cus) * per;
        if (best_cost < 0 || cost < best_cost) best = {eff, per}, best_cost = cost;
    }
    return best;
}

}  // namespace

size_t q4k_gemm_f32_part_floats(const DevWeight& w, size_t m) {
    const F32Split sp = f32_split(w, m);
    return sp.splits > 1 ? sp.splits * m * w.rows : 0;
}

void launch_q4k_gemm_f32(const DevWeight& w, const float* X, float* Y, size_t m, float* part, size_t part_floats,
                         hipStream_t s, size_t ldy) {
    if (ldy == 0) ldy = w.rows;
    if (ldy < w.rows || ldy > 0x7FFFFFFF) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: bad output row stride");
    if (w.format != LARQL_Q4_K && w.format != LARQL_Q6_K)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "prefill GEMM: Q4_K or Q6_K weights only");
    if (m == 0) return;
    if (m > 0x7FFFFFFF / w.cols) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: too many tokens");
    F32Split sp = f32_split(w, m);
    if (sp.splits > 1 && (!part || part_floats < sp.splits * m * w.rows)) sp = {1, static_cast<int>(w.cols / 256)};
    const dim3 grid(static_cast<unsigned>((w.rows + kNwg - 1) / kNwg),
                    static_cast<unsigned>((m + 16 * kMt - 1) / (16 * kMt)), static_cast<unsigned>(sp.splits));
    const int ld_out = static_cast<int>(sp.splits > 1 ? w.rows : ldy);
    if (w.format == LARQL_Q4_K)
        q4k_gemm_f32_kernel<<<grid, dim3(kThreads), 0, s>>>(
            w.qs, reinterpret_cast<const v4u*>(w.hdr), X, sp.splits > 1 ? part : Y, static_cast<int>(m),
            static_cast<int>(w.rows), static_cast<int>(w.cols), static_cast<int>(w.rows_pad / 16), sp.sb_per, ld_out);
    else
        q6k_gemm_f32_kernel<<<grid, dim3(kThreads), 0, s>>>(
            w.qs, w.qh, w.sc, static_cast<const uint16_t*>(w.d), X, sp.splits > 1 ? part : Y, static_cast<int>(m),
            static_cast<int>(w.rows), static_cast<int>(w.cols), sp.sb_per, ld_out);
    LARQL_HIP_CHECK(hipGetLastError());
    if (sp.splits > 1) {
        const size_t n = m * w.rows;
        sum_splits_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s>>>(
            part, Y, n, sp.splits, static_cast<int>(w.rows), static_cast<int>(ldy));
        LARQL_HIP_CHECK(hipGetLastError());
    }
}

size_t q4k_gemm_ws_bytes(size_t m, size_t cols) {
    const size_t m_pad = (m + 16 * kMt - 1) / (16 * kMt) * (16 * kMt);
    return m_pad * cols * sizeof(uint16_t);
}

void launch_q4k_gemm(const DevWeight& w, const float* X, float* Y, size_t m, void* ws, hipStream_t s) {
    if (w.format != LARQL_Q4_K) fail(LARQL_HIP_ERR_UNSUPPORTED, "prefill GEMM: Q4_K weights only");
    if (m == 0) return;
    if (!ws) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: no workspace");
    if (m > 0x7FFFFFFF / w.cols) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: too many tokens");
    const size_t mtiles = (m + 16 * kMt - 1) / (16 * kMt) * kMt;  // 16-token tiles, padded
    x16_pack_kernel<<<dim3(static_cast<unsigned>(w.cols / 256), static_cast<unsigned>(mtiles)), dim3(256), 0, s>>>(
        X, static_cast<v4u*>(ws), static_cast<int>(m), static_cast<int>(w.cols));
    LARQL_HIP_CHECK(hipGetLastError());
    const dim3 grid(static_cast<unsigned>((w.rows + kNwg - 1) / kNwg), static_cast<unsigned>(mtiles / kMt));
    q4k_gemm_kernel<<<grid, dim3(kThreads), 0, s>>>(w.qs, reinterpret_cast<const v4u*>(w.hdr),
                                                     static_cast<const v4u*>(ws), Y, static_cast<int>(m),
                                                     static_cast<int>(w.rows), static_cast<int>(w.cols),
                                                     static_cast<int>(w.rows_pad / 16));
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
