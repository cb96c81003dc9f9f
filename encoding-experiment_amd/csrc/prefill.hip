// Quantized prefill: Y[M x N] = X[M x K] . deq(W)^T for a Q4_K weight W [N x K],
// M tokens at once (M = 512 in the prefill workload).
//
// Reference semantics: the trait's prefill (LC/src/backend.rs:143-152) runs, per token,
// the Q4_K matvec (LC/src/cpu/ops/q4k_matvec.rs:31-90; the Metal prefill is that matvec
// in a loop over positions, LC/src/metal/prefill.rs:21-110).  Here the M matvecs are one
// GEMM on the matrix cores, v_mfma_f32_16x16x32_f16 with f32 accumulation:
//   * x16_pack_kernel converts X to fp16 once, laid out as ready-made A operands:
//     one 1 KB block (64 lanes x 8 halves) per (16 tokens, super-block, half, step);
//   * the GEMM (q4k_gemm_shared_kernel) streams the tile-major Q4_K weights and
//     dequantizes each 16-row tile and k-step once per 256 tokens into fp16 B operands in
//     LDS, w = (1024 + q) * (d sc_j) - (1024 d sc_j + dmin m_j) in one f32 fma per element,
//     rounded to fp16 (the same value as d sc_j q - dmin m_j, to ~2^-14 d sc_j);
//   * each of its eight waves multiplies its own 32 tokens, A operands straight from the
//     packed X into registers, by the shared B operands of 80 weight rows.
// The MFMA k order within a step is free as long as A and B agree: lane (g, c) of step s
// in half h supplies elements 8s + {0,4,1,5,2,6,3,7} of sub-block 4h + g (the order in
// which the nibble bytes unpack), and x16_pack_kernel writes X in that order.
// fp16 operands carry 11 significant bits: over K = 2560 random terms the error is
// ~1e-4 of max|Y|, inside the 1e-3 bar.
#include <type_traits>

#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Tiling of the f32-accuracy GEMMs (q4k_gemm_sq_kernel, q6k_gemm_hp_kernel); the packed
// X of the fp16 GEMM is padded to kMt tiles of 16 tokens.
constexpr int kMt = 4;                 // 16-token tiles per workgroup (64 tokens)
constexpr int kNT = 5;                 // 16-row weight tiles per wave (80 rows; Q4_K: 4 or 5)
constexpr int kWaves = 4;              // waves per workgroup, side by side along N
constexpr int kThreads = 64 * kWaves;

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

// ── fp16 operands with the dequantization shared by the workgroup ─────────
// 256 tokens x 80 weight rows per workgroup (grid 128 x 2 = one workgroup per CU at
// M = 512, N = 10240), eight waves, two per SIMD (one wave's loads wait while the other
// multiplies).  Each unit (half super-block, 128 k, four k-steps of 32) is dequantized
// once: wave w turns k-step w % 4 of tiles 0-2 (w < 4) or 3-4 (w >= 4) into fp16 B
// operands in LDS, then every wave multiplies its own 32 tokens (two A tiles from the
// packed X, straight into registers) by the B operands of all four steps.  Per unit and
// SIMD: five 8-weight dequantizations and their scales against 80 MFMAs, where a wave that
// dequantizes its own rows for its own 64 tokens does twenty.
constexpr int kShTiles = 5;                   // 16-row weight tiles per workgroup
constexpr int kShWaves = 8;
constexpr int kShThreads = 64 * kShWaves;
constexpr int kShMt = 2;                      // 16-token tiles per wave
constexpr int kShTok = 16 * kShMt * kShWaves;  // 256 tokens per workgroup
constexpr int kShDq = 3;                      // most tiles one wave dequantizes per unit

__global__ __launch_bounds__(kShThreads) void q4k_gemm_shared_kernel(const uint8_t* __restrict__ qs,
                                                                     const v4u* __restrict__ hdr,
                                                                     const v4u* __restrict__ XP, float* __restrict__ Y,
                                                                     int M, int N, int K, int ntiles, int mtiles) {
    __shared__ v4u Bs[3][kShTiles][4][64];  // B operands of three units (60 KB)
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c = lane & 15;
    const int S = K / 256;
    const int n = 2 * S;  // units: (super-block u / 2, half u % 2)
    const int nt0 = blockIdx.x * kShTiles;
    const int mtw = blockIdx.y * (kShTok / 16) + wave * kShMt;  // first 16-token tile of this wave
    const int step = wave & 3;                                  // the k-step this wave dequantizes
    const int dj0 = wave < 4 ? 0 : 3, dn = wave < 4 ? 3 : 2;    // and its tiles dj0 .. dj0 + dn - 1

    // qs block (sb 0, half 0) of dequantized tile jj, offset to this wave's dword of the
    // lane's 16-byte nibble slot, and the tile's header block
    uint32_t qo[kShDq], ho[kShDq];
#pragma unroll
    for (int jj = 0; jj < kShDq; jj++) {
        const uint32_t t = static_cast<uint32_t>(min(nt0 + dj0 + min(jj, dn - 1), ntiles - 1));
        qo[jj] = __builtin_amdgcn_readfirstlane(t * S * 2048u + 4u * step);
        ho[jj] = __builtin_amdgcn_readfirstlane(t * S * 256u);
    }
    // Every load is a raw buffer load: the wave-uniform part of the offset in the scalar
    // operand, the lane's byte offset in the vector operand, so no vector ALU goes to
    // addresses.  All offsets are in range (tiles clamped, units below n).
    const uint32_t lo16 = lane * 16u, lc16 = c * 16u;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(qs), 0, static_cast<int>(static_cast<uint32_t>(ntiles) * S * 2048u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<v4u*>(hdr), 0, static_cast<int>(static_cast<uint32_t>(ntiles) * S * 256u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<v4u*>(XP), 0, static_cast<int>(static_cast<uint32_t>(mtiles) * n * 4096u), 0x00020000);
    // A tile i of this wave: XP[(mt n + u) 256 + s 64 + lane], mt clamped into the packed X
    // (tiles past it hold tokens >= M, whose rows are not stored)
    uint32_t xo[kShMt];
#pragma unroll
    for (int i = 0; i < kShMt; i++)
        xo[i] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(min(mtw + i, mtiles - 1)) * n * 4096u);

    struct Au {
        v4u v[kShMt][4];  // [tile][k-step]
    };
    auto load_a = [&a_rs = rx, &xo, lo16](int u, Au& a) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kShMt; i++)
#pragma unroll
            for (int s = 0; s < 4; s++)
                a.v[i][s] = __builtin_bit_cast(
                    v4u, __builtin_amdgcn_raw_buffer_load_b128(a_rs, lo16, xo[i] + u * 4096u + s * 1024u, 0));
    };
    struct Wu {
        uint32_t q[kShDq];
        v4u hd[kShDq];
    };
    auto load_w = [&qo, &ho, rq, rh, lo16, lc16](int u, Wu& w) __attribute__((always_inline)) {
#pragma unroll
        for (int jj = 0; jj < kShDq; jj++) {
            w.q[jj] = __builtin_amdgcn_raw_buffer_load_b32(rq, lo16, qo[jj] + u * 1024u, 0);
            w.hd[jj] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rh, lc16, ho[jj] + (u >> 1) * 256u, 0));
        }
    };
    uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u;
    asm volatile("" : "+v"(m_lo), "+v"(m_hi));  // keep the masks in VGPRs
    // this wave's k-step of unit u for its tiles -> LDS buffer b
    auto dequant = [&](int u, const Wu& w, int b) __attribute__((always_inline)) {
        const int h = u & 1;
#pragma unroll
        for (int jj = 0; jj < kShDq; jj++) {
            if (jj >= dn) break;
            const float d = h2f(w.hd[jj].x & 0xFFFFu), dmin = h2f(w.hd[jj].x >> 16);
            const uint32_t scw = h ? w.hd[jj].z : w.hd[jj].y;
            const float sc = d * static_cast<float>((scw >> (8 * g)) & 0x3Fu);
            const float mn = dmin * static_cast<float>((w.hd[jj].w >> (8 * g + 4 * h)) & 0xFu);
            SubScale k;
            k.sc = sc;
            // -(1024 sc + mn) as one fma with negated operands (no separate negation)
            k.c_lo = __builtin_fmaf(-1024.f, sc, -mn);
            k.sc16 = sc * 0.0625f;
            k.c_hi = __builtin_fmaf(-64.f, sc, -mn);
            Bs[b][dj0 + jj][step][lane] = __builtin_bit_cast(v4u, deq8(w.q[jj], k, m_lo, m_hi));
        }
    };
    floatx4 acc[kShMt][kShTiles];
#pragma unroll
    for (int i = 0; i < kShMt; i++)
#pragma unroll
        for (int j = 0; j < kShTiles; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    const bool live = mtw < mtiles;  // wave-uniform: this wave has tokens to multiply
    // the B operands of step s + 1 are read from LDS before the MFMAs of step s are issued
    auto mfma = [&](const Au& a, int b) __attribute__((always_inline)) {
        if (!live) return;
        v4u bq[2][kShTiles];
#pragma unroll
        for (int j = 0; j < kShTiles; j++) bq[0][j] = Bs[b][j][0][lane];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            if (s < 3) {
#pragma unroll
                for (int j = 0; j < kShTiles; j++) bq[(s + 1) & 1][j] = Bs[b][j][s + 1][lane];
            }
            __builtin_amdgcn_sched_barrier(0);  // keep those reads ahead of this step's MFMAs
#pragma unroll
            for (int i = 0; i < kShMt; i++)
#pragma unroll
                for (int j = 0; j < kShTiles; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a.v[i][s]),
                                                                       __builtin_bit_cast(half8, bq[s & 1][j]),
                                                                       acc[i][j], 0, 0, 0);
        }
    };

    // Three-unit ring: unit u multiplies from LDS buffer u % 3 and A registers u % 3 and
    // was dequantized from weight registers u % 3.  In the stage of unit u the wave first
    // dequantizes unit u + 1 (its weights were requested two stages before) into buffer
    // (u + 1) % 3, requests the weights of unit u + 3, multiplies unit u, then requests the
    // A tiles of unit u + 3 into the registers it just used.  A barrier ends each stage:
    // buffer (u + 1) % 3 is complete, and the buffer the next stage overwrites was last
    // read two stages before.  Loads past the last unit re-read it (unused).
    Au a0, a1, a2;
    Wu w0, w1, w2;
    load_w(0, w0);
    load_a(0, a0);
    load_w(min(1, n - 1), w1);
    load_a(min(1, n - 1), a1);
    load_w(min(2, n - 1), w2);
    load_a(min(2, n - 1), a2);
    dequant(0, w0, 0);
    __syncthreads();
    auto stage = [&](int u, int b, Au& a, const Wu& wn, Wu& wr) __attribute__((always_inline)) {
        if (u + 1 < n) dequant(u + 1, wn, b == 2 ? 0 : b + 1);
        load_w(min(u + 3, n - 1), wr);
        mfma(a, b);
        load_a(min(u + 3, n - 1), a);
        __syncthreads();
    };
    int u = 0;
    for (; u + 3 <= n; u += 3) {
        stage(u, 0, a0, w1, w0);
        stage(u + 1, 1, a1, w2, w1);
        stage(u + 2, 2, a2, w0, w2);
    }
    if (u < n) stage(u, 0, a0, w1, w0);
    if (u + 1 < n) stage(u + 1, 1, a1, w2, w1);

    // D lane (g, c) holds rows 4g .. 4g + 3 of column c of each 16 x 16 tile
    if (!live) return;
#pragma unroll
    for (int i = 0; i < kShMt; i++)
#pragma unroll
        for (int j = 0; j < kShTiles; j++) {
            const int col = (nt0 + j) * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = (mtw + i) * 16 + 4 * g + r;
                if (m < M && col < N) Y[static_cast<size_t>(m) * N + col] = acc[i][j][r];
            }
        }
}

// ── f32 inputs to f32 accuracy: fp16 operand pairs on the matrix cores ────
// The accurate GEMMs for chains of projections (the batched prompt pass; Q6_K with m > 1):
// q4k_gemm_sq_kernel (Q4_K) and q6k_gemm_hp_kernel (Q6_K).  64 tokens x 320 weight rows per
// workgroup, 80 rows per wave (each wave prepares its own rows' operands for the
// workgroup's tokens), two-unit ring of X staged in LDS.  Every f32 operand v is split into
// two fp16 parts, hi = fp16(v) and lo = fp16(v - hi) (v - hi exact in f32), so v = hi + lo
// to ~2^-22; a product of two split operands runs as three v_mfma_f32_16x16x32_f16 with f32
// accumulation, x_hi w_hi + x_hi w_lo + x_lo w_hi (the dropped x_lo w_lo is ~2^-22 of it),
// one with an exact fp16 weight operand as two.  Single fp16 operands (2^-11) compounded
// past the bar through 8 and 16 layers, and bf16 pairs (hi = 8 bits, 2^-16 per product)
// doubled the error.  fp16's range is made safe per token: row_exp_kernel gives each X row
// the power of two that puts its largest |x| in [2^14, 2^15), the staging scales the row by
// it and the epilogue divides it out, both exact.  Q6_K weights are dequantized,
// w = d sc (q - 32) in f32, then split (|w| must stay below 65504).  A k-step of 32 takes
// elements 8 s .. 8 s + 7 of the lane's sub-block 4 h + g for lane group g (Q6_K), in the
// order the nibbles unpack (0, 2, 4, 6, 1, 3, 5, 7), and the X staging writes its fp16
// pairs in that order.  An infinite operand gives NaN (its lo part is inf - inf).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// v - (f32) the low / high f16 half of h2, one v_fma_mix_f32 (the half widened inside the
// instruction; written out because the compiler otherwise emits a conversion and a subtract)
__device__ __forceinline__ float sub_f16_lo(float v, uint32_t h2) {
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(v));
    return r;
}
__device__ __forceinline__ float sub_f16_hi(float v, uint32_t h2) {
    float r;
    asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h2), "v"(v));
    return r;
}

// {a, b} -> hi pair {fp16(a), fp16(b)} and lo pair {fp16(a - hi_a), fp16(b - hi_b)}
__device__ __forceinline__ void hp_split2(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
    const float la = sub_f16_lo(a, hi), lb = sub_f16_hi(b, hi);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){la, lb}, f16x2));
}

// Eight f32 values in the k-step order -> the step's hi and lo operands.
__device__ __forceinline__ void hp_split8(const float (&v)[8], v4u& hi, v4u& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) hp_split2(v[2 * i], v[2 * i + 1], h[i], l[i]);
    hi = v4u{h[0], h[1], h[2], h[3]};
    lo = v4u{l[0], l[1], l[2], l[3]};
}

constexpr int kHpPitch = 36;  // dwords per lane slot in LDS: 16 hi + 16 lo + 4 (spread the banks)

// X staging: the thread's 32 elements (8 float4) times its token's power of two -> hi
// dwords 0..15 and lo dwords 16..31 of its LDS slot, step s at dwords 4 s .. 4 s + 3 in
// the order (0, 2), (4, 6), (1, 3), (5, 7) of elements 8 s + ...
// (STEP, LO: dwords from step s to s + 1 and from a step's hi to its lo dwords; the
// defaults are the slot layout above)
template <int STEP = 4, int LO = 16>
__device__ __forceinline__ void hp_store_x(uint32_t* d, const float4 (&v)[8], float scale) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const float4 a = v[2 * s], b = v[2 * s + 1];
        const float e[8] = {a.x * scale, a.z * scale, b.x * scale, b.z * scale,
                            a.y * scale, a.w * scale, b.y * scale, b.w * scale};
        v4u hi, lo;
        hp_split8(e, hi, lo);
        *reinterpret_cast<v4u*>(d + STEP * s) = hi;
        *reinterpret_cast<v4u*>(d + STEP * s + LO) = lo;
    }
}

// acc[i] += A_i . B for the three operand-pair products of one k-step
template <int MT>
__device__ __forceinline__ void hp3_mfma(floatx4 (&acc)[MT], const v4u (&ah)[MT], const v4u (&al)[MT], const v4u& bh,
                                         const v4u& bl) {
    const half8 Bh = __builtin_bit_cast(half8, bh), Bl = __builtin_bit_cast(half8, bl);
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ah[i]), Bh, acc[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ah[i]), Bl, acc[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < MT; i++) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, al[i]), Bh, acc[i], 0, 0, 0);
}

// One workgroup per row: the row's exponent and (with xs) scaled sub-block sums
// (gemm_row_stats).
__global__ __launch_bounds__(256) void row_exp_kernel(const float* __restrict__ X, int K, int* __restrict__ e,
                                                      float* __restrict__ xs) {
    gemm_row_stats(X + static_cast<size_t>(blockIdx.x) * K, K, e + blockIdx.x,
                   xs ? xs + static_cast<size_t>(blockIdx.x) * (K / 32) : nullptr);
}

// The staging thread's token scale and the workgroup's per-token inverses (the first 64
// threads), from the row exponents.
__device__ __forceinline__ float hp_token_scales(const int* __restrict__ xe, int M, int mt0, int xr_row, float* inv) {
    if (threadIdx.x < 16 * kMt) {
        const int t = mt0 * 16 + static_cast<int>(threadIdx.x);
        inv[threadIdx.x] = t < M ? ldexpf(1.0f, -xe[t]) : 1.0f;
    }
    return ldexpf(1.0f, xe[min(xr_row, M - 1)]);
}

// ── Q4_K prompt GEMM on exact integer weight operands ─────────────────────
// The Q4_K form of the f32-accuracy GEMM.  A Q4_K weight is w = d s_j q - dmin m_j (q the
// 4-bit code, s_j and m_j the 6-bit scale and 4-bit min of its 32-element sub-block j, d
// and dmin f16 per super-block), so per super-block and token
//   sum_k x_k w_k = d sum_j s_j (sum_{k in j} x_k q_k) - dmin sum_j m_j X_j,  X_j = sum_{k in j} x_k.
// s_j q <= 945 is an exact fp16 integer: the first sum runs on v_mfma_f32_16x16x32_f16 with
// the weight operand s_j q and the token operand split into fp16 hi and lo parts (two
// products, both exact in f32; only the split's 2^-22 is lost), one k-step per sub-block
// and a fresh accumulator per super-block, added into the total times d.  The min term
// comes after the K loop: the sub-block sums X_j 2^(e - 5) (row_exp_kernel) against
// -32 dmin m_j per row, both as fp16 pairs (three products), 32 sub-blocks per k-step.
// Tiling and X staging as the other f32-accuracy GEMMs; a lane's 16-byte nibble load holds one
// sub-block (lane group g: sub-block 4 h + g), so a 4 x 4 transpose of its words across the
// lane groups (two v_permlane32_swap, two v_permlane16_swap) gives lane group g word g
// (elements 8 g .. 8 g + 7) of each of the unit's four sub-blocks.  The weight operand is
// built as fp16 pairs: 0x64 above each code byte is 1024 + q, and
// fma(1024 + q, s, -1024 s) = s q exactly.  Weights need dmin below ~136 (fp16 range of
// 32 dmin m_j); d has no limit.
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
constexpr int kSqPitch = 12;  // dwords per staged cell: 4 hi + 4 lo + 4 (spread the banks)

__device__ __forceinline__ uint32_t sq_pair(uint32_t codes, uint32_t sel, h2v s, h2v ns) {
    const h2v b = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, codes, sel));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(b, s, ns));
}

template <int NT>
__global__ __launch_bounds__(kThreads) void q4k_gemm_sq_kernel(const uint8_t* __restrict__ qs,
                                                               const v4u* __restrict__ hdr,
                                                               const float* __restrict__ X, const int* __restrict__ xe,
                                                               const float* __restrict__ xs, float* __restrict__ Y,
                                                               int M, int N, int K, int ntiles, int sb_per, int ldy,
                                                               int gx, int gy, int gz) {
    // staged X by k-step: cell [t][16 s + token] holds step s (elements 8 s .. 8 s + 7) of
    // sub-block 4h + t, hi dwords 0..3 and lo 4..7, so the k-step t operand of lane l is
    // cell [t][l] (12-dword pitch: no bank conflicts for the reads or the writes)
    __shared__ uint32_t Aq[2][kMt][4][64][kSqPitch];
    __shared__ float tok_inv[16 * kMt];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int S = K / 256;
    // Workgroup -> (weight block bx, token block by, K split bz), a 1-D grid: the gy token
    // blocks of one (bx, bz) get consecutive ids that are equal mod 8, i.e. one XCD (ids go
    // round-robin over the 8) at about the same time, so a weight block is fetched into
    // that XCD's L2 once for all tokens; ids past the gx gz pairs (rounded up to 8) exit.
    const int L = static_cast<int>(blockIdx.x), slot = L >> 3, by = slot % gy;
    const int grp = (slot / gy) * 8 + (L & 7);
    if (grp >= gx * gz) return;
    const int bx = grp % gx, bz = grp / gx;
    const int mt0 = by * kMt;
    const int nt0 = (bx * kWaves + wave) * NT;
    // split bz of K: super-blocks [bz sb_per, (bz + 1) sb_per), partial sums to Y[bz]
    const int u0 = 2 * bz * sb_per, u1 = min(2 * S, u0 + 2 * sb_per), last = u1 - 1;
    Y += static_cast<size_t>(bz) * M * ldy;
    uint32_t qo[NT], ho[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) {
        const uint32_t t = static_cast<uint32_t>(min(nt0 + j, ntiles - 1));
        qo[j] = __builtin_amdgcn_readfirstlane(t * S * 2048u);
        ho[j] = __builtin_amdgcn_readfirstlane(t * S * 256u);
    }
    // X staging: slot l of tile r holds sub-block 4h + l / 16 of token 16 (mt0 + r) + l % 16;
    // a token past M re-reads row M - 1 (its D rows are never stored, and MFMA rows do not
    // mix; no branch around the loads)
    const int xr_row = (mt0 + (tid >> 6)) * 16 + (lane & 15);
    // raw buffer loads: the wave-uniform part of each offset in the scalar operand, the
    // lane's in the vector operand (the launcher keeps X, the nibbles and the headers below
    // 2 GiB)
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X), 0, static_cast<int>(static_cast<uint32_t>(M) * K * 4u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(qs), 0, static_cast<int>(static_cast<uint32_t>(ntiles) * S * 2048u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<v4u*>(hdr), 0, static_cast<int>(static_cast<uint32_t>(ntiles) * S * 256u), 0x00020000);
    const uint32_t xoff = (static_cast<uint32_t>(min(xr_row, M - 1)) * K + 32u * g) * 4u;
    const uint32_t lo16 = lane * 16u, lc16 = c * 16u;
    const float xscale = hp_token_scales(xe, M, mt0, xr_row, tok_inv);
    struct Xu {
        float4 v[8];
    };
    // (each group of loads kept whole and in program order, so that the wait before a
    // group's first use counts just the loads issued after it)
    auto load_x = [&](int u, Xu& x) __attribute__((always_inline)) {
        const uint32_t so = static_cast<uint32_t>(u) * 512u;  // (256 (u >> 1) + 128 (u & 1)) floats
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < 8; k++)
            x.v[k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, xoff + 16u * k, so, 0));
        __builtin_amdgcn_sched_barrier(0);
    };
    auto store_x = [&](int b, const Xu& x) __attribute__((always_inline)) {
        hp_store_x<16 * kSqPitch, 4>(&Aq[b][tid >> 6][lane >> 4][lane & 15][0], x.v, xscale);
    };
    // a unit's nibbles and the header words it uses: h = 0 (the first half of a super-block)
    // d | dmin and the scales of sub-blocks 0..3, h = 1 the scales of 4..7
    struct Wu {
        v4u q[NT];
        uint32_t hx[NT], hs[NT];
    };
    const uint8_t* hdrb = reinterpret_cast<const uint8_t*>(hdr) + c * 16;
    auto load_w = [&](int u, Wu& w) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < NT; j++) {
            w.q[j] = __builtin_bit_cast(
                v4u, __builtin_amdgcn_raw_buffer_load_b128(rq, lo16, qo[j] + static_cast<uint32_t>(u) * 1024u, 2));
            const uint32_t hso = ho[j] + static_cast<uint32_t>(u >> 1) * 256u;
            if (u & 1) {
                w.hs[j] = __builtin_amdgcn_raw_buffer_load_b32(rh, lc16, hso + 8u, 0);
            } else {
                const auto h2 = __builtin_amdgcn_raw_buffer_load_b64(rh, lc16, hso, 0);
                w.hx[j] = h2[0];
                w.hs[j] = h2[1];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    floatx4 acc[NT][kMt], dp[NT][kMt];
    float dsb[NT];  // d of the super-block in progress, per tile (row c)
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
        for (int i = 0; i < kMt; i++) acc[j][i] = dp[j][i] = floatx4{0.f, 0.f, 0.f, 0.f};

    // unit (sb, h) of buffer b: k-step t = sub-block 4h + t, lane (g, token c) takes its
    // elements 8 g .. 8 g + 7 (step g of the staging thread of token c, sub-block 4h + t)
    auto compute = [&](int b, auto hc, const Wu& w) __attribute__((always_inline)) {
        constexpr int h = decltype(hc)::value;
        v4u n[NT];
        uint32_t s6[NT];
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const auto a02 = __builtin_amdgcn_permlane32_swap(w.q[j].x, w.q[j].z, false, false);
            const auto a13 = __builtin_amdgcn_permlane32_swap(w.q[j].y, w.q[j].w, false, false);
            const auto r01 = __builtin_amdgcn_permlane16_swap(a02[0], a13[0], false, false);
            const auto r23 = __builtin_amdgcn_permlane16_swap(a02[1], a13[1], false, false);
            n[j] = v4u{r01[0], r01[1], r23[0], r23[1]};
            s6[j] = w.hs[j] & 0x3F3F3F3Fu;
            if constexpr (h == 0) dsb[j] = h2f(w.hx[j] & 0xFFFFu);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            v4u ah[kMt], al[kMt];
#pragma unroll
            for (int i = 0; i < kMt; i++) {
                ah[i] = *reinterpret_cast<const v4u*>(&Aq[b][i][t][lane][0]);
                al[i] = *reinterpret_cast<const v4u*>(&Aq[b][i][t][lane][4]);
            }
#pragma unroll
            for (int j = 0; j < NT; j++) {
                // s = scale of sub-block 4h + t (both halves), ns = -1024 s
                const h2v sv = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, s6[j], 0x04000400u + 0x00010001u * t)) -
                               h2v{1024.0f16, 1024.0f16};
                const h2v ns = sv * h2v{-1024.0f16, -1024.0f16};
                const uint32_t word = n[j][t];
                const uint32_t lo = word & 0x0F0F0F0Fu, hi = (word >> 4) & 0x0F0F0F0Fu;
                // elements (0, 2), (4, 6), (1, 3), (5, 7) of the eight, the staging's order
                const v4u bq = {sq_pair(lo, 0x04010400u, sv, ns), sq_pair(lo, 0x04030402u, sv, ns),
                                sq_pair(hi, 0x04010400u, sv, ns), sq_pair(hi, 0x04030402u, sv, ns)};
                const half8 B = __builtin_bit_cast(half8, bq);
#pragma unroll
                for (int i = 0; i < kMt; i++)
                    dp[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8, ah[i]), B, (h == 0 && t == 0) ? floatx4{0.f, 0.f, 0.f, 0.f} : dp[j][i],
                        0, 0, 0);
#pragma unroll
                for (int i = 0; i < kMt; i++)
                    dp[j][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, al[i]), B, dp[j][i], 0, 0, 0);
            }
        }
        if constexpr (h == 1) {  // the super-block's sum times d (row c)
#pragma unroll
            for (int j = 0; j < NT; j++) {
                const float d = dsb[j];
#pragma unroll
                for (int i = 0; i < kMt; i++)
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[j][i][r] = fmaf(d, dp[j][i][r], acc[j][i][r]);
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
    lds_barrier();
    for (int u = u0; u < u1; u += 2) {
        store_x(1, x1);
        load_x(min(u + 2, last), x0);
        compute(0, std::integral_constant<int, 0>{}, w0);
        load_w(min(u + 2, last), w0);
        lds_barrier();
        store_x(0, x0);
        load_x(min(u + 3, last), x1);
        compute(1, std::integral_constant<int, 1>{}, w1);
        load_w(min(u + 3, last), w1);
        lds_barrier();
    }

    // min term over super-blocks [SB0, SB1), four per k-step: lane group g takes super-block
    // q + g, its eight sub-blocks in order (token side: scaled sums; row side: -32 dmin m_j)
    const int SB0 = u0 >> 1, SB1 = u1 >> 1, nsb = K / 32;
    struct Mu {
        float4 x[kMt][2];
        v4u hd[NT];
    };
    auto load_m = [&](int q, Mu& mu) __attribute__((always_inline)) {
        const int sb = q + g;
        const bool sv = sb < SB1;
#pragma unroll
        for (int i = 0; i < kMt; i++) {
            const int tok = (mt0 + i) * 16 + c;
            const bool ok = sv && tok < M;
            const float4* p = reinterpret_cast<const float4*>(xs + static_cast<size_t>(min(tok, M - 1)) * nsb + 8 * min(sb, S - 1));
            mu.x[i][0] = ok ? p[0] : make_float4(0.f, 0.f, 0.f, 0.f);
            mu.x[i][1] = ok ? p[1] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < NT; j++)
            mu.hd[j] = sv ? *reinterpret_cast<const v4u*>(hdrb + ho[j] + static_cast<uint32_t>(sb) * 256u)
                          : v4u{0u, 0u, 0u, 0u};
    };
    auto apply_m = [&](const Mu& mu) __attribute__((always_inline)) {
        v4u ah[kMt], al[kMt];
#pragma unroll
        for (int i = 0; i < kMt; i++) {
            const float v[8] = {mu.x[i][0].x, mu.x[i][0].y, mu.x[i][0].z, mu.x[i][0].w,
                                mu.x[i][1].x, mu.x[i][1].y, mu.x[i][1].z, mu.x[i][1].w};
            hp_split8(v, ah[i], al[i]);
        }
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const float nd = -32.0f * h2f(mu.hd[j].x >> 16);
            float cm[8];
#pragma unroll
            for (int k = 0; k < 8; k++) cm[k] = nd * static_cast<float>((mu.hd[j].w >> (8 * (k & 3) + 4 * (k >> 2))) & 0xFu);
            v4u bh, bl;
            hp_split8(cm, bh, bl);
            hp3_mfma<kMt>(acc[j], ah, al, bh, bl);
        }
    };
    Mu m0, m1;
    load_m(SB0, m0);
    for (int q = SB0; q < SB1; q += 8) {
        load_m(q + 4, m1);
        apply_m(m0);
        if (q + 4 >= SB1) break;
        load_m(q + 8, m0);
        apply_m(m1);
    }

    // D lane (g, c) holds tokens 4g .. 4g + 3 of weight row c of each 16 x 16 tile
#pragma unroll
    for (int i = 0; i < kMt; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int col = (nt0 + j) * 16 + c;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = (mt0 + i) * 16 + 4 * g + r;
                if (m < M && col < N) Y[static_cast<size_t>(m) * ldy + col] = acc[j][i][r] * tok_inv[i * 16 + 4 * g + r];
            }
        }
}

// Q6_K weights (tile-major blocks, q6k_block in larql_hip_internal.h: ql nibble of element
// e at byte e / 2, its two high bits regrouped per 16-element group G: element 16 G + 8 w +
// 2 j + p at bits 8 j + 4 w + 2 p of word G; int8 scale per group; f16 d per block) with
// the same X staging and tiling: lane (g, c) of unit (sb, h) takes elements
// 32 (4h + g) .. + 31 of row c of each tile, i.e. 16 ql bytes, two high-bit words and two
// scales; w = fma(q, d sc, -32 d sc) = d sc (q - 32).
__global__ __launch_bounds__(kThreads) void q6k_gemm_hp_kernel(const uint8_t* __restrict__ q6,
                                                               const float* __restrict__ X, const int* __restrict__ xe,
                                                               float* __restrict__ Y, int M, int N, int K, int sb_per,
                                                               int ldy) {
    __shared__ uint32_t As[2][kMt][64][kHpPitch];
    __shared__ float tok_inv[16 * kMt];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int S = K / 256;
    const int mt0 = blockIdx.y * kMt;
    const int nt0 = (blockIdx.x * kWaves + wave) * kNT;
    const int u0 = 2 * static_cast<int>(blockIdx.z) * sb_per, u1 = min(2 * S, u0 + 2 * sb_per), last = u1 - 1;
    Y += static_cast<size_t>(blockIdx.z) * M * ldy;
    // the lane's row in tile j (rows past N re-read row N - 1): its tile's first block and
    // its offset in each part of a block (lane group gq = 2h + g / 2 of the unit's half h)
    size_t blk[kNT];
    uint32_t rc[kNT];
#pragma unroll
    for (int j = 0; j < kNT; j++) {
        const size_t row = static_cast<size_t>(min((nt0 + j) * 16 + c, N - 1));
        blk[j] = q6k_block(row, 0, S);
        rc[j] = static_cast<uint32_t>(row & 15);
    }
    const int xr_row = (mt0 + (tid >> 6)) * 16 + (lane & 15);
    const bool xr_ok = xr_row < M;
    const float* xrow = X + static_cast<size_t>(min(xr_row, M - 1)) * K + 32 * g;
    const float xscale = hp_token_scales(xe, M, mt0, xr_row, tok_inv);
    struct Xu {
        float4 v[8];
    };
    auto load_x = [&](int u, Xu& x) __attribute__((always_inline)) {
        const float4* p = reinterpret_cast<const float4*>(xrow + 256 * (u >> 1) + 128 * (u & 1));
#pragma unroll
        for (int k = 0; k < 8; k++) x.v[k] = xr_ok ? p[k] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    auto store_x = [&](int b, const Xu& x) __attribute__((always_inline)) {
        hp_store_x(&As[b][tid >> 6][lane][0], x.v, xscale);
    };
    struct Wu {
        v4u l[kNT];
        uint2 h[kNT];
        uint32_t sd[kNT];  // scales of groups G0, G0 + 1 | d << 16
    };
    auto load_w = [&](int u, Wu& w) __attribute__((always_inline)) {
        const uint32_t gq = 2 * (u & 1) + (g >> 1), g1 = g & 1;
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const uint8_t* b = q6 + blk[j] + static_cast<size_t>(u >> 1) * kQ6Block;
            const uint32_t lc = 16 * gq + rc[j];
            w.l[j] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(b + g1 * 1024 + lc * 16));
            w.h[j] = *reinterpret_cast<const uint2*>(b + kQ6Qh + lc * 16 + 8 * g1);
            w.sd[j] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(b + kQ6Sc + lc * 4 + 2 * g1)) |
                      (static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(b + kQ6D + 2 * rc[j])) << 16);
        }
    };
    floatx4 acc[kNT][kMt];
#pragma unroll
    for (int j = 0; j < kNT; j++)
#pragma unroll
        for (int i = 0; i < kMt; i++) acc[j][i] = floatx4{0.f, 0.f, 0.f, 0.f};

    // element e (0 .. 31) of the lane's part: the 6-bit code from its ql nibble and two
    // regrouped high bits, d sc (q - 32) as one fma
    auto q6w = [](const Wu& w, int j, int e, float sc, float nb) __attribute__((always_inline)) {
        const int e4 = e >> 2, t = e & 3;
        const uint32_t lo = w.l[j][e4 >> 1], hi = (e4 >> 2) ? w.h[j].y : w.h[j].x;
        const uint32_t q4 = (lo >> (16 * (e4 & 1) + 4 * t)) & 0xFu;
        const uint32_t q2 = (hi >> (16 * (e4 & 1) + 8 * (t >> 1) + 4 * ((e4 >> 1) & 1) + 2 * (t & 1))) & 3u;
        return __builtin_fmaf(static_cast<float>(q4 | (q2 << 4)), sc, nb);
    };
    auto compute = [&](int b, const Wu& w) __attribute__((always_inline)) {
        float ds[kNT][2];
#pragma unroll
        for (int j = 0; j < kNT; j++) {
            const float d = h2f(w.sd[j] >> 16);
            ds[j][0] = d * static_cast<float>(static_cast<int8_t>(w.sd[j] & 0xFFu));
            ds[j][1] = d * static_cast<float>(static_cast<int8_t>((w.sd[j] >> 8) & 0xFFu));
        }
#pragma unroll
        for (int s = 0; s < 4; s++) {
            v4u ah[kMt], al[kMt];
#pragma unroll
            for (int i = 0; i < kMt; i++) {
                ah[i] = *reinterpret_cast<const v4u*>(&As[b][i][lane][4 * s]);
                al[i] = *reinterpret_cast<const v4u*>(&As[b][i][lane][16 + 4 * s]);
            }
#pragma unroll
            for (int j = 0; j < kNT; j++) {
                const float sc = ds[j][s >> 1], nb = -32.f * sc;
                const int e0 = 8 * s;
                const float wt[8] = {q6w(w, j, e0 + 0, sc, nb), q6w(w, j, e0 + 2, sc, nb), q6w(w, j, e0 + 4, sc, nb),
                                     q6w(w, j, e0 + 6, sc, nb), q6w(w, j, e0 + 1, sc, nb), q6w(w, j, e0 + 3, sc, nb),
                                     q6w(w, j, e0 + 5, sc, nb), q6w(w, j, e0 + 7, sc, nb)};
                v4u bh, bl;
                hp_split8(wt, bh, bl);
                hp3_mfma<kMt>(acc[j], ah, al, bh, bl);
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
                if (m < M && col < N) Y[static_cast<size_t>(m) * ldy + col] = acc[j][i][r] * tok_inv[i * 16 + 4 * g + r];
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

// K-splits for the f32-accuracy GEMM (1..4, whole super-blocks each) and, for Q4_K, the
// 16-row weight tiles per wave (4 or 5; a workgroup's rows are 64 nt): the choice with the
// least modelled time, rounds of workgroups over the CUs (one workgroup per CU at a time)
// x units per workgroup (super-blocks x tiles, ~1.35 us each on MI355X), plus, when split,
// the partial sums written and summed ((splits + 1) m N floats at ~5 TB/s).  Measured at
// the 8B shape and 512 tokens: 4 tiles take the 4096-row projections from 63.6 to 55.7 us
// and [1024 x 4096] from 35.7 to 32.8 us; the [28672 x 4096] gate|up keeps 5 (323 us, 1
// split, against 370 + 31.5 us for 4 tiles, 2 splits and their sum).
struct F32Split {
    int splits, sb_per, nt;
};
F32Split f32_split(const DevWeight& w, size_t m) {
    const int S = static_cast<int>(w.cols / 256);
    const long cus = current_device_cus();
    const double unit_ns = 1350.0, sum_ns_per_float = 4.0 / 5000.0;  // 5 TB/s = 5000 bytes per ns
    F32Split best{1, S, kNT};
    double best_cost = -1.0;
    for (int nt = (w.format == LARQL_Q4_K ? 4 : kNT); nt <= kNT; nt++) {
        const long rows_wg = 16L * nt * kWaves;
        const long wgs = static_cast<long>((w.rows + rows_wg - 1) / rows_wg) * static_cast<long>((m + 16 * kMt - 1) / (16 * kMt));
        for (int s = 1; s <= 4 && s <= S; s++) {
            const int per = (S + s - 1) / s, eff = (S + per - 1) / per;
            double cost = static_cast<double>((wgs * eff + cus - 1) / cus) * per * nt * unit_ns;
            if (eff > 1) cost += static_cast<double>(eff + 1) * static_cast<double>(m) * static_cast<double>(w.rows) * sum_ns_per_float;
            if (best_cost < 0 || cost < best_cost) best = {eff, per, nt}, best_cost = cost;
        }
    }
    return best;
}

}  // namespace

// workspace: the K-split partials (when split), the m row exponents (ints), then for Q4_K
// the m x K / 32 scaled sub-block sums
size_t q4k_gemm_f32_part_floats(const DevWeight& w, size_t m) {
    const F32Split sp = f32_split(w, m);
    return (sp.splits > 1 ? sp.splits * m * w.rows : 0) + m + (w.format == LARQL_Q4_K ? 4 + m * (w.cols / 32) : 0);
}

size_t gemm_row_stats_floats(size_t m, size_t cols) { return m + 4 + m * (cols / 32); }

GemmRowStats gemm_row_stats_at(float* ws, size_t m, size_t /*cols*/) {
    // the exponents, then the sub-block sums from a 16-byte boundary (float4 reads)
    const uintptr_t at = reinterpret_cast<uintptr_t>(ws + m);
    return {reinterpret_cast<int*>(ws), reinterpret_cast<float*>((at + 15) & ~uintptr_t{15})};
}

void launch_gemm_row_stats(const float* X, size_t m, size_t cols, const GemmRowStats& st, hipStream_t s) {
    if (m == 0) return;
    if (cols % 32 != 0 || cols > 0x7FFFFFFF) fail(LARQL_HIP_ERR_INVALID, "GEMM row statistics: cols must be a multiple of 32");
    row_exp_kernel<<<dim3(static_cast<unsigned>(m)), dim3(256), 0, s>>>(X, static_cast<int>(cols), st.xe, st.xs);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_q4k_gemm_f32(const DevWeight& w, const float* X, float* Y, size_t m, float* part, size_t part_floats,
                         hipStream_t s, size_t ldy, const GemmRowStats* pre, GemmSplits* defer) {
    if (ldy == 0) ldy = w.rows;
    if (ldy < w.rows || ldy > 0x7FFFFFFF) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: bad output row stride");
    if (defer && ldy != w.rows) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: deferred split sums need dense output rows");
    if (w.format != LARQL_Q4_K && w.format != LARQL_Q6_K)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "prefill GEMM: Q4_K or Q6_K weights only");
    if (pre && (!pre->xe || (w.format == LARQL_Q4_K && !pre->xs)))
        fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: incomplete row statistics");
    if (m == 0) return;
    if (m > 0x7FFFFFFF / w.cols) fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: too many tokens");
    // row exponents, then for Q4_K the sub-block sums from a 16-byte boundary (float4 reads),
    // unless the caller computed them
    const size_t extra = pre ? 0 : m + (w.format == LARQL_Q4_K ? 4 + m * (w.cols / 32) : 0);
    if (extra && (!part || part_floats < extra))
        fail(LARQL_HIP_ERR_INVALID, "prefill GEMM: no workspace for the row exponents");
    F32Split sp = f32_split(w, m);
    if (sp.splits > 1 && (!part || part_floats < sp.splits * m * w.rows + extra))
        sp = {1, static_cast<int>(w.cols / 256), sp.nt};
    const size_t xe_at = sp.splits > 1 ? sp.splits * m * w.rows : 0;
    GemmRowStats st;
    if (pre) {
        st = {pre->xe, w.format == LARQL_Q4_K ? pre->xs : nullptr};
    } else {
        st = gemm_row_stats_at(part + xe_at, m, w.cols);
        if (w.format != LARQL_Q4_K) st.xs = nullptr;
        row_exp_kernel<<<dim3(static_cast<unsigned>(m)), dim3(256), 0, s>>>(X, static_cast<int>(w.cols), st.xe, st.xs);
        LARQL_HIP_CHECK(hipGetLastError());
    }
    const int* xe = st.xe;
    const float* xs = st.xs;
    const unsigned rows_wg = 16u * static_cast<unsigned>(sp.nt) * kWaves;
    const dim3 grid(static_cast<unsigned>((w.rows + rows_wg - 1) / rows_wg),
                    static_cast<unsigned>((m + 16 * kMt - 1) / (16 * kMt)), static_cast<unsigned>(sp.splits));
    const int ld_out = static_cast<int>(sp.splits > 1 ? w.rows : ldy);
    if (w.format == LARQL_Q4_K) {
        // (raw buffer offsets: X, the nibbles and the headers below 2 GiB)
        if (m * w.cols * 4 > 0x7FFFFFFF || (w.rows_pad / 16) * (w.cols / 256) * 2048 > 0x7FFFFFFF)
            fail(LARQL_HIP_ERR_UNSUPPORTED, "prefill GEMM: operands above 2 GiB");
        const unsigned pairs = grid.x * grid.z, lin = (pairs + 7) / 8 * 8 * grid.y;
        auto go = [&](auto ntc) {
            q4k_gemm_sq_kernel<decltype(ntc)::value><<<dim3(lin), dim3(kThreads), 0, s>>>(
                w.qs, reinterpret_cast<const v4u*>(w.hdr), X, xe, xs, sp.splits > 1 ? part : Y, static_cast<int>(m),
                static_cast<int>(w.rows), static_cast<int>(w.cols), static_cast<int>(w.rows_pad / 16), sp.sb_per, ld_out,
                static_cast<int>(grid.x), static_cast<int>(grid.y), static_cast<int>(grid.z));
        };
        if (sp.nt == 4) go(std::integral_constant<int, 4>{});
        else go(std::integral_constant<int, kNT>{});
    }
    else
        q6k_gemm_hp_kernel<<<grid, dim3(kThreads), 0, s>>>(
            w.qs, X, xe, sp.splits > 1 ? part : Y, static_cast<int>(m), static_cast<int>(w.rows), static_cast<int>(w.cols),
            sp.sb_per, ld_out);
    LARQL_HIP_CHECK(hipGetLastError());
    if (defer) *defer = {sp.splits > 1 ? part : nullptr, sp.splits};
    if (sp.splits > 1 && !defer) {
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
    // the kernel addresses X, the nibbles and the headers with 31-bit buffer offsets
    if (mtiles * 16 * w.cols * 2 > 0x7FFFFFFF || w.rows_pad * (w.cols / 2) > 0x7FFFFFFF)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "prefill GEMM: operands above 2 GiB");
    x16_pack_kernel<<<dim3(static_cast<unsigned>(w.cols / 256), static_cast<unsigned>(mtiles)), dim3(256), 0, s>>>(
        X, static_cast<v4u*>(ws), static_cast<int>(m), static_cast<int>(w.cols));
    LARQL_HIP_CHECK(hipGetLastError());
    const size_t ntiles = w.rows_pad / 16;
    const dim3 grid(static_cast<unsigned>((ntiles + kShTiles - 1) / kShTiles),
                    static_cast<unsigned>((mtiles * 16 + kShTok - 1) / kShTok));
    q4k_gemm_shared_kernel<<<grid, dim3(kShThreads), 0, s>>>(
        w.qs, reinterpret_cast<const v4u*>(w.hdr), static_cast<const v4u*>(ws), Y, static_cast<int>(m),
        static_cast<int>(w.rows), static_cast<int>(w.cols), static_cast<int>(ntiles), static_cast<int>(mtiles));
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
