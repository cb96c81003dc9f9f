// Vindex gate-KNN: batched gate scores and top-k selection.
//
//   scores (f32)  : LV/src/index/gate.rs:14-29 (gemv / gate_matmul: gate[F,K] . x[K]),
//                   batched over queries as gate_knn_batch does (:500-537).
//   scores (Q4_0) : gate_knn_q4, LV/src/index/gate.rs:711-731: quantize_to_q8(x), then
//                   ComputeBackend::q4_matvec, i.e. per block (float)isum_b * (f16(s) * q8s_b)
//                   accumulated in block order (LC/csrc/q4_dot.c:58-89).
//   top-k         : top_k_from_scores, LV/src/index/gate.rs:307-316 (|score| descending);
//                   signed variant for the lm-head walk, LV/src/index/walk.rs:563-580.
//
// The f32 scores are single fma chains over k from +0 per (feature, query), the
// oracle's canonical order, so scores and therefore top-k indices are bit-exact.
#include "device_common.h"
#include "knn.h"

#include <algorithm>
#include <type_traits>

// The Q4_0 path must round the product and the sum separately, as the reference's
// `acc += (float)isum * cs` does; explicit fmaf() calls (the f32 path) are unaffected.
#pragma clang fp contract(off)

namespace larql {

namespace {

constexpr int kThreads = 256;

// ── f32 scores ─────────────────────────────────────────────────────────────
// Workgroup tile: 64 features x 256 queries; thread tile 8 queries x 8 features
// (64 accumulators).  K advances in LDS stages of 16, double-buffered, with the
// next stage's global loads in registers while the current stage is consumed.
constexpr int kF32TileF = 64, kF32TileQ = 256, kF32Ks = 16;

__global__ __launch_bounds__(kThreads, 3) void gate_scores_f32_kernel(KnnLayers g, const float* __restrict__ X,
                                                                   float* __restrict__ S, int F, int K, int Q) {
    __shared__ float Gs[2][kF32Ks][kF32TileF];
    __shared__ float Xs[2][kF32Ks][kF32TileQ];
    const int l = blockIdx.z;
    const float* __restrict__ G = static_cast<const float*>(g.p[l]);
    const int f0 = blockIdx.x * kF32TileF, q0 = blockIdx.y * kF32TileQ;
    const int tid = threadIdx.x;
    const int tq = tid & 31, tf = tid >> 5;  // queries q0 + 8 tq .., features f0 + 8 tf ..
    // global -> LDS: G row f0 + (tid & 63), k-quarter tid >> 6; X row q0 + tid, all 16 k
    const int lf = tid & 63, lk = 4 * (tid >> 6);
    const float* gp = G + static_cast<size_t>(min(f0 + lf, F - 1)) * K + lk;
    const float* xp = X + static_cast<size_t>(min(q0 + tid, Q - 1)) * K;
    float4 gr, xr[4];
    auto gload = [&](int k0) __attribute__((always_inline)) {
        gr = *reinterpret_cast<const float4*>(gp + k0);
#pragma unroll
        for (int i = 0; i < 4; i++) xr[i] = *reinterpret_cast<const float4*>(xp + k0 + 4 * i);
    };
    auto lstore = [&](int b) __attribute__((always_inline)) {
        Gs[b][lk + 0][lf] = gr.x;
        Gs[b][lk + 1][lf] = gr.y;
        Gs[b][lk + 2][lf] = gr.z;
        Gs[b][lk + 3][lf] = gr.w;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            Xs[b][4 * i + 0][tid] = xr[i].x;
            Xs[b][4 * i + 1][tid] = xr[i].y;
            Xs[b][4 * i + 2][tid] = xr[i].z;
            Xs[b][4 * i + 3][tid] = xr[i].w;
        }
    };
    float acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[i][j] = 0.f;

    const int nk = K / kF32Ks;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int s = 0; s < nk; s++) {
        const int b = s & 1;
        if (s + 1 < nk) gload((s + 1) * kF32Ks);
#pragma unroll 2
        for (int k = 0; k < kF32Ks; k++) {
            const float4 xa = *reinterpret_cast<const float4*>(&Xs[b][k][tq * 8]);
            const float4 xb = *reinterpret_cast<const float4*>(&Xs[b][k][tq * 8 + 4]);
            const float4 ga = *reinterpret_cast<const float4*>(&Gs[b][k][tf * 8]);
            const float4 gb = *reinterpret_cast<const float4*>(&Gs[b][k][tf * 8 + 4]);
            const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
            for (int i = 0; i < 8; i++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc[i][j] = fmaf(gv[j], xv[i], acc[i][j]);
        }
        // buffer b ^ 1 was last read in stage s - 1, before that stage's barrier
        if (s + 1 < nk) lstore(b ^ 1);
        __syncthreads();
    }
    float* Sl = S + static_cast<size_t>(l) * Q * F;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int q = q0 + tq * 8 + i;
        if (q >= Q) continue;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int f = f0 + tf * 8 + j;
            if (f < F) Sl[static_cast<size_t>(q) * F + f] = acc[i][j];
        }
    }
}

// ── Q4_0 x Q8 scores on the matrix cores ───────────────────────────────────
// v_mfma_i32_16x16x64_i8 gives exact int32 block dots for 16 features x 8 queries x one
// block pair: B (64 x 16) = the features' codes minus 8 (column c = feature c, k-group g
// = block g / 2, half g % 2), A (16 x 64) = row 2m + h holding query m's int8 block
// 2bp + h in that block's k-groups and zeros in the other block's, so D[2m + h][c] is
// block 2bp + h's dot sum((nib - 8) * x) for query m and feature c.  D lane (g, c)
// holds queries 2g and 2g + 1 of the group, both blocks of the pair: the lane forms
// (float)isum * (f16(d) * xs) and adds it to the query's running sum in block order,
// exactly as the reference's serial loop (product and sum rounded separately).
// The queries are laid out once per walk (q4_xa_kernel) as the A operands of every
// (block pair, group of 8 queries), zeros included, plus their block scales; a
// workgroup (128 features x 128 queries) stages one block pair of them in LDS per step,
// and each wave applies every A operand it reads to two sets of 16 features (two MFMAs
// per LDS read).  The loop is bound by VALU issue: the reference's accumulate costs four
// VALU operations per (feature, query, block) (conversion, two products, sum).
constexpr int kQ4TileF = 128, kQ4TileG = 16;  // features, groups of 8 queries

// XA[bp][G][lane][16 B], XSP[bp][G][8 m][2 h] = xs of query 8G + m, block 2bp + h.
// One thread per (bp, G, lane).  Element order within a 16-element half block matches
// the nibble unpack: even elements 0..6, odd 1..7, even 8..14, odd 9..15.
__global__ void q4_xa_kernel(const int8_t* __restrict__ X8, const float* __restrict__ XS, uint4* __restrict__ XA,
                             float* __restrict__ XSP, int K, int Q, int ng) {
    const size_t t = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    const int nbp = K / 64, nb = K / 32;
    if (t >= static_cast<size_t>(nbp) * ng * 64) return;
    const int lane = static_cast<int>(t & 63);
    const size_t bg = t >> 6;
    const int G = static_cast<int>(bg % ng), bp = static_cast<int>(bg / ng);
    const int g = lane >> 4, i = lane & 15, m = i >> 1, h = i & 1;
    const int q = 8 * G + m;
    uint4 v = make_uint4(0, 0, 0, 0);
    if ((g >> 1) == h && q < Q) {
        const uint4 raw = *reinterpret_cast<const uint4*>(X8 + static_cast<size_t>(q) * K + (2 * bp + h) * 32 + 16 * (g & 1));
        v.x = __builtin_amdgcn_perm(raw.y, raw.x, 0x06040200u);  // elements 0, 2, 4, 6
        v.y = __builtin_amdgcn_perm(raw.y, raw.x, 0x07050301u);  // 1, 3, 5, 7
        v.z = __builtin_amdgcn_perm(raw.w, raw.z, 0x06040200u);  // 8 .. 14
        v.w = __builtin_amdgcn_perm(raw.w, raw.z, 0x07050301u);  // 9 .. 15
    }
    XA[t] = v;
    if (lane < 16) XSP[bg * 16 + lane] = q < Q ? XS[static_cast<size_t>(q) * nb + 2 * bp + h] : 0.f;
}

typedef int v4i_t __attribute__((ext_vector_type(4)));

// Bytes of the codes minus 8 (signed), without borrows between bytes.
__device__ __forceinline__ int nib_s8(uint32_t w4) {
    return static_cast<int>(((w4 | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
}

// Grid (F / 128, ceil(groups / 16), layers); wave w: features f0 + 32 w + c (set 0) and
// f0 + 32 w + 16 + c (set 1).
__global__ __launch_bounds__(kThreads, 2) void gate_scores_q4_kernel(KnnLayers g, KnnLayers gd,
                                                                  const uint4* __restrict__ XA,
                                                                  const float* __restrict__ XSP, float* __restrict__ S,
                                                                  int F, int K, int Q, int ng) {
    __shared__ uint4 As[2][kQ4TileG][64];
    __shared__ float4 Xs[2][kQ4TileG][4];
    const int l = blockIdx.z;
    const uint8_t* __restrict__ nib = static_cast<const uint8_t*>(g.p[l]);
    const uint16_t* __restrict__ dsc = static_cast<const uint16_t*>(gd.p[l]);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int gl = lane >> 4, c = lane & 15;
    const int G0 = blockIdx.y * kQ4TileG, nG = min(kQ4TileG, ng - G0);
    const int fb = blockIdx.x * kQ4TileF + 32 * wave + c;  // set 0; set 1 is fb + 16
    const int nbp = K / 64, nb = K / 32;
    const uint8_t* wrow[2];
    const uint32_t* drow[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int f = min(fb + 16 * e, F - 1);
        wrow[e] = nib + static_cast<size_t>(f) * (K / 2) + (gl >> 1) * 16 + (gl & 1) * 8;
        drow[e] = reinterpret_cast<const uint32_t*>(dsc + static_cast<size_t>(f) * nb);
    }

    // staging: thread tid covers A items tid + 256 j of the tile's 16 x 64, and (tid < 64)
    // one float4 of the scales
    uint4 ar[4];
    float4 xr = make_float4(0.f, 0.f, 0.f, 0.f);
    uint2 wr[2];
    uint32_t dr[2];
    auto gload = [&](int bp) __attribute__((always_inline)) {
        const uint4* src = XA + (static_cast<size_t>(bp) * ng + G0) * 64;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int it = tid + 256 * j;
            ar[j] = (it >> 6) < nG ? src[it] : make_uint4(0, 0, 0, 0);
        }
        if (tid < 64 && (tid >> 2) < nG)
            xr = reinterpret_cast<const float4*>(XSP + (static_cast<size_t>(bp) * ng + G0) * 16)[tid];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            wr[e] = *reinterpret_cast<const uint2*>(wrow[e] + static_cast<size_t>(bp) * 32);
            dr[e] = drow[e][bp];
        }
    };
    auto lstore = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int it = tid + 256 * j;
            As[s][it >> 6][it & 63] = ar[j];
        }
        if (tid < 64) Xs[s][tid >> 2][tid & 3] = xr;
    };

    float acc[2][kQ4TileG][2];
#pragma unroll
    for (int e = 0; e < 2; e++)
#pragma unroll
        for (int G = 0; G < kQ4TileG; G++) acc[e][G][0] = acc[e][G][1] = 0.f;

    gload(0);
    lstore(0);
    __syncthreads();
    for (int bp = 0; bp < nbp; bp++) {
        const int s = bp & 1;
        v4i_t B[2];
        float d0[2], d1[2];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const uint2 w = wr[e];
            B[e] = v4i_t{nib_s8(w.x & 0x0F0F0F0Fu), nib_s8((w.x >> 4) & 0x0F0F0F0Fu), nib_s8(w.y & 0x0F0F0F0Fu),
                         nib_s8((w.y >> 4) & 0x0F0F0F0Fu)};
            d0[e] = h2f(dr[e]);
            d1[e] = h2f(dr[e] >> 16);
        }
        if (bp + 1 < nbp) gload(bp + 1);
#pragma unroll
        for (int G = 0; G < kQ4TileG; G++) {
            if (G < nG) {
                const uint4 av = As[s][G][lane];
                const v4i_t A = {static_cast<int>(av.x), static_cast<int>(av.y), static_cast<int>(av.z),
                                 static_cast<int>(av.w)};
                const float4 xs = Xs[s][G][gl];  // xs of queries 2g, 2g + 1, blocks 2bp, 2bp + 1
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const v4i_t D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B[e], v4i_t{0, 0, 0, 0}, 0, 0, 0);
                    // reference order: cs = f16(s) * q8s; acc += (float)isum * cs
                    acc[e][G][0] = acc[e][G][0] + static_cast<float>(D[0]) * (d0[e] * xs.x);
                    acc[e][G][0] = acc[e][G][0] + static_cast<float>(D[1]) * (d1[e] * xs.y);
                    acc[e][G][1] = acc[e][G][1] + static_cast<float>(D[2]) * (d0[e] * xs.z);
                    acc[e][G][1] = acc[e][G][1] + static_cast<float>(D[3]) * (d1[e] * xs.w);
                }
            }
        }
        // buffer s ^ 1 was last read in step bp - 1, before that step's barrier
        if (bp + 1 < nbp) lstore(s ^ 1);
        __syncthreads();
    }
    float* Sl = S + static_cast<size_t>(l) * Q * F;
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int fo = fb + 16 * e;
        if (fo >= F) continue;
#pragma unroll
        for (int G = 0; G < kQ4TileG; G++) {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int q = 8 * (G0 + G) + 2 * gl + j;
                if (G < nG && q < Q) Sl[static_cast<size_t>(q) * F + fo] = acc[e][G][j];
            }
        }
    }
}

// ── top-k ──────────────────────────────────────────────────────────────────
// Row views of the selection kernels.  C > 1 (chunks): output row i is chunk i % C of
// input row i / C, elements [chunk (i % C), min(n, chunk (i % C + 1))), indices relative to
// the chunk.  cand set (a selection over chunk candidates): output index p of row i is
// written as (p / ck) chunk + cand[i * crow + p], the row index of candidate p.
struct TopkView {
    int C = 1, chunk = 0;
    const uint32_t* cand = nullptr;
    int ck = 0, crow = 0;
};
__device__ __forceinline__ uint32_t topk_out_index(const TopkView& v, size_t row, uint32_t p) {
    return v.cand ? (p / v.ck) * static_cast<uint32_t>(v.chunk) + v.cand[row * v.crow + p] : p;
}

// Order key: (k32(score) descending, index ascending) as one 64-bit composite
// c = k32 << 32 | (0xFFFFFFFF - index), unique per element.  k32 is the f32 bit
// pattern of |s| (abs mode; -0 and +0 equal), or an order-preserving map of s
// (signed mode).  A radix select over 8-bit digits of c (8 passes) finds the k-th
// largest composite exactly; the k elements at or above it are ranked and written.
// (The sign mode is a template parameter, not a run-time flag: a branch per element
// between a load and its use makes the compiler wait for each load before issuing the
// next.)  k32 is order_key<SG> (knn.h).

// Inclusive scan of one value per lane over the wave (DPP within rows of 16, then the
// row totals through SGPRs).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    const int lane = threadIdx.x & 63;
    v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    const uint32_t r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
                   r2 = __builtin_amdgcn_readlane(v, 47);
    const int row = lane >> 4;
    return v + (row >= 1 ? r0 : 0u) + (row >= 2 ? r1 : 0u) + (row >= 3 ? r2 : 0u);
}

// Radix select of the k-th largest 32-bit key among the values every thread visits
// (gen(visit) makes the same visits in every pass): four passes of 8-bit digits.
// Returns the key; *above = number of visited values strictly greater than it.
template <class Gen>
__device__ __forceinline__ uint32_t select_kth32(int k, Gen gen, uint32_t (*hist)[256], uint32_t* sel, int* above) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t prefix = 0, pmask = 0;
    int remaining = k;
    for (int pass = 0; pass < 4; pass++) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < (kThreads / 64) * 256; i += kThreads) (&hist[0][0])[i] = 0u;
        __syncthreads();
        gen([&](uint32_t c) __attribute__((always_inline)) {
            if ((c & pmask) == prefix) atomicAdd(&hist[wave][(c >> shift) & 0xFF], 1u);
        });
        __syncthreads();
        if (wave == 0) {
            // lane covers digits 255 - 4 lane .. 252 - 4 lane (descending)
            uint32_t h[4], tot = 0;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int dgt = 255 - 4 * lane - u;
                h[u] = hist[0][dgt] + hist[1][dgt] + hist[2][dgt] + hist[3][dgt];
                tot += h[u];
            }
            const uint32_t incl = wave_incl_scan(tot);
            const uint32_t excl = incl - tot;
            if (excl < static_cast<uint32_t>(remaining) && incl >= static_cast<uint32_t>(remaining)) {
                uint32_t cum = excl;
                int dsel = 0, rem = remaining;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    if (cum + h[u] >= static_cast<uint32_t>(remaining)) {
                        dsel = 255 - 4 * lane - u;
                        rem = remaining - static_cast<int>(cum);
                        break;
                    }
                    cum += h[u];
                }
                sel[0] = prefix | (static_cast<uint32_t>(dsel) << shift);
                sel[1] = static_cast<uint32_t>(rem);
            }
        }
        __syncthreads();
        prefix = sel[0];
        remaining = static_cast<int>(sel[1]);
        pmask |= 0xFFu << shift;
        __syncthreads();
    }
    *above = k - remaining;
    return prefix;
}

constexpr int kTopkCap = 2048;  // candidates kept in LDS

// One workgroup per row.  Order: key descending, index ascending (the composite
// key << 32 | (0xFFFFFFFF - index), unique per element).  T, the k-th largest of the 256
// per-thread maximum keys, is a lower bound of the k-th largest key (k distinct threads
// hold an element >= T; with k above the thread count T = 0), so the elements with
// key >= T are compacted into LDS (the score magnitudes of a row share their top key
// bits: a select over every element would spend its passes on them) and the exact select
// runs there: the k-th largest key K, every element above it, then the elements equal to
// K in index order — when more of them tie than are needed, a second select over their
// indices finds the largest index kept, so ties cost linear time however many there are
// (an all-zero row is one big tie).  Rows whose candidates overflow the LDS list run the
// selects over all elements instead.  k <= n; the output rows are kstride apart and
// slots k .. kstride - 1 receive index 0xFFFFFFFF and score 0.
// v: the row view (TopkView).
template <int PER, bool SG>
__global__ __launch_bounds__(kThreads) void topk_kernel(const float* __restrict__ S, size_t row_stride, int n, int k,
                                                        int kstride, uint32_t* __restrict__ idx_out,
                                                        float* __restrict__ val_out, TopkView v) {
    __shared__ uint32_t hist[kThreads / 64][256];
    __shared__ uint32_t sel[2];
    __shared__ int cnt, nout, nties;
    __shared__ uint32_t ckey[kTopkCap], cidx[kTopkCap];
    __shared__ uint64_t out_c[kTopkMaxK];
    __shared__ float out_v[kTopkMaxK];
    const int tid = threadIdx.x;
    const float* __restrict__ s = S + static_cast<size_t>(blockIdx.x) * row_stride;
    if (v.C > 1) {
        const int r = blockIdx.x / v.C, c = blockIdx.x - r * v.C;
        s = S + static_cast<size_t>(r) * row_stride + static_cast<size_t>(c) * v.chunk;
        n = min(v.chunk, n - c * v.chunk);
        k = min(k, n);
    }
    // element i = tid + kThreads * j (coalesced); held in registers when PER > 0
    uint32_t key[PER > 0 ? PER : 1];
    if constexpr (PER > 0) {
        // clamped, unpredicated loads first (all in flight together), then the keys
#pragma unroll
        for (int j = 0; j < PER; j++) key[j] = __float_as_uint(s[min(tid + kThreads * j, n - 1)]);
#pragma unroll
        for (int j = 0; j < PER; j++)
            key[j] = tid + kThreads * j < n ? order_key<SG>(__uint_as_float(key[j])) : 0u;
    }
    const int nper = (n + kThreads - 1) / kThreads;
    // f(key, i) for this thread's elements i = tid + kThreads * j < n
    auto each = [&](auto f) __attribute__((always_inline)) {
        if constexpr (PER > 0) {
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int i = tid + kThreads * j;
                if (i < n) f(key[j], i);
            }
        } else {
            for (int j = 0; j < nper; j++) {
                const int i = tid + kThreads * j;
                if (i >= n) break;
                f(order_key<SG>(s[i]), i);
            }
        }
    };

    // 1. T: the k-th largest per-thread maximum key (threads without elements do not vote)
    uint32_t T = 0;
    int above = 0;
    if (k <= kThreads) {
        uint32_t kmax = 0;
        bool has = false;
        each([&](uint32_t kk, int) __attribute__((always_inline)) {
            kmax = max(kmax, kk);
            has = true;
        });
        T = select_kth32(
            k, [&](auto visit) __attribute__((always_inline)) { if (has) visit(kmax); }, hist, sel, &above);
    }

    // 2. candidates (key >= T) into LDS
    if (tid == 0) {
        cnt = 0;
        nout = 0;
        nties = 0;
    }
    __syncthreads();
    each([&](uint32_t kk, int i) __attribute__((always_inline)) {
        if (kk >= T) {
            const int p = atomicAdd(&cnt, 1);
            if (p < kTopkCap) {
                ckey[p] = kk;
                cidx[p] = static_cast<uint32_t>(i);
            }
        }
    });
    __syncthreads();
    const int nc = cnt;
    const bool inlds = nc <= kTopkCap;
    // g(key, index) over the candidates: the LDS list, or every element of the row
    auto cands = [&](auto g) __attribute__((always_inline)) {
        if (inlds) {
            for (int p = tid; p < nc; p += kThreads) g(ckey[p], cidx[p]);
        } else {
            each([&](uint32_t kk, int i) __attribute__((always_inline)) { g(kk, static_cast<uint32_t>(i)); });
        }
    };

    // 3. K = the k-th largest key; `above` elements are strictly greater
    const uint32_t K = select_kth32(
        k,
        [&](auto visit) __attribute__((always_inline)) {
            cands([&](uint32_t kk, uint32_t) __attribute__((always_inline)) { visit(kk); });
        },
        hist, sel, &above);

    // 4. the k winners: every key > K, then the (k - above) lowest indices with key == K.
    // imax = the largest index kept among the ties (all of them when no more tie than needed).
    const int need = k - above;
    int mine = 0;
    cands([&](uint32_t kk, uint32_t) __attribute__((always_inline)) { mine += kk == K; });
    if (mine) atomicAdd(&nties, mine);
    __syncthreads();
    uint32_t imax = 0xFFFFFFFFu;
    if (nties > need) {
        int above2 = 0;
        const uint32_t r = select_kth32(
            need,
            [&](auto visit) __attribute__((always_inline)) {
                cands([&](uint32_t kk, uint32_t i) __attribute__((always_inline)) {
                    if (kk == K) visit(0xFFFFFFFFu - i);
                });
            },
            hist, sel, &above2);
        imax = 0xFFFFFFFFu - r;
    }
    cands([&](uint32_t kk, uint32_t i) __attribute__((always_inline)) {
        if (kk > K || (kk == K && i <= imax)) {
            const int p = atomicAdd(&nout, 1);
            out_c[p] = (static_cast<uint64_t>(kk) << 32) | (0xFFFFFFFFu - i);
            out_v[p] = s[i];
        }
    });
    __syncthreads();
    const size_t row0 = static_cast<size_t>(blockIdx.x) * kstride;
    for (int p = tid; p < k; p += kThreads) {
        const uint64_t me = out_c[p];
        int rank = 0;
        for (int j = 0; j < k; j++) rank += out_c[j] > me;
        idx_out[row0 + rank] = topk_out_index(v, blockIdx.x, 0xFFFFFFFFu - static_cast<uint32_t>(me & 0xFFFFFFFFu));
        val_out[row0 + rank] = out_v[p];
    }
    for (int p = k + tid; p < kstride; p += kThreads) {
        idx_out[row0 + p] = 0xFFFFFFFFu;
        val_out[row0 + p] = 0.0f;
    }
}

// ── top-k, one wave per row ────────────────────────────────────────────────
// Rows of n <= 64 PW elements with k <= 64.  Each wave owns one row (element i = lane +
// 64 j in register j) and runs without workgroup barriers, so a CU works on many rows at
// once instead of one.  Same order and result as topk_kernel:
//   1. T = the k-th largest of the 64 lane maxima: k distinct lanes hold an element >= T,
//      so T bounds the k-th largest key from below;
//   2. the elements with key >= T go to the wave's LDS list (a wave scan of the lanes'
//      counts gives each lane its slots);
//   3. K = the k-th largest key of the list; `above` keys exceed it;
//   4. ties at K are kept in index order: imax = the (k - above)-th smallest tie index;
//   5. the k winners are ranked by (key descending, index ascending) and written.
// A row whose list would overflow (many equal keys) runs steps 3-4 over its registers.
// Every k-th-largest search is a radix descent over the 32 key bits with wave ballots.
// Register slots past n hold key 0 with an index >= n: with k <= n they rank below k
// real elements (no key is below 0, and ties go to the smaller index), so they take
// part in every step without a validity test.
constexpr int kWCap = 512;      // list entries per wave
constexpr int kWSmallK = 8;     // k up to this (and rows up to 4096) take k rounds of a wave arg-max
constexpr int kWWaves = 4;      // rows per workgroup

__device__ __forceinline__ uint64_t wave_ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }
__device__ __forceinline__ int wave_popc(bool p) { return __builtin_popcountll(wave_ballot(p)); }
// Set bits of m below this lane.
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
}

// The k-th largest of the values v[t] with ok[t] over the wave (the largest x that at
// least k of them reach); 0 when fewer than k are valid.  Wave-uniform.
template <int R, class V, class Ok>
__device__ __forceinline__ uint32_t wave_kth_largest(V v, Ok ok, int k) {
    uint32_t prefix = 0;
    for (int b = 31; b >= 0; b--) {
        const uint32_t c = prefix | (1u << b);
        int cnt = 0;
#pragma unroll
        for (int t = 0; t < R; t++) cnt += wave_popc(ok(t) && v(t) >= c);
        if (cnt >= k) prefix = c;
    }
    return prefix;
}

// 64-bit wave maximum: DPP butterflies within rows of 16 lanes, then the four row results.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v)), CTRL, 0xF, 0xF, false));
    const uint32_t hi = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v >> 32)), CTRL, 0xF, 0xF, false));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), l));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), l));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    v = max(v, dpp_u64<0xB1>(v));   // quad_perm 1,0,3,2
    v = max(v, dpp_u64<0x4E>(v));   // quad_perm 2,3,0,1
    v = max(v, dpp_u64<0x141>(v));  // row_half_mirror
    v = max(v, dpp_u64<0x140>(v));  // row_mirror
    return max(max(readlane_u64(v, 0), readlane_u64(v, 16)), max(readlane_u64(v, 32), readlane_u64(v, 48)));
}

template <int PW, bool SG>
__global__ __launch_bounds__(64 * kWWaves) void topk_wave_kernel(const float* __restrict__ S, size_t row_stride,
                                                                 int n, int k, int kstride,
                                                                 uint32_t* __restrict__ idx_out,
                                                                 float* __restrict__ val_out, int rows,
                                                                 TopkView v) {
    __shared__ uint32_t lkey[kWWaves][kWCap], lidx[kWWaves][kWCap];
    __shared__ uint32_t wkey[kWWaves][64], widx[kWWaves][64];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row = blockIdx.x * kWWaves + w;
    if (row >= rows) return;  // whole wave; the kernel has no workgroup barrier
    const float* __restrict__ s = S + static_cast<size_t>(row) * row_stride;
    if (v.C > 1) {  // chunk view, as topk_kernel
        const int r = row / v.C, c = row - r * v.C;
        s = S + static_cast<size_t>(r) * row_stride + static_cast<size_t>(c) * v.chunk;
        n = min(v.chunk, n - c * v.chunk);
        k = min(k, n);
    }
    uint32_t key[PW];
    if (n == 64 * PW) {  // every register holds an element: one base, immediate offsets
        const float* __restrict__ sl = s + lane;
#pragma unroll
        for (int j = 0; j < PW; j++) key[j] = order_key<SG>(sl[64 * j]);
    } else {
        // raw buffer loads over exactly the row's n floats (offsets past it read 0; the
        // whole offset is in the vector operand, which the range check covers), all in
        // flight together, then the keys; the mask is all ones for i < n, zero past the row
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(s), 0, n * static_cast<int>(sizeof(float)), 0x00020000);
#pragma unroll
        for (int j = 0; j < PW; j++) key[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * lane + 256 * j, 0, 0);
#pragma unroll
        for (int j = 0; j < PW; j++) {
            const uint32_t live = static_cast<uint32_t>((lane + 64 * j - n) >> 31);
            key[j] = order_key<SG>(__uint_as_float(key[j])) & live;
        }
    }
    // element index of register j; the opaque copy of the lane keeps the compiler from
    // holding one index register per j
    auto index_of = [&](int j) __attribute__((always_inline)) {
        int l = lane;
        asm volatile("" : "+v"(l));
        return static_cast<uint32_t>(l + 64 * j);
    };
    auto all = [](int) { return true; };

    if (PW <= 64 && k <= kWSmallK) {
        // A few winners: round r takes the largest composite key << 32 | ~index below the
        // previous winner (composites are unique per element, so nothing is taken twice);
        // slots past n hold key 0 with an index >= n, below every real element.
        uint64_t win[kWSmallK];
        uint64_t prev = ~uint64_t{0};
#pragma unroll
        for (int r = 0; r < kWSmallK; r++) {
            if (r >= k) break;  // wave-uniform
            uint64_t best = 0;
#pragma unroll
            for (int j = 0; j < PW; j++) {
                const uint64_t c = (static_cast<uint64_t>(key[j]) << 32) | (0xFFFFFFFFu - index_of(j));
                if (c < prev && c > best) best = c;
            }
            prev = wave_max_u64(best);
            win[r] = prev;
        }
        const size_t row0 = static_cast<size_t>(row) * kstride;
        uint64_t mine = 0;
#pragma unroll
        for (int r = 0; r < kWSmallK; r++)
            if (r == lane) mine = win[r];
        if (lane < k) {
            const uint32_t mi = 0xFFFFFFFFu - static_cast<uint32_t>(mine);
            idx_out[row0 + lane] = topk_out_index(v, row, mi);
            val_out[row0 + lane] = s[mi];
        }
        for (int p = k + lane; p < kstride; p += 64) {
            idx_out[row0 + p] = 0xFFFFFFFFu;
            val_out[row0 + p] = 0.0f;
        }
        return;
    }

    // 1. T from the lane maxima
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < PW; j++) m = max(m, key[j]);
    const uint32_t T = wave_kth_largest<1>([&](int) { return m; }, all, k);

    // 2. the list of keys >= T (slots past the capacity are not written)
    int total = 0;
#pragma unroll
    for (int j = 0; j < PW; j++) {
        const bool c = key[j] >= T;
        const uint64_t b = wave_ballot(c);
        if (b) {  // wave-uniform
            const int q = total + lanes_below(b);
            if (c && q < kWCap) {
                lkey[w][q] = key[j];
                lidx[w][q] = index_of(j);
            }
            total += __builtin_popcountll(b);
        }
    }
    uint32_t K, imax = 0xFFFFFFFFu;
    int nwin = 0;
    if (total <= kWCap) {
        // the wave reads what its own lanes wrote: keep the LDS accesses in program order
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        constexpr int R = kWCap / 64;
        uint32_t ck[R], ci[R];
#pragma unroll
        for (int t = 0; t < R; t++) {
            const int q = lane + 64 * t;
            ck[t] = q < total ? lkey[w][q] : 0u;
            ci[t] = q < total ? lidx[w][q] : 0u;
        }
        auto cok = [&](int t) __attribute__((always_inline)) { return lane + 64 * t < total; };
        // 3. K and the keys above it
        K = wave_kth_largest<R>([&](int t) { return ck[t]; }, cok, k);
        int above = 0, nt = 0;
#pragma unroll
        for (int t = 0; t < R; t++) {
            above += wave_popc(cok(t) && ck[t] > K);
            nt += wave_popc(cok(t) && ck[t] == K);
        }
        // 4. the (k - above) smallest tie indices: the largest kept is the need-th largest
        // of the complemented indices
        const int need = k - above;
        if (nt > need)
            imax = ~wave_kth_largest<R>([&](int t) { return ~ci[t]; },
                                         [&](int t) { return cok(t) && ck[t] == K; }, need);
        // 5. the winners to the wave's winner list
#pragma unroll
        for (int t = 0; t < R; t++) {
            const bool win = cok(t) && (ck[t] > K || (ck[t] == K && ci[t] <= imax));
            const uint64_t b = wave_ballot(win);
            if (win) {
                const int q = nwin + lanes_below(b);
                wkey[w][q] = ck[t];
                widx[w][q] = ci[t];
            }
            nwin += __builtin_popcountll(b);
        }
    } else {
        // 3-4 over the keys in the registers (rows with many equal keys): K by four 8-bit
        // radix passes with a wave histogram in LDS, then the ties in index order (j, then
        // lane) and the winners, one sweep each.
        uint32_t* hist = lkey[w];  // 256 bins
        uint32_t prefix = 0, pmask = 0;
        int remaining = k;
        for (int pass = 0; pass < 4; pass++) {
            const int shift = 24 - 8 * pass;
#pragma unroll
            for (int u = 0; u < 4; u++) hist[lane + 64 * u] = 0u;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int j = 0; j < PW; j++)
                if ((key[j] & pmask) == prefix) atomicAdd(&hist[(key[j] >> shift) & 0xFFu], 1u);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // lane covers digits 255 - 4 lane .. 252 - 4 lane (descending)
            uint32_t h[4], tot = 0;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                h[u] = hist[255 - 4 * lane - u];
                tot += h[u];
            }
            const uint32_t inc = wave_incl_scan(tot), exc = inc - tot;
            const bool here = exc < static_cast<uint32_t>(remaining) && inc >= static_cast<uint32_t>(remaining);
            uint32_t dsel = 0, rem = 0, cum = exc;
            bool found = false;
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (here && !found && cum + h[u] >= static_cast<uint32_t>(remaining)) {
                    dsel = 255 - 4 * lane - u;
                    rem = static_cast<uint32_t>(remaining) - cum;
                    found = true;
                }
                cum += h[u];
            }
            const uint64_t at = wave_ballot(here);
            const int src = __builtin_ctzll(at);
            prefix |= static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(dsel), src)) << shift;
            remaining = __builtin_amdgcn_readlane(static_cast<int>(rem), src);
            pmask |= 0xFFu << shift;
            // the histogram's area is rewritten by the next pass
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        K = prefix;
        const int need = remaining;  // ties kept; k - need keys exceed K
        // the two sweeps read the keys again from memory, eight registers at a time (a
        // loop over the register array would need a ballot per register, all unrolled)
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(s), 0, n * static_cast<int>(sizeof(float)), 0x00020000);
        auto load8 = [&](int j0, uint32_t (&kk)[8]) __attribute__((always_inline)) {
#pragma unroll
            for (int u = 0; u < 8; u++) kk[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, 4 * (lane + 64 * (j0 + u)), 0, 0);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t live = static_cast<uint32_t>((lane + 64 * (j0 + u) - n) >> 31);
                kk[u] = order_key<SG>(__uint_as_float(kk[u])) & live;
            }
        };
        int run = 0;
        for (int j0 = 0; j0 < PW && run < need; j0 += 8) {
            uint32_t kk[8];
            load8(j0, kk);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const bool tie = kk[u] == K;
                const uint64_t b = wave_ballot(tie);
                const int c = __builtin_popcountll(b);
                if (run < need && run + c >= need) {  // wave-uniform
                    const uint64_t at = wave_ballot(tie && lanes_below(b) == need - run - 1);
                    imax = static_cast<uint32_t>(__builtin_ctzll(at) + 64 * (j0 + u));
                }
                run += c;
            }
        }
        for (int j0 = 0; j0 < PW; j0 += 8) {
            uint32_t kk[8];
            load8(j0, kk);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const uint32_t i = static_cast<uint32_t>(lane + 64 * (j0 + u));
                const bool win = kk[u] > K || (kk[u] == K && i <= imax);
                const uint64_t b = wave_ballot(win);
                if (win) {
                    const int q = nwin + lanes_below(b);
                    wkey[w][q] = kk[u];
                    widx[w][q] = i;
                }
                nwin += __builtin_popcountll(b);
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // 5. rank the k winners: key descending, index ascending
    const size_t row0 = static_cast<size_t>(row) * kstride;
    if (lane < k) {
        const uint32_t mk = wkey[w][lane], mi = widx[w][lane];
        int rank = 0;
        for (int j = 0; j < k; j++) {
            const uint32_t ok = wkey[w][j], oi = widx[w][j];
            rank += (ok > mk || (ok == mk && oi < mi)) ? 1 : 0;
        }
        idx_out[row0 + rank] = topk_out_index(v, row, mi);
        val_out[row0 + rank] = s[mi];
    }
    for (int p = k + lane; p < kstride; p += 64) {
        idx_out[row0 + p] = 0xFFFFFFFFu;
        val_out[row0 + p] = 0.0f;
    }
}

}  // namespace

void launch_gate_scores_f32(const KnnLayers& g, int n_layers, const float* X, float* S, int F, int K, int Q,
                            hipStream_t s) {
    if (K % kF32Ks) fail(LARQL_HIP_ERR_INVALID, "gate scores: hidden must be a multiple of 16");
    const dim3 grid((F + kF32TileF - 1) / kF32TileF, (Q + kF32TileQ - 1) / kF32TileQ, n_layers);
    gate_scores_f32_kernel<<<grid, dim3(kThreads), 0, s>>>(g, X, S, F, K, Q);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_gate_scores_q4(const KnnLayers& nib, const KnnLayers& scales, int n_layers, const int8_t* X8,
                           const float* XS, uint4* XA, float* XSP, float* S, int F, int K, int Q, hipStream_t s) {
    if (K % 64) fail(LARQL_HIP_ERR_INVALID, "gate scores: Q4_0 hidden must be a multiple of 64");
    const int ng = (Q + 7) / 8;
    const size_t nxa = static_cast<size_t>(K / 64) * ng * 64;
    q4_xa_kernel<<<dim3(static_cast<unsigned>((nxa + 255) / 256)), dim3(256), 0, s>>>(X8, XS, XA, XSP, K, Q, ng);
    LARQL_HIP_CHECK(hipGetLastError());
    const dim3 grid((F + kQ4TileF - 1) / kQ4TileF, (ng + kQ4TileG - 1) / kQ4TileG, n_layers);
    gate_scores_q4_kernel<<<grid, dim3(kThreads), 0, s>>>(nib, scales, XA, XSP, S, F, K, Q, ng);
    LARQL_HIP_CHECK(hipGetLastError());
}

size_t q4_xa_bytes(int K, int Q) { return static_cast<size_t>(K / 64) * ((Q + 7) / 8) * 64 * sizeof(uint4); }
size_t q4_xsp_bytes(int K, int Q) { return static_cast<size_t>(K / 64) * ((Q + 7) / 8) * 16 * sizeof(float); }

// The selection kernels over `nrows` rows (v.C > 1: chunk views, rows = input rows x C) of
// at most nmax elements, k requested per row (kstride output slots).
static void topk_select(const float* S, size_t nrows, size_t row_stride, int n, int nmax, int k, int kstride,
                        const TopkView& v, int signed_mode, uint32_t* idx, float* val, hipStream_t s) {
    const int ke = std::min(k, nmax);  // top_k.min(len), LV/src/index/walk.rs:569 (per chunk in the kernels)
    auto go = [&](auto sg) {
        constexpr bool SG = decltype(sg)::value;
        const dim3 grid(static_cast<unsigned>(nrows));
        if (ke <= 64 && nmax <= 64 * 224 && nrows <= 0x7FFFFFFF) {  // a wave per row
            const dim3 gw(static_cast<unsigned>((nrows + kWWaves - 1) / kWWaves)), bw(64 * kWWaves);
            const int r = static_cast<int>(nrows);
            // register slots per lane: the fewest that hold the row (every slot costs time)
            if (nmax <= 64 * 4)
                topk_wave_kernel<4, SG><<<gw, bw, 0, s>>>(S, row_stride, n, ke, kstride, idx, val, r, v);
            else if (nmax <= 64 * 16)
                topk_wave_kernel<16, SG><<<gw, bw, 0, s>>>(S, row_stride, n, ke, kstride, idx, val, r, v);
            else if (nmax <= 64 * 64)
                topk_wave_kernel<64, SG><<<gw, bw, 0, s>>>(S, row_stride, n, ke, kstride, idx, val, r, v);
            else if (nmax <= 64 * 160)
                topk_wave_kernel<160, SG><<<gw, bw, 0, s>>>(S, row_stride, n, ke, kstride, idx, val, r, v);
            else
                topk_wave_kernel<224, SG><<<gw, bw, 0, s>>>(S, row_stride, n, ke, kstride, idx, val, r, v);
        } else if (nmax <= kThreads * 48) {
            topk_kernel<48, SG><<<grid, dim3(kThreads), 0, s>>>(S, row_stride, n, ke, kstride, idx, val, v);
        } else {
            topk_kernel<0, SG><<<grid, dim3(kThreads), 0, s>>>(S, row_stride, n, ke, kstride, idx, val, v);
        }
    };
    if (signed_mode) go(std::true_type{});
    else go(std::false_type{});
    LARQL_HIP_CHECK(hipGetLastError());
}

// Long rows are split into chunks whose selection runs in registers: 1024 elements for k
// <= 64 (a wave per chunk), 12288 above; a row of n elements has C = ceil(n / chunk).
static int topk_chunk_len(int k) { return k <= 64 ? 1024 : kThreads * 48; }
static bool topk_chunked(int n, int k) { return n > (k <= 64 ? 64 * 224 : kThreads * 48); }

size_t topk_candidate_slots(size_t rows, int n, int k) {
    if (!topk_chunked(n, k)) return 0;
    const int chunk = topk_chunk_len(k);
    return rows * static_cast<size_t>((n + chunk - 1) / chunk) * static_cast<size_t>(k);
}

namespace {
// Slots a chunk left empty (index 0xFFFFFFFF) take the lowest key of the signed order, so
// the second selection ranks them after every real score (in abs mode their 0 is already
// the lowest key, and they sit after all real candidates of the row).
__global__ void topk_cand_fix_kernel(const uint32_t* __restrict__ ci, float* __restrict__ cv, size_t n) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i < n && ci[i] == 0xFFFFFFFFu) cv[i] = -INFINITY;
}
}  // namespace

void launch_topk(const float* S, size_t rows, size_t row_stride, int n, int k, int signed_mode, uint32_t* idx,
                 float* val, hipStream_t s, uint32_t* cand_idx, float* cand_val) {
    if (k < 1 || k > kTopkMaxK || n < 1) fail(LARQL_HIP_ERR_INVALID, "top-k: need 1 <= k <= 512 and n >= 1");
    if (rows == 0) return;
    if (!cand_idx || !cand_val || !topk_chunked(n, k)) {
        topk_select(S, rows, row_stride, n, n, k, k, TopkView{}, signed_mode, idx, val, s);
        return;
    }
    // Stage 1: the top k of every chunk, [rows][C][k] candidates with chunk-relative
    // indices.  Stage 2: the top k of each row's C k candidates.  An element of a row's top
    // k is within its chunk's top k (else k elements of its chunk outrank it), and the
    // candidates sit in chunk order, each chunk's in rank order, so equal keys still
    // resolve by ascending row index.
    const int chunk = topk_chunk_len(k), C = (n + chunk - 1) / chunk;
    TopkView v1;
    v1.C = C;
    v1.chunk = chunk;
    topk_select(S, rows * C, row_stride, n, chunk, k, k, v1, signed_mode, cand_idx, cand_val, s);
    const size_t nc = rows * static_cast<size_t>(C) * k;
    if (signed_mode && n % chunk != 0 && n % chunk < k) {
        topk_cand_fix_kernel<<<dim3(static_cast<unsigned>((nc + 255) / 256)), dim3(256), 0, s>>>(cand_idx, cand_val, nc);
        LARQL_HIP_CHECK(hipGetLastError());
    }
    TopkView v2;  // candidate positions written as row indices
    v2.chunk = chunk;
    v2.cand = cand_idx;
    v2.ck = k;
    v2.crow = C * k;
    topk_select(cand_val, rows, static_cast<size_t>(C) * k, C * k, C * k, k, k, v2, signed_mode, idx, val, s);
}

}  // namespace larql
