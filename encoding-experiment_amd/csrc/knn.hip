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

// ── Q4_0 x Q8 scores ───────────────────────────────────────────────────────
// Workgroup tile: 64 features x 128 queries; thread tile 8 features x 4 queries.
// Each LDS stage holds two 32-element blocks: the features' nibble bytes and f16
// scales, and the queries' int8 blocks re-laid out as even / odd element dwords
// (matching lo / hi nibbles), their f32 scales and their element sums (for the -8
// offset: isum = sum(nib * x) - 8 sum(x), exact).
constexpr int kQ4TileF = 64, kQ4TileQ = 128, kQ4Bps = 2;

__device__ __forceinline__ uint32_t pick4(uint32_t a, uint32_t b, uint32_t sel) {
    return __builtin_amdgcn_perm(b, a, sel);
}

__global__ __launch_bounds__(kThreads, 2) void gate_scores_q4_kernel(KnnLayers g, KnnLayers gd, const int8_t* __restrict__ X8,
                                                                  const float* __restrict__ XS, float* __restrict__ S,
                                                                  int F, int K, int Q) {
    __shared__ uint4 Gn[2][kQ4Bps][kQ4TileF];        // nibble bytes
    __shared__ float Gd[2][kQ4Bps][kQ4TileF];        // decoded scales
    __shared__ uint4 Xb[2][kQ4Bps][kQ4TileQ][2];     // even dwords, odd dwords
    __shared__ float Xsc[2][kQ4Bps][kQ4TileQ];
    __shared__ int Xsum[2][kQ4Bps][kQ4TileQ];
    const int l = blockIdx.z;
    const uint8_t* __restrict__ nib = static_cast<const uint8_t*>(g.p[l]);
    const uint16_t* __restrict__ dsc = static_cast<const uint16_t*>(gd.p[l]);
    const int f0 = blockIdx.x * kQ4TileF, q0 = blockIdx.y * kQ4TileQ;
    const int tid = threadIdx.x;
    const int tf = tid >> 5, tq = tid & 31;  // features f0 + 8 tf .., queries q0 + 4 tq ..
    const int nb = K / 32;
    // global -> LDS mapping: features: threads 0..127 -> (block tid >> 6, feature tid & 63);
    // queries: all 256 threads -> (block tid >> 7, query tid & 127)
    const int gfb = (tid >> 6) & 1, gff = tid & 63;
    const size_t grow = static_cast<size_t>(min(f0 + gff, F - 1));
    const int xqb = tid >> 7, xqq = tid & 127;
    const size_t xrow = static_cast<size_t>(min(q0 + xqq, Q - 1));
    uint4 gr = make_uint4(0, 0, 0, 0);
    uint16_t gdr = 0;
    uint4 xr0, xr1;
    float xsr;
    auto gload = [&](int b0) __attribute__((always_inline)) {
        if (tid < 128) {
            const int b = b0 + gfb;
            gr = *reinterpret_cast<const uint4*>(nib + grow * (K / 2) + static_cast<size_t>(b) * 16);
            gdr = dsc[grow * nb + b];
        }
        const int b = b0 + xqb;
        const uint4* xp = reinterpret_cast<const uint4*>(X8 + xrow * K + static_cast<size_t>(b) * 32);
        xr0 = xp[0];
        xr1 = xp[1];
        xsr = XS[xrow * nb + b];
    };
    auto lstore = [&](int s) __attribute__((always_inline)) {
        if (tid < 128) {
            Gn[s][gfb][gff] = gr;
            Gd[s][gfb][gff] = h2f(gdr);
        }
        // natural order dwords w0..w7 hold elements 4w..4w+3; even dword i needs elements
        // 8i, 8i+2, 8i+4, 8i+6 = bytes 0, 2 of w(2i) and bytes 0, 2 of w(2i+1)
        const uint32_t w[8] = {xr0.x, xr0.y, xr0.z, xr0.w, xr1.x, xr1.y, xr1.z, xr1.w};
        uint32_t ev[4], od[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            ev[i] = pick4(w[2 * i], w[2 * i + 1], 0x06040200u);
            od[i] = pick4(w[2 * i], w[2 * i + 1], 0x07050301u);
        }
        int sum = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) sum = __builtin_amdgcn_sdot4(static_cast<int>(w[i]), 0x01010101, sum, false);
        Xb[s][xqb][xqq][0] = make_uint4(ev[0], ev[1], ev[2], ev[3]);
        Xb[s][xqb][xqq][1] = make_uint4(od[0], od[1], od[2], od[3]);
        Xsc[s][xqb][xqq] = xsr;
        Xsum[s][xqb][xqq] = sum;
    };

    float acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.f;

    const int ns = nb / kQ4Bps;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int st = 0; st < ns; st++) {
        const int s = st & 1;
        if (st + 1 < ns) gload((st + 1) * kQ4Bps);
#pragma unroll
        for (int bb = 0; bb < kQ4Bps; bb++) {
            // the four queries' x words, then one feature at a time
            uint32_t ew[4][4], ow[4][4];
            float xs[4];
            int off[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int qq = tq * 4 + j;
                const uint4 e = Xb[s][bb][qq][0], o = Xb[s][bb][qq][1];
                ew[j][0] = e.x; ew[j][1] = e.y; ew[j][2] = e.z; ew[j][3] = e.w;
                ow[j][0] = o.x; ow[j][1] = o.y; ow[j][2] = o.z; ow[j][3] = o.w;
                xs[j] = Xsc[s][bb][qq];
                off[j] = 8 * Xsum[s][bb][qq];
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint4 v = Gn[s][bb][tf * 8 + i];
                const uint32_t vw[4] = {v.x, v.y, v.z, v.w};
                uint32_t lo[4], hi[4];
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    lo[w] = vw[w] & 0x0F0F0F0Fu;
                    hi[w] = (vw[w] >> 4) & 0x0F0F0F0Fu;
                }
                const float d = Gd[s][bb][tf * 8 + i];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int isum = 0;
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        isum = __builtin_amdgcn_sdot4(static_cast<int>(lo[w]), static_cast<int>(ew[j][w]), isum, false);
                        isum = __builtin_amdgcn_sdot4(static_cast<int>(hi[w]), static_cast<int>(ow[j][w]), isum, false);
                    }
                    // reference order: cs = f16(s) * q8s; acc += (float)isum * cs, product and
                    // sum rounded separately (fp contract is off in this file)
                    const float cs = d * xs[j];
                    const float prod = static_cast<float>(isum - off[j]) * cs;
                    acc[i][j] = acc[i][j] + prod;
                }
            }
        }
        if (st + 1 < ns) lstore(s ^ 1);
        __syncthreads();
    }
    float* Sl = S + static_cast<size_t>(l) * Q * F;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int q = q0 + tq * 4 + j;
        if (q >= Q) continue;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int f = f0 + tf * 8 + i;
            if (f < F) Sl[static_cast<size_t>(q) * F + f] = acc[i][j];
        }
    }
}

// ── top-k ──────────────────────────────────────────────────────────────────
// Order key: (k32(score) descending, index ascending) as one 64-bit composite
// c = k32 << 32 | (0xFFFFFFFF - index), unique per element.  k32 is the f32 bit
// pattern of |s| (abs mode; -0 and +0 equal), or an order-preserving map of s
// (signed mode).  A radix select over 8-bit digits of c (8 passes) finds the k-th
// largest composite exactly; the k elements at or above it are ranked and written.
__device__ __forceinline__ uint32_t order_key(float v, int signed_mode) {
    uint32_t b = __float_as_uint(v);
    if (!signed_mode) return b & 0x7FFFFFFFu;
    if ((b & 0x7FFFFFFFu) == 0) b = 0;  // -0 == +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int PER>
__global__ __launch_bounds__(kThreads) void topk_kernel(const float* __restrict__ S, size_t row_stride, int n, int k,
                                                        int signed_mode, uint32_t* __restrict__ idx_out,
                                                        float* __restrict__ val_out) {
    __shared__ uint32_t hist[kThreads / 64][256];
    __shared__ uint64_t sel_prefix;
    __shared__ int sel_remaining;
    __shared__ int cnt;
    __shared__ uint64_t cand_c[kTopkMaxK];
    __shared__ float cand_v[kTopkMaxK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* __restrict__ s = S + static_cast<size_t>(blockIdx.x) * row_stride;
    // element i = tid + kThreads * j (coalesced); held in registers when PER > 0
    uint32_t key[PER > 0 ? PER : 1];
    if constexpr (PER > 0) {
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const int i = tid + kThreads * j;
            key[j] = i < n ? order_key(s[i], signed_mode) : 0u;
        }
    }
    auto comp = [&](int j, int i) __attribute__((always_inline)) -> uint64_t {
        const uint32_t kk = PER > 0 ? key[j] : order_key(s[i], signed_mode);
        return (static_cast<uint64_t>(kk) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(i));
    };
    const int nper = PER > 0 ? PER : (n + kThreads - 1) / kThreads;

    uint64_t prefix = 0, pmask = 0;
    int remaining = k;
    for (int pass = 0; pass < 8; pass++) {
        const int shift = 56 - 8 * pass;
        for (int i = tid; i < (kThreads / 64) * 256; i += kThreads) (&hist[0][0])[i] = 0u;
        __syncthreads();
        for (int j = 0; j < nper; j++) {
            const int i = tid + kThreads * j;
            if (i >= n) break;
            const uint64_t c = comp(j, i);
            if ((c & pmask) == prefix) atomicAdd(&hist[wave][(c >> shift) & 0xFF], 1u);
        }
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
            // inclusive scan over lanes (descending digit order)
            uint32_t incl = tot;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t v = __shfl_up(incl, off, 64);
                if (lane >= off) incl += v;
            }
            const uint32_t excl = incl - tot;
            const bool here = excl < static_cast<uint32_t>(remaining) && incl >= static_cast<uint32_t>(remaining);
            if (here) {
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
                sel_prefix = prefix | (static_cast<uint64_t>(dsel) << shift);
                sel_remaining = rem;
            }
        }
        __syncthreads();
        prefix = sel_prefix;
        remaining = sel_remaining;
        pmask |= static_cast<uint64_t>(0xFF) << shift;
        __syncthreads();
    }
    // prefix is now the k-th largest composite: collect the k elements >= it
    if (tid == 0) cnt = 0;
    __syncthreads();
    for (int j = 0; j < nper; j++) {
        const int i = tid + kThreads * j;
        if (i >= n) break;
        const uint64_t c = comp(j, i);
        if (c >= prefix) {
            const int p = atomicAdd(&cnt, 1);
            if (p < kTopkMaxK) {
                cand_c[p] = c;
                cand_v[p] = s[i];
            }
        }
    }
    __syncthreads();
    if (tid < k) {
        const uint64_t me = cand_c[tid];
        int rank = 0;
        for (int j = 0; j < k; j++) rank += cand_c[j] > me;
        const size_t o = static_cast<size_t>(blockIdx.x) * k + rank;
        idx_out[o] = 0xFFFFFFFFu - static_cast<uint32_t>(me & 0xFFFFFFFFu);
        val_out[o] = cand_v[tid];
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
                           const float* XS, float* S, int F, int K, int Q, hipStream_t s) {
    if (K % (32 * kQ4Bps)) fail(LARQL_HIP_ERR_INVALID, "gate scores: Q4_0 hidden must be a multiple of 64");
    const dim3 grid((F + kQ4TileF - 1) / kQ4TileF, (Q + kQ4TileQ - 1) / kQ4TileQ, n_layers);
    gate_scores_q4_kernel<<<grid, dim3(kThreads), 0, s>>>(nib, scales, X8, XS, S, F, K, Q);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_topk(const float* S, size_t rows, size_t row_stride, int n, int k, int signed_mode, uint32_t* idx,
                 float* val, hipStream_t s) {
    if (k < 1 || k > kTopkMaxK || k > n) fail(LARQL_HIP_ERR_INVALID, "top-k: need 1 <= k <= min(n, 64)");
    if (rows == 0) return;
    const dim3 grid(static_cast<unsigned>(rows));
    if (n <= kThreads * 48) topk_kernel<48><<<grid, dim3(kThreads), 0, s>>>(S, row_stride, n, k, signed_mode, idx, val);
    else topk_kernel<0><<<grid, dim3(kThreads), 0, s>>>(S, row_stride, n, k, signed_mode, idx, val);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
