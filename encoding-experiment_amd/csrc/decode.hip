// Decode step: single-query GQA attention over the fp16 KV cache, the KV cache
// itself, the device-resident decoder model and the per-token kernel sequence.
//
// Per layer (Llama, pre-norm, LI/src/attention/block.rs:52-157, LI/src/forward/layer.rs:50-94;
// op order of the reference GPU decode LC/src/metal/decode.rs:144-715):
//   1. qkv   = [Wq|Wk|Wv] . rms_norm(h, input_norm)          fused norm + matvec
//   2. attn  = softmax(RoPE(q) . RoPE(K)^T * scale) . V      split over T + merge, this file
//              (the new K/V row is RoPE'd, rounded to fp16 and appended at pos)
//   3. h1    = h + Wo . attn                                  matvec + residual epilogue
//   4. act   = silu(Wg . n) * (Wu . n), n = rms_norm(h1)      fused norm + interleaved gate/up
//   5. h     = h1 + Wd . act                                  matvec + residual epilogue
// Six launches per layer (attention is two); the final norm + head is one more.
#include "decode.h"
#include "matvec_common.h"

#include <algorithm>
#include <type_traits>
#include <cmath>
#include <vector>

namespace larql {

constexpr int kAttnThreads = 256;
constexpr int kAttnChunk = 64;  // positions per workgroup

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Split-half RoPE of element d of head vector x (LI/src/attention/rope.rs:22-55):
// pairs (i, i + rdim/2), dims >= rdim untouched.  cs[i] = (cos, sin) of pair i.
__device__ __forceinline__ float rope_elem(const float* x, int d, int half, const float2* cs) {
    if (d < half) return x[d] * cs[d].x - x[d + half] * cs[d].y;
    if (d < 2 * half) return x[d - half] * cs[d - half].y + x[d] * cs[d - half].x;
    return x[d];
}

// Wave max / sum without LDS traffic: DPP butterflies inside each row of 16 lanes, then
// the four row results through SGPRs.  Every lane gets the result.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp<0xB1>(v));   // quad_perm 1,0,3,2
    v = fmaxf(v, dpp<0x4E>(v));   // quad_perm 2,3,0,1
    v = fmaxf(v, dpp<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp<0x140>(v));  // row_mirror
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

// Value of lane (this lane + R) within its row of 16 (row_shl:R).
template <int R>
__device__ __forceinline__ float from_lane_plus(float v) {
    return dpp<0x100 + R>(v);
}
__device__ __forceinline__ floatx4 add_lane_plus(floatx4 v, int reps) {
    floatx4 o = v;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float w;
        switch (reps) {
            case 1: w = from_lane_plus<1>(v[r]); break;
            case 2: w = from_lane_plus<2>(v[r]); break;
            case 3: w = from_lane_plus<3>(v[r]); break;
            case 4: w = from_lane_plus<4>(v[r]); break;
            case 5: w = from_lane_plus<5>(v[r]); break;
            case 6: w = from_lane_plus<6>(v[r]); break;
            case 7: w = from_lane_plus<7>(v[r]); break;
            default: w = from_lane_plus<8>(v[r]); break;
        }
        o[r] = v[r] + w;
    }
    return o;
}

__device__ __forceinline__ uint32_t f2_to_h2(float a, float b) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a))) |
           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(b))) << 16);
}

// Eight f32 values as fp16 pairs: the rounded value (part 0) or the rounding residue
// (part 1); the two parts sum to the value within 2^-22 of it.
__device__ __forceinline__ v4u split8(const float* x, int part) {
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float hi = static_cast<float>(static_cast<_Float16>(x[e]));
        y[e] = part ? x[e] - hi : hi;
    }
    return v4u{f2_to_h2(y[0], y[1]), f2_to_h2(y[2], y[3]), f2_to_h2(y[4], y[5]), f2_to_h2(y[6], y[7])};
}

// Grid (S, num_kv).  Workgroup (s, kvh) covers positions [t0, t0 + 64), t0 = t_begin
// rounded down to a multiple of 8, plus 64 s, for the reps = num_q / num_kv query heads
// of kv head kvh (GQA: kv_h = h / reps, LI/src/attention/gqa.rs:53).  Both products run
// on v_mfma_f32_16x16x32_f16 with f32 accumulation; the fp16 operands are exact: the
// cached K and V are fp16, and each f32 query element or probability is split into two
// fp16 parts, placed in two operand columns and summed after the product.
//   scores: D[t][col] = sum_d K[t][d] Qx[d][col], col = head (rounded part) or reps +
//           head (residue); wave w takes positions 16 w .. 16 w + 15 of the chunk.
//   P.V:    D[d][col] = sum_t Vt[d][t] Px[t][col]; wave w takes the 16-dim tiles
//           w, w + 4, ...; the V cache is stored as [t / 8][kv][hd][8] so that a lane's
//           eight consecutive positions of one dim are one 16-byte load.
// The row at pos = T - 1 comes from the fresh projections: RoPE'd, rounded to fp16 and
// written to the cache by the workgroup that owns it, which uses it from LDS.
// attn_combine_kernel merges the S softmax partials of each kv head's query heads.
// Prompt mode: this workgroup's query (grid z) and its view of the arguments.
__device__ __forceinline__ void attn_select_query(AttnArgs& a) {
    if (a.batch == 0) return;
    const int p = blockIdx.z;
    a.T += p;
    a.t_begin = (a.window > 0 && a.T > a.window) ? a.T - a.window : 0;
    a.qkv += static_cast<size_t>(p) * a.qkv_ld;
    a.part += static_cast<size_t>(p) * a.num_q * a.S * a.pst;
    a.out += static_cast<size_t>(p) * a.num_q * a.hd;
}

// o = sum_s e_s o_s / sum_s e_s l_s with e_s = exp(m_s - max_s m_s), in split order, for
// HD dims of nh consecutive query heads: partial entry (head h, split s) at
// base + (h sst + s) pst = {o[HD], ...}, its (m, l) pair mlo floats further, outputs at
// out + h HD.  One workgroup; ml holds 2 nh S floats of LDS.
// The loads of every (m, l) pair and of the first PF splits of each thread's first output
// pair are issued together, so for S <= PF (T <= 2176) the merge waits on memory once.
template <int HD>
__device__ __forceinline__ void attn_merge_heads(const float* __restrict__ base, int mlo, int pst, int sst, int S,
                                                 int nh, float* __restrict__ out, float* ml, float* inv_l) {
    constexpr int H2 = HD / 2, PF = 34;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nout = nh * H2;  // float2 outputs
    // the first (m, l) pair of each thread first: loads complete in order, so storing it
    // to LDS then waits for it alone, not for the prefetch behind it
    const int nk = nh * S, k0 = min(tid, nk - 1);
    const float2 ml0 = [&] {
        const int h = k0 / S, s = k0 - h * S;
        return *reinterpret_cast<const float2*>(base + (static_cast<size_t>(h) * sst + s) * pst + mlo);
    }();
    __builtin_amdgcn_sched_barrier(0);
    float2 ov[PF];
    {
        // unconditional loads (thread and split clamped into range; a load under a
        // condition becomes a branch, and the loads would then wait one by one): threads
        // past nout and splits past S load data they do not use
        const int t = min(tid, nout - 1), h = t / H2, d = 2 * (t - h * H2);
        const float* src = base + static_cast<size_t>(h) * sst * pst + d;
#pragma unroll
        for (int u = 0; u < PF; u++) ov[u] = *reinterpret_cast<const float2*>(src + static_cast<size_t>(min(u, S - 1)) * pst);
    }
    ml[2 * k0] = ml0.x;  // (threads past nk write pair nk - 1's value again)
    ml[2 * k0 + 1] = ml0.y;
    for (int k = tid + kAttnThreads; k < nk; k += kAttnThreads) {
        const int h = k / S, s = k - h * S;
        const float2 v = *reinterpret_cast<const float2*>(base + (static_cast<size_t>(h) * sst + s) * pst + mlo);
        ml[2 * k] = v.x;
        ml[2 * k + 1] = v.y;
    }
    lds_barrier();
    for (int h = wave; h < nh; h += kAttnThreads / 64) {  // one wave per head
        float mx = -INFINITY;
        for (int s = lane; s < S; s += 64) mx = fmaxf(mx, ml[2 * (h * S + s)]);
        mx = wave_max_dpp(mx);
        float L = 0.f;
        for (int s = lane; s < S; s += 64) {
            const float e = expf(ml[2 * (h * S + s)] - mx);
            ml[2 * (h * S + s)] = e;
            L = fmaf(ml[2 * (h * S + s) + 1], e, L);
        }
        L = wave_sum_dpp(L);
        if (lane == 0) inv_l[h] = 1.0f / L;
    }
    lds_barrier();
    for (int i = tid; i < nout; i += kAttnThreads) {
        const int h = i / H2, d = 2 * (i - h * H2);
        const float* e = ml + 2 * h * S;
        const float* src = base + static_cast<size_t>(h) * sst * pst + d;
        float2 o = make_float2(0.f, 0.f);
        int s = 0;
        if (i == tid) {
            // every weight read from LDS before the first is used; splits past S keep o
            float ev[PF];
#pragma unroll
            for (int u = 0; u < PF; u++) ev[u] = e[2 * min(u, S - 1)];
#pragma unroll
            for (int u = 0; u < PF; u++) {
                const float x = fmaf(ov[u].x, ev[u], o.x), y = fmaf(ov[u].y, ev[u], o.y);
                o.x = u < S ? x : o.x;
                o.y = u < S ? y : o.y;
            }
            s = PF;
        }
        for (; s < S; s += 16) {  // splits past PF: sixteen loads in flight per round
            float2 v[16];
#pragma unroll
            for (int u = 0; u < 16; u++)
                v[u] = s + u < S ? *reinterpret_cast<const float2*>(src + static_cast<size_t>(s + u) * pst)
                                 : make_float2(0.f, 0.f);
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (s + u < S) {
                    o.x = fmaf(v[u].x, e[2 * (s + u)], o.x);
                    o.y = fmaf(v[u].y, e[2 * (s + u)], o.y);
                }
        }
        const float il = inv_l[h];
        *reinterpret_cast<float2*>(out + static_cast<size_t>(h) * HD + d) = make_float2(o.x * il, o.y * il);
    }
}

// LDS of one head's merge: S (m, l) pairs and its reciprocal sum.
constexpr int kMergeLdsMax = 48 * 1024;
constexpr int kMergeParts = 1;  // workgroups per query head, each merging HD / kMergeParts dims
inline size_t merge_lds_bytes(int S) { return sizeof(float) * (2 * static_cast<size_t>(S) + 8); }

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnArgs a) {
    attn_select_query(a);
    constexpr int KS = HD / 32;                 // score k-steps
    constexpr int NDT = HD / 16;                // P.V dim tiles
    constexpr int DTW = (NDT + 3) / 4;          // dim tiles per wave (upper bound)
    __shared__ float qr_s[8 * HD];              // raw query heads
    __shared__ float q_s[8 * HD];               // RoPE'd query heads
    __shared__ float kr_s[HD];                  // raw new key
    __shared__ float2 cs_s[HD / 2];
    __shared__ v4u qop[KS * 64];                // score B operands
    __shared__ float p_s[8][kAttnChunk];
    __shared__ float ml_s[16];
    __shared__ v4u pop[2 * 64];                 // P.V B operands
    __shared__ __attribute__((aligned(16))) uint16_t knew[HD];
    __shared__ uint16_t vnew[HD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int s = blockIdx.x, kvh = blockIdx.y;
    const int reps = a.num_q / a.num_kv, half = a.rdim / 2;
    const int q_dim = a.num_q * HD, kv_dim = a.num_kv * HD;
    const int t0 = (a.t_begin & ~7) + s * kAttnChunk;
    const int pos = a.T - 1;
    if (t0 > pos) return;  // prompt mode: a chunk past this query's position
    // the last chunk holds pos; outside prompt mode its row comes from the projections
    const bool owner = pos < t0 + kAttnChunk;
    const bool fresh = owner && a.batch == 0;
    const int klim = a.batch ? pos + 1 : pos;  // K rows read from the cache: t < klim

    // 1. Global loads, all issued up front: first the query heads, the RoPE row and the
    // new K/V row (needed first, and loads return in order), then K rows below pos as
    // score A operands (lane (g, c) of wave w: position t0 + 16 w + c, dims 32 ks + 8 g ..)
    // and V blocks at or below pos as P.V A operands (dims 16 dt + c, positions
    // t0 + 32 ts + 8 g ..).
    constexpr int QPT = (8 * HD + kAttnThreads - 1) / kAttnThreads;  // query elements per thread
    float qv[QPT];
#pragma unroll
    for (int u = 0; u < QPT; u++) {
        const int i = tid + u * kAttnThreads;
        qv[u] = i < reps * HD ? a.qkv[static_cast<size_t>(kvh * reps) * HD + i] : 0.f;
    }
    const float2 csv = tid < half ? a.rope[static_cast<size_t>(pos) * half + tid] : make_float2(0.f, 0.f);
    constexpr int KPT = (HD + kAttnThreads - 1) / kAttnThreads;  // new K/V elements per thread
    float krv[KPT], vnv[KPT];
#pragma unroll
    for (int u = 0; u < KPT; u++) {
        const int d = tid + u * kAttnThreads;
        krv[u] = fresh && d < HD ? a.qkv[q_dim + static_cast<size_t>(kvh) * HD + d] : 0.f;
        vnv[u] = fresh && d < HD ? a.qkv[q_dim + kv_dim + static_cast<size_t>(kvh) * HD + d] : 0.f;
    }
    const int tk = t0 + 16 * wave + c;
    v4u kA[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
    {   // (unconditional loads from a row inside the cache, then a select: no branch around
        // the loads, so each later wait counts only the loads issued after the one it needs)
        const v4u kv = *reinterpret_cast<const v4u*>(
            a.kc + (static_cast<size_t>(max(min(tk, klim - 1), 0)) * a.num_kv + kvh) * HD + 32 * ks + 8 * g);
        kA[ks] = tk < klim ? kv : v4u{0u, 0u, 0u, 0u};
    }
    v4u vA[DTW][2];
#pragma unroll
    for (int i = 0; i < DTW; i++) {
        const int dt = wave + 4 * i;
#pragma unroll
        for (int ts = 0; ts < 2; ts++) {
            const int tv = t0 + 32 * ts + 8 * g;
            const v4u vv = *reinterpret_cast<const v4u*>(
                a.vc + ((static_cast<size_t>(min(tv, pos) >> 3) * a.num_kv + kvh) * HD + 16 * min(dt, NDT - 1) + c) * 8);
            vA[i][ts] = (dt < NDT && tv <= pos) ? vv : v4u{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int u = 0; u < QPT; u++) {
        const int i = tid + u * kAttnThreads;
        if (i < reps * HD) qr_s[i] = qv[u];
    }
    if (tid < half) cs_s[tid] = csv;  // half <= HD / 2 <= kAttnThreads
#pragma unroll
    for (int u = 0; u < KPT; u++) {
        const int d = tid + u * kAttnThreads;
        if (fresh && d < HD) {
            kr_s[d] = krv[u];
            vnew[d] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(vnv[u]));
        }
    }
    lds_barrier();
    for (int i = tid; i < reps * HD; i += kAttnThreads) {
        const int h = i / HD, d = i - h * HD;
        q_s[i] = rope_elem(qr_s + h * HD, d, half, cs_s);
    }
    if (fresh)
        for (int d = tid; d < HD; d += kAttnThreads) {
            const uint16_t kh = __builtin_bit_cast(uint16_t, static_cast<_Float16>(rope_elem(kr_s, d, half, cs_s)));
            knew[d] = kh;
            // append the new row to the cache
            a.kc[(static_cast<size_t>(pos) * a.num_kv + kvh) * HD + d] = __ushort_as_half(kh);
            a.vc[((static_cast<size_t>(pos >> 3) * a.num_kv + kvh) * HD + d) * 8 + (pos & 7)] = __ushort_as_half(vnew[d]);
        }
    lds_barrier();
    if (a.qk_norm) {  // unit-length query heads: one wave per head
        for (int h = wave; h < reps; h += kAttnThreads / 64) {
            float ss = 0.f;
            for (int d = lane; d < HD; d += 64) ss += q_s[h * HD + d] * q_s[h * HD + d];
            const float r = 1.0f / sqrtf(wave_sum_dpp(ss) + 1e-6f);
            for (int d = lane; d < HD; d += 64) q_s[h * HD + d] *= r;
        }
        lds_barrier();
    }
    // score B operands: lane (g, col) of k-step ks holds dims 32 ks + 8 g .. of column col
    for (int i = tid; i < KS * 64; i += kAttnThreads) {
        const int ks = i >> 6, l = i & 63, lg = l >> 4, col = l & 15;
        v4u op = {0u, 0u, 0u, 0u};
        if (col < 2 * reps) {
            const int h = col < reps ? col : col - reps;
            op = split8(q_s + h * HD + 32 * ks + 8 * lg, col >= reps);
        }
        qop[i] = op;
    }
    if (owner) {
        if (fresh && tk == pos) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kA[ks] = *reinterpret_cast<const v4u*>(&knew[32 * ks + 8 * g]);
        }
        // the block holding pos: the new value at pos (prompt mode: the cached one), zeros
        // above it (beyond this query)
#pragma unroll
        for (int i = 0; i < DTW; i++) {
            const int dt = wave + 4 * i;
#pragma unroll
            for (int ts = 0; ts < 2; ts++) {
                const int tv = t0 + 32 * ts + 8 * g;
                if (dt < NDT && tv <= pos && pos < tv + 8) {
                    const int e = pos - tv;
                    const bool sub = fresh;
                    const uint32_t vn = sub ? vnew[16 * dt + c] : 0u;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t w = vA[i][ts][k];
                        const uint32_t lo = 2 * k < e ? (w & 0xFFFFu)
                                                      : (2 * k == e ? (sub ? vn : (w & 0xFFFFu)) : 0u);
                        const uint32_t hi = 2 * k + 1 < e ? (w >> 16) : (2 * k + 1 == e ? (sub ? vn : (w >> 16)) : 0u);
                        vA[i][ts][k] = lo | (hi << 16);
                    }
                }
            }
        }
    }
    lds_barrier();

    // 2. Scores of positions t0 + 16 w + 4 g + r for lanes (g, col < reps).
    floatx4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
        sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, kA[ks]),
                                                      __builtin_bit_cast(half8, qop[ks * 64 + lane]), sacc, 0, 0, 0);
    sacc = add_lane_plus(sacc, reps);
    if (c < reps) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int tl = 16 * wave + 4 * g + r, t = t0 + tl;
            float sv = sacc[r] * a.scale;
            if (a.softcap > 0.f) sv = tanhf(sv / a.softcap) * a.softcap;
            p_s[c][tl] = (t >= a.t_begin && t <= pos) ? sv : -INFINITY;
        }
    }
    lds_barrier();
    // 3. Softmax partials of the chunk: one wave per head.
    for (int h = wave; h < reps; h += kAttnThreads / 64) {
        const float sc = p_s[h][lane];
        const float m = wave_max_dpp(sc);
        const float p = sc == -INFINITY ? 0.f : expf(sc - m);
        const float l = wave_sum_dpp(p);
        p_s[h][lane] = p;
        if (lane == 0) {
            ml_s[2 * h] = m;
            ml_s[2 * h + 1] = l;
        }
    }
    lds_barrier();
    // P.V B operands: lane (g, col) of position step ts holds positions 32 ts + 8 g ..
    if (tid < 2 * 64) {
        const int ts = tid >> 6, lg = (tid >> 4) & 3, col = tid & 15;
        v4u op = {0u, 0u, 0u, 0u};
        if (col < 2 * reps) {
            const int h = col < reps ? col : col - reps;
            op = split8(&p_s[h][32 * ts + 8 * lg], col >= reps);
        }
        pop[tid] = op;
    }
    lds_barrier();
    // 4. Unnormalised P.V: dims 16 dt + 4 g + r for lanes (g, col < reps).
#pragma unroll
    for (int i = 0; i < DTW; i++) {
        const int dt = wave + 4 * i;
        if (dt >= NDT) break;
        floatx4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ts = 0; ts < 2; ts++)
            o = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, vA[i][ts]),
                                                       __builtin_bit_cast(half8, pop[ts * 64 + lane]), o, 0, 0, 0);
        o = add_lane_plus(o, reps);
        if (c < reps) {
            float* dst = a.part + (static_cast<size_t>(kvh * reps + c) * a.S + s) * a.pst;
#pragma unroll
            for (int r = 0; r < 4; r++) dst[16 * dt + 4 * g + r] = o[r];
        }
    }
    if (tid < reps) {
        float* dst = a.part + (static_cast<size_t>(kvh * reps + tid) * a.S + s) * a.pst;
        dst[HD] = ml_s[2 * tid];
        dst[HD + 1] = ml_s[2 * tid + 1];
    }
}

// Merge of the S softmax partials (a second launch: the kernel boundary makes every
// partial visible), grid (num_q, 1, batch): one workgroup per query head and query (one
// per kv head, merging its query heads in turn, was 1.5275 against 1.4915 ms per 8B decode
// step: 8 workgroups each reading 4 heads' partials, against 32 reading one).  A merge
// in the split launch itself (the kv head's last workgroup to finish merging, all of its
// workgroups placed on one XCD and meeting in its L2 through an atomic arrival count) was
// measured: 1.5405 against 1.5408 ms per 8B decode step, so the chain of memory round
// trips, not the launch between them, sets the cost; the merge stays a launch.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(AttnArgs a) {
    extern __shared__ float lds[];
    const int sst = a.S;  // partial stride per head
    attn_select_query(a);
    const int S = (a.T - (a.t_begin & ~7) + kAttnChunk - 1) / kAttnChunk;  // this query's splits
    // query head h, dims [p DH, (p + 1) DH)
    constexpr int DH = HD / kMergeParts;
    const size_t h = blockIdx.x / kMergeParts;
    const int d0 = (blockIdx.x % kMergeParts) * DH;
    attn_merge_heads<DH>(a.part + h * sst * a.pst + d0, HD - d0, a.pst, sst, S, 1, a.out + h * HD + d0, lds,
                         lds + 2 * S);
}

// ── Prompt attention in one pass per block of queries ────────────────────
// Prompt mode (a.batch queries, every K/V row already in the cache): one workgroup per
// (block of queries, kv head) instead of one per (query, kv head, 64-position split) plus
// a merge launch, so each K/V row is read once per block of queries, not once per query.
// Wave w owns 16 score columns: queries q0 + w QPW .. q0 + (w + 1) QPW - 1 (QPW = 16 /
// reps) times the reps query heads of the kv head, column c = query c / reps, head c % reps.
// It walks its causal key range (from its first query's window start to its last query's
// position) in blocks of 64 positions with an online softmax: per 16-key tile the scores
// D[t][c] = K[t] . q_c on v_mfma_f32_16x16x32_f16 (K fp16 from the cache; each RoPE'd
// query split into an fp16 part and its residue, two products, as in attn_decode_kernel),
// masked outside [t_begin(q), pos(q)], scaled and capped; the block's column maxima and
// sums across the four lane groups of a column by two lane swaps; the probabilities go
// through LDS into the P.V operand order and are split the same way; O[d][c] +=
// V[t][d] P[t][c] with V read as 8-position fp16 runs.  Positions past the wave's last
// query read zeros (never stale cache rows).  The order of the sums differs from the split
// kernel's (within f32 rounding).  Head dims up to 256 and reps in {1, 2, 4, 8}.
constexpr int kPaBlock = 64;  // positions per online-softmax step

template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_prompt_kernel(AttnArgs a) {
    constexpr int KS = HD / 32, NDT = HD / 16;
    __shared__ float qraw[4][16][HD];
    __shared__ __attribute__((aligned(16))) float pblk[4][2 * 4 * 16 * 8];  // [ts][g][c][8 e] per wave
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c = lane & 15;
    const int kvh = blockIdx.y;
    const int reps = a.num_q / a.num_kv, qpw = 16 / reps, half = a.rdim / 2;
    const int q_first = (blockIdx.x * 4 + wave) * qpw;      // this wave's first query
    const int q_last = min(q_first + qpw, a.batch) - 1;     // and its last (< q_first: none)
    const int qc = q_first + c / reps, hc = c % reps;       // column c's query and head
    const bool col_ok = c < qpw * reps && qc <= q_last;
    const int pos_c = a.T - 1 + qc;                          // column c's position
    const int tb_c = (a.window > 0 && pos_c + 1 > a.window) ? pos_c + 1 - a.window : 0;

    // 1. The wave's query rows (raw), RoPE'd per lane for its dims, QK-normed, split.  All
    // of a lane's loads are issued before the first is used (rows clamped into the batch,
    // then zeros selected for columns without a query), not one round trip each.
    {
        constexpr int QL = 16 * HD / 64;
        float qt[QL];
#pragma unroll
        for (int k = 0; k < QL; k++) {
            const int i = lane + 64 * k, col = i / HD, d = i - col * HD;
            const int q = max(0, min(q_first + col / reps, a.batch - 1));
            qt[k] = a.qkv[static_cast<size_t>(q) * a.qkv_ld + static_cast<size_t>(kvh * reps + col % reps) * HD + d];
        }
#pragma unroll
        for (int k = 0; k < QL; k++) {
            const int i = lane + 64 * k, col = i / HD, d = i - col * HD, q = q_first + col / reps;
            qraw[wave][col][d] = (col < qpw * reps && q <= q_last) ? qt[k] : 0.f;
        }
    }
    __syncthreads();
    float qv[KS][8];
    {
        // the (cos, sin) pair of each of the lane's dims, loaded together (dims past the
        // rotated ones read pair 0 and do not use it; no table when nothing rotates)
        const float2* cs = a.rope + static_cast<size_t>(col_ok ? pos_c : 0) * half;
        float2 csv[KS][8];
        if (half > 0) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int d = 32 * ks + 8 * g + e;
                    csv[ks][e] = cs[d < half ? d : (d < 2 * half ? d - half : 0)];
                }
        }
        float ss = 0.f;
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int d = 32 * ks + 8 * g + e;
                const float* x = qraw[wave][c];
                const float2 p = csv[ks][e];
                const float v = d < half ? x[d] * p.x - x[d + half] * p.y
                                         : (d < 2 * half ? x[d - half] * p.y + x[d] * p.x : x[d]);
                qv[ks][e] = v;
                ss += v * v;
            }
        if (a.qk_norm) {  // 1 / sqrt(sum q^2 + 1e-6) over the head: the four lane groups of column c
            ss += __shfl_xor(ss, 16, 64);
            ss += __shfl_xor(ss, 32, 64);
            const float r = 1.0f / sqrtf(ss + 1e-6f);
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int e = 0; e < 8; e++) qv[ks][e] *= r;
        }
    }
    v4u qh[KS], ql[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        qh[ks] = split8(qv[ks], 0);
        ql[ks] = split8(qv[ks], 1);
    }

    floatx4 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; dt++) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;
    if (q_last >= q_first) {
        const int pos_hi = a.T - 1 + q_last;  // the wave's last position
        const int tq0 = a.T - 1 + q_first + 1;
        const int t_lo = ((a.window > 0 && tq0 > a.window) ? tq0 - a.window : 0) & ~7;
        float* pw = pblk[wave];
        for (int kb = t_lo; kb <= pos_hi; kb += kPaBlock) {
            // every K and V load of the block issued together, the K tiles first (loads
            // return in order): A operand lane (g, c) of tile kt = position kb + 16 kt + c,
            // dims 32 ks + 8 g ..; of V = dim 16 dt + c, positions kb + 32 ts + 8 g ..  Rows
            // past pos_hi read row pos_hi instead, unconditionally, so no load sits under a
            // branch: their scores are masked below and their V runs replaced by zeros.
            v4u ka[4][KS], vb[NDT][2];
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                const int tk = min(kb + 16 * kt + c, pos_hi);
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    ka[kt][ks] = *reinterpret_cast<const v4u*>(a.kc + (static_cast<size_t>(tk) * a.num_kv + kvh) * HD +
                                                               32 * ks + 8 * g);
            }
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
#pragma unroll
                for (int ts = 0; ts < 2; ts++) {
                    const int tv = kb + 32 * ts + 8 * g;
                    const v4u v = *reinterpret_cast<const v4u*>(
                        a.vc + ((static_cast<size_t>(min(tv, pos_hi) >> 3) * a.num_kv + kvh) * HD + 16 * dt + c) * 8);
                    vb[dt][ts] = tv <= pos_hi ? v : v4u{0u, 0u, 0u, 0u};
                }
            // scores of 4 tiles of 16 positions: lane (g, c) holds positions kb + 16 kt + 4 g + r
            float sv[4][4];
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                floatx4 d4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    d4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ka[kt][ks]), __builtin_bit_cast(half8, qh[ks]),
                                                                d4, 0, 0, 0);
                    d4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ka[kt][ks]), __builtin_bit_cast(half8, ql[ks]),
                                                                d4, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int t = kb + 16 * kt + 4 * g + r;
                    float v = d4[r] * a.scale;
                    if (a.softcap > 0.f) v = tanhf(v / a.softcap) * a.softcap;
                    sv[kt][r] = (col_ok && t >= tb_c && t <= pos_c) ? v : -INFINITY;
                }
            }
            // online softmax over the block, column c
            float mb = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) mb = fmaxf(mb, sv[kt][r]);
            mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
            mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
            const float m_new = fmaxf(m_run, mb);
            const float alpha = m_new == -INFINITY ? 1.f : expf(m_run - m_new);
            float ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                float p4[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    p4[r] = sv[kt][r] == -INFINITY ? 0.f : expf(sv[kt][r] - m_new);
                    ls += p4[r];
                }
                // positions 16 kt + 4 g .. + 3 -> P.V step ts, lane group gp, elements e0 .. e0 + 3
                const int k0 = 16 * kt + 4 * g, ts = k0 >> 5, gp = (k0 & 31) >> 3, e0 = k0 & 7;
                *reinterpret_cast<float4*>(pw + ((ts * 4 + gp) * 16 + c) * 8 + e0) = make_float4(p4[0], p4[1], p4[2], p4[3]);
            }
            ls += __shfl_xor(ls, 16, 64);
            ls += __shfl_xor(ls, 32, 64);
            l_run = l_run * alpha + ls;
            m_run = m_new;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) o[dt] *= alpha;
            // the wave reads what its lanes wrote: keep the LDS accesses in program order
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            v4u ph[2], pl[2];
#pragma unroll
            for (int ts = 0; ts < 2; ts++) {
                const float4* src = reinterpret_cast<const float4*>(pw + ((ts * 4 + g) * 16 + c) * 8);
                const float4 u0 = src[0], u1 = src[1];
                const float pv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
                ph[ts] = split8(pv, 0);
                pl[ts] = split8(pv, 1);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // O[d][c] += sum_t V[t][d] P[t][c]: A lane (g, c) = dim 16 dt + c, positions kb + 32 ts + 8 g ..
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) {
#pragma unroll
                for (int ts = 0; ts < 2; ts++) {
                    const int tv = kb + 32 * ts + 8 * g;
                    v4u va = vb[dt][ts];
                    if (tv + 7 > pos_hi) {  // the run holding pos_hi: zeros past it (rows not written)
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            const uint32_t lo = 2 * k <= pos_hi - tv ? (va[k] & 0xFFFFu) : 0u;
                            const uint32_t hi = 2 * k + 1 <= pos_hi - tv ? (va[k] >> 16) : 0u;
                            va[k] = lo | (hi << 16);
                        }
                    }
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, va), __builtin_bit_cast(half8, ph[ts]),
                                                                   o[dt], 0, 0, 0);
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, va), __builtin_bit_cast(half8, pl[ts]),
                                                                   o[dt], 0, 0, 0);
                }
            }
        }
    }
    // out[q][(kvh reps + h) HD + d] = O / l: lane (g, c) holds dims 16 dt + 4 g + r of column c
    if (col_ok) {
        const float inv = 1.0f / l_run;
        float* dst = a.out + static_cast<size_t>(qc) * a.num_q * HD + static_cast<size_t>(kvh * reps + hc) * HD;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++)
#pragma unroll
            for (int r = 0; r < 4; r++) dst[16 * dt + 4 * g + r] = o[dt][r] * inv;
    }
}

bool attn_supported(int reps, int hd) { return reps >= 1 && reps <= 8 && hd % 32 == 0 && hd >= 32 && hd <= 512; }

int attn_partial_stride(int hd) { return hd + 2; }

__global__ void rope_table_kernel(float2* cs, size_t n, int half, int rdim, double base) {
    const size_t idx = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (idx >= n) return;
    const size_t p = idx / half;
    const int i = static_cast<int>(idx - p * half);
    const double inv_freq = 1.0 / pow(base, 2.0 * i / static_cast<double>(rdim));
    const double th = static_cast<double>(p) * inv_freq;
    cs[idx] = make_float2(static_cast<float>(cos(th)), static_cast<float>(sin(th)));
}

void launch_rope_table(float2* cs, size_t cap, int rdim, double base, hipStream_t s) {
    const size_t n = cap * static_cast<size_t>(rdim / 2);
    if (n == 0) return;
    rope_table_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s>>>(cs, n, rdim / 2, rdim, base);
    LARQL_HIP_CHECK(hipGetLastError());
}

// ── small utility kernels ──────────────────────────────────────────────
__global__ void copy_f32_kernel(const float* __restrict__ src, float* __restrict__ dst, size_t n) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

__global__ void f32_to_f16_kernel(const float* __restrict__ src, __half* __restrict__ dst, size_t n) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i < n) dst[i] = __float2half_rn(src[i]);
}

// [seq][num_kv][hd] rows (f32, or fp16 bits) -> the V cache layout [t / 8][num_kv][hd][8].
template <typename T>
__global__ void v_to_cache_kernel(const T* __restrict__ src, __half* __restrict__ dst, size_t seq, int num_kv,
                                  int hd) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    const size_t row = static_cast<size_t>(num_kv) * hd;
    if (i >= seq * row) return;
    const size_t t = i / row, j = i - t * row;  // j = kvh * hd + d
    __half v;
    if constexpr (sizeof(T) == 4) v = __float2half_rn(src[i]);
    else v = __ushort_as_half(src[i]);
    dst[((t >> 3) * row + j) * 8 + (t & 7)] = v;
}

void launch_v_to_cache(const void* src, bool src_f32, __half* dst, size_t seq, int num_kv, int hd, hipStream_t s) {
    const size_t n = seq * static_cast<size_t>(num_kv) * hd;
    if (n == 0) return;
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    if (src_f32) v_to_cache_kernel<float><<<grid, dim3(256), 0, s>>>(static_cast<const float*>(src), dst, seq, num_kv, hd);
    else v_to_cache_kernel<uint16_t><<<grid, dim3(256), 0, s>>>(static_cast<const uint16_t*>(src), dst, seq, num_kv, hd);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s) {
    if (n == 0) return;
    copy_f32_kernel<<<dim3((n + 255) / 256), dim3(256), 0, s>>>(src, dst, n);
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_f32_to_f16(const float* src, __half* dst, size_t n, hipStream_t s) {
    if (n == 0) return;
    f32_to_f16_kernel<<<dim3((n + 255) / 256), dim3(256), 0, s>>>(src, dst, n);
    LARQL_HIP_CHECK(hipGetLastError());
}

int attn_splits(int T, int t_begin) { return (T - (t_begin & ~7) + kAttnChunk - 1) / kAttnChunk; }

int attn_prompt_splits(int T0, int batch, int window) {
    int S = 1;
    for (int p = 0; p < batch; p++) {
        const int T = T0 + p, tb = (window > 0 && T > window) ? T - window : 0;
        S = std::max(S, attn_splits(T, tb));
    }
    return S;
}

// f(std::integral_constant<int, hd>) for the instantiated head dims, the multiples of 32
// from HD up to 512; false for any other hd.
template <int HD, typename F>
bool dispatch_head_dim(int hd, F&& f) {
    if (hd == HD) {
        f(std::integral_constant<int, HD>{});
        return true;
    }
    if constexpr (HD < 512) return dispatch_head_dim<HD + 32>(hd, f);
    return false;
}

void launch_attention(const AttnArgs& a0, hipStream_t s) {
    AttnArgs a = a0;
    const int reps = a.num_q / a.num_kv;
    if (!attn_supported(reps, a.hd)) fail(LARQL_HIP_ERR_UNSUPPORTED, "attention: head geometry");
    if (a.batch && a.hd <= 256 && 16 % reps == 0) {  // prompt mode: one pass per block of queries
        const int qpb = 4 * (16 / reps);
        const dim3 gp(static_cast<unsigned>((a.batch + qpb - 1) / qpb), a.num_kv), bp(kAttnThreads);
        if (!dispatch_head_dim<32>(a.hd, [&](auto h) {
                constexpr int H = decltype(h)::value;
                if constexpr (H <= 256) attn_prompt_kernel<H><<<gp, bp, 0, s>>>(a);
            }))
            fail(LARQL_HIP_ERR_UNSUPPORTED, "attention: head_dim");
        LARQL_HIP_CHECK(hipGetLastError());
        return;
    }
    a.S = a.batch ? attn_prompt_splits(a.T, a.batch, a.window) : attn_splits(a.T, a.t_begin);
    a.pst = attn_partial_stride(a.hd);
    if (2 * static_cast<size_t>(a.S) * sizeof(float) + 32 > static_cast<size_t>(kMergeLdsMax))
        fail(LARQL_HIP_ERR_UNSUPPORTED, "attention: too many position splits");
    const int nz = a.batch ? a.batch : 1;
    const size_t lds = merge_lds_bytes(a.S);
    const dim3 grid(a.S, a.num_kv, nz), block(kAttnThreads);
    if (!dispatch_head_dim<32>(a.hd, [&](auto h) { attn_decode_kernel<decltype(h)::value><<<grid, block, 0, s>>>(a); }))
        fail(LARQL_HIP_ERR_UNSUPPORTED, "attention: head_dim");
    LARQL_HIP_CHECK(hipGetLastError());
    const dim3 g2(a.num_q * kMergeParts, 1, nz);
    dispatch_head_dim<32>(a.hd, [&](auto h) { attn_combine_kernel<decltype(h)::value><<<g2, block, lds, s>>>(a); });
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
