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
#include <cmath>
#include <vector>

namespace larql {

constexpr int kAttnThreads = 256;
constexpr int kAttnChunk = 64;   // positions per workgroup (= wave size: one score per lane)

// Split-half RoPE of element d of head vector x (LI/src/attention/rope.rs:22-55):
// pairs (i, i + rdim/2), dims >= rdim untouched.  cs[i] = (cos, sin) of pair i.
__device__ __forceinline__ float rope_elem(const float* x, int d, int half, const float2* cs) {
    if (d < half) return x[d] * cs[d].x - x[d + half] * cs[d].y;
    if (d < 2 * half) return x[d - half] * cs[d - half].y + x[d] * cs[d - half].x;
    return x[d];
}

// Workgroup-wide max / sum through `scratch` (>= kAttnThreads / 64 floats); every
// thread gets the result.
__device__ __forceinline__ float block_max(float v, float* scratch) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < kAttnThreads / 64; w++) r = fmaxf(r, scratch[w]);
    __syncthreads();
    return r;
}
__device__ __forceinline__ float block_sum(float v, float* scratch) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < kAttnThreads / 64; w++) r += scratch[w];
    __syncthreads();
    return r;
}

__device__ __forceinline__ float2 h2_to_f2(uint32_t v) {
    return make_float2(h2f(v & 0xFFFFu), h2f(v >> 16));
}

__device__ __forceinline__ uint32_t f2_to_h2(float a, float b) {
    const uint32_t lo = __half_as_ushort(__float2half_rn(a));
    const uint32_t hi = __half_as_ushort(__float2half_rn(b));
    return lo | (hi << 16);
}

// Grid (S, num_kv).  Workgroup (s, kvh) covers positions [t_begin + 64 s, ...) for the
// reps = num_q/num_kv query heads of kv head kvh (GQA: kv_h = h / reps,
// LI/src/attention/gqa.rs:53).  Every stage gives each thread one independent item
// with split accumulators (a dependent VALU result is ~32 cycles away on gfx950):
// scores = one (head, position) per thread, P.V = one (head, dim pair) per thread.
// attn_combine_kernel merges the S softmax partials of each head.
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnArgs a) {
    extern __shared__ float lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int nw = kAttnThreads / 64;
    const int s = blockIdx.x, kvh = blockIdx.y;
    const int reps = a.num_q / a.num_kv;
    const int hd = a.hd, hd2 = hd / 2, half = a.rdim / 2;
    const int q_dim = a.num_q * hd, kv_dim = a.num_kv * hd;
    float* q_s = lds;                                               // reps * hd
    float2* cs_s = reinterpret_cast<float2*>(q_s + reps * hd);      // half
    uint32_t* k_s = reinterpret_cast<uint32_t*>(cs_s + half);       // chunk * (hd2 + 1), padded rows
    uint32_t* v_s = k_s + kAttnChunk * (hd2 + 1);                   // chunk * hd2
    float* p_s = reinterpret_cast<float*>(v_s + kAttnChunk * hd2);  // reps * max(chunk, hd)
    float* ml_s = p_s + reps * max(kAttnChunk, hd);                 // reps * 2

    const int t0 = a.t_begin + s * kAttnChunk;
    const int t1 = min(a.T, t0 + kAttnChunk);
    const int nt = t1 - t0;
    const int pos = a.T - 1;

    // Every global load of the workgroup is issued up front: the K/V tile (into
    // registers), the raw query heads and this position's RoPE row (into LDS); one
    // barrier then covers all of them.
    const int c8n = hd / 8;
    constexpr int kMaxItems = 8;  // nt * c8n <= 64 * 32 = kMaxItems * kAttnThreads (hd <= 256)
    uint4 kk[kMaxItems], vv[kMaxItems];
#pragma unroll
    for (int it = 0; it < kMaxItems; it++) {
        const int idx = tid + it * kAttnThreads;
        const int tl = idx / c8n, c8 = idx - tl * c8n, t = t0 + tl;
        if (idx < nt * c8n && t != pos) {
            const size_t off = (static_cast<size_t>(t) * a.num_kv + kvh) * hd + c8 * 8;
            kk[it] = *reinterpret_cast<const uint4*>(a.kc + off);
            vv[it] = *reinterpret_cast<const uint4*>(a.vc + off);
        }
    }
    float* qraw_s = p_s;  // reps * hd floats, free until the scores are written
    for (int idx = tid; idx < reps * hd; idx += kAttnThreads)
        qraw_s[idx] = a.qkv[static_cast<size_t>(kvh * reps) * hd + idx];
    for (int i = tid; i < half; i += kAttnThreads) cs_s[i] = a.rope[static_cast<size_t>(pos) * half + i];
    __syncthreads();
    for (int idx = tid; idx < reps * hd; idx += kAttnThreads) {
        const int g = idx / hd, d = idx - g * hd;
        q_s[idx] = rope_elem(qraw_s + g * hd, d, half, cs_s);
    }
    // K/V tile into LDS.  The row at pos comes from the fresh projections: RoPE'd,
    // rounded to fp16 and appended to the cache by the one workgroup that owns it.
#pragma unroll
    for (int it = 0; it < kMaxItems; it++) {
        const int idx = tid + it * kAttnThreads;
        if (idx >= nt * c8n) continue;
        const int tl = idx / c8n, c8 = idx - tl * c8n, t = t0 + tl;
        uint32_t kw[4], vw[4];
        if (t == pos) {
            const float* kh = a.qkv + q_dim + static_cast<size_t>(kvh) * hd;
            const float* vh = a.qkv + q_dim + kv_dim + static_cast<size_t>(kvh) * hd;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = c8 * 8 + 2 * j;
                kw[j] = f2_to_h2(rope_elem(kh, d, half, cs_s), rope_elem(kh, d + 1, half, cs_s));
                vw[j] = f2_to_h2(vh[d], vh[d + 1]);
            }
            const size_t off = (static_cast<size_t>(t) * a.num_kv + kvh) * hd + c8 * 8;
            *reinterpret_cast<uint4*>(a.kc + off) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
            *reinterpret_cast<uint4*>(a.vc + off) = make_uint4(vw[0], vw[1], vw[2], vw[3]);
        } else {
            kw[0] = kk[it].x; kw[1] = kk[it].y; kw[2] = kk[it].z; kw[3] = kk[it].w;
            vw[0] = vv[it].x; vw[1] = vv[it].y; vw[2] = vv[it].z; vw[3] = vv[it].w;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            k_s[tl * (hd2 + 1) + c8 * 4 + j] = kw[j];
            v_s[tl * hd2 + c8 * 4 + j] = vw[j];
        }
    }
    __syncthreads();

    // Scores: thread (g, t), four accumulators over the head dimension.
    for (int idx = tid; idx < reps * kAttnChunk; idx += kAttnThreads) {
        const int g = idx / kAttnChunk, t = idx - g * kAttnChunk;
        float sc = -INFINITY;
        if (t < nt) {
            const uint32_t* kr = k_s + t * (hd2 + 1);
            const float2* qg = reinterpret_cast<const float2*>(q_s + g * hd);
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int j = 0; j < hd2; j += 2) {
                const float2 k0 = h2_to_f2(kr[j]), k1 = h2_to_f2(kr[j + 1]);
                const float2 q0 = qg[j], q1 = qg[j + 1];
                acc[0] = fmaf(k0.x, q0.x, acc[0]);
                acc[1] = fmaf(k0.y, q0.y, acc[1]);
                acc[2] = fmaf(k1.x, q1.x, acc[2]);
                acc[3] = fmaf(k1.y, q1.y, acc[3]);
            }
            sc = ((acc[0] + acc[1]) + (acc[2] + acc[3])) * a.scale;
        }
        p_s[idx] = sc;
    }
    __syncthreads();
    // Softmax partials of the chunk: one wave per head.
    for (int g = wave; g < reps; g += nw) {
        const float sc = p_s[g * kAttnChunk + lane];
        const float m = wave_max(sc);
        const float p = lane < nt ? expf(sc - m) : 0.f;
        const float l = wave_sum(p);
        p_s[g * kAttnChunk + lane] = p;
        if (lane == 0) {
            ml_s[2 * g] = m;
            ml_s[2 * g + 1] = l;
        }
    }
    __syncthreads();
    // Unnormalised P.V: thread (g, dim pair j), even / odd positions on separate chains.
    for (int idx = tid; idx < reps * hd2; idx += kAttnThreads) {
        const int g = idx / hd2, j = idx - g * hd2;
        const int h = kvh * reps + g;
        const float* pg = p_s + g * kAttnChunk;
        float ox[2] = {0.f, 0.f}, oy[2] = {0.f, 0.f};
        int t = 0;
        for (; t + 1 < nt; t += 2) {
            const float2 v0 = h2_to_f2(v_s[t * hd2 + j]), v1 = h2_to_f2(v_s[(t + 1) * hd2 + j]);
            ox[0] = fmaf(pg[t], v0.x, ox[0]);
            oy[0] = fmaf(pg[t], v0.y, oy[0]);
            ox[1] = fmaf(pg[t + 1], v1.x, ox[1]);
            oy[1] = fmaf(pg[t + 1], v1.y, oy[1]);
        }
        if (t < nt) {
            const float2 v0 = h2_to_f2(v_s[t * hd2 + j]);
            ox[0] = fmaf(pg[t], v0.x, ox[0]);
            oy[0] = fmaf(pg[t], v0.y, oy[0]);
        }
        float* dst = a.part + (static_cast<size_t>(h) * a.S + s) * (hd + 2);
        dst[2 * j] = ox[0] + ox[1];
        dst[2 * j + 1] = oy[0] + oy[1];
        if (j == 0) {
            dst[hd] = ml_s[2 * g];
            dst[hd + 1] = ml_s[2 * g + 1];
        }
    }
}

// Merge of the S softmax partials of each head (a second launch: the kernel boundary
// makes every partial visible, with no device-scope fences in the split kernel):
//   o = sum_s e_s o_s / sum_s e_s l_s,   e_s = exp(m_s - max_s m_s).
// Grid (num_q); thread (group g, dim pair j) sums splits g, g + 256/(hd/2), ... with
// the per-split weights computed once per workgroup in LDS.
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(AttnArgs a) {
    extern __shared__ float lds[];
    const int h = blockIdx.x, tid = threadIdx.x, hd = a.hd, hd2 = hd / 2;
    const int ngrp = kAttnThreads / hd2;                 // split groups (hd2 divides 256)
    float* e_s = lds;                                    // S weights
    float2* o_s = reinterpret_cast<float2*>(e_s + a.S);  // ngrp * hd2 partial outputs
    float* red = reinterpret_cast<float*>(o_s + ngrp * hd2);
    const float* src = a.part + static_cast<size_t>(h) * a.S * (hd + 2);
    float M = -INFINITY;
    for (int s2 = tid; s2 < a.S; s2 += kAttnThreads) M = fmaxf(M, src[s2 * (hd + 2) + hd]);
    M = block_max(M, red);
    float L = 0.f;
    for (int s2 = tid; s2 < a.S; s2 += kAttnThreads) {
        const float e = expf(src[s2 * (hd + 2) + hd] - M);
        e_s[s2] = e;
        L = fmaf(src[s2 * (hd + 2) + hd + 1], e, L);
    }
    L = block_sum(L, red);  // also orders the e_s writes before their reads
    // thread (grp, j): splits grp, grp + ngrp, ...; loads unrolled by four
    const int grp = tid / hd2, j = tid - grp * hd2;
    float2 o = make_float2(0.f, 0.f);
    int s2 = grp;
    for (; s2 + 3 * ngrp < a.S; s2 += 4 * ngrp) {
        float2 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = *reinterpret_cast<const float2*>(src + (s2 + u * ngrp) * (hd + 2) + 2 * j);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            o.x = fmaf(v[u].x, e_s[s2 + u * ngrp], o.x);
            o.y = fmaf(v[u].y, e_s[s2 + u * ngrp], o.y);
        }
    }
    for (; s2 < a.S; s2 += ngrp) {
        const float2 v = *reinterpret_cast<const float2*>(src + s2 * (hd + 2) + 2 * j);
        o.x = fmaf(v.x, e_s[s2], o.x);
        o.y = fmaf(v.y, e_s[s2], o.y);
    }
    o_s[grp * hd2 + j] = o;
    __syncthreads();
    if (tid < hd2) {
        float2 t = o_s[tid];
        for (int g = 1; g < ngrp; g++) {
            t.x += o_s[g * hd2 + tid].x;
            t.y += o_s[g * hd2 + tid].y;
        }
        const float invL = 1.0f / L;
        *reinterpret_cast<float2*>(a.out + static_cast<size_t>(h) * hd + 2 * tid) = make_float2(t.x * invL, t.y * invL);
    }
}

size_t attn_lds_bytes(int reps, int hd, int rdim) {
    return sizeof(float) * reps * hd + sizeof(float2) * (rdim / 2) +
           sizeof(uint32_t) * (kAttnChunk * (hd / 2 + 1) + kAttnChunk * hd / 2) +
           sizeof(float) * (reps * std::max(kAttnChunk, hd) + 2 * reps);
}

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

void launch_attention(const AttnArgs& a0, hipStream_t s) {
    AttnArgs a = a0;
    a.S = (a.T - a.t_begin + kAttnChunk - 1) / kAttnChunk;
    const int reps = a.num_q / a.num_kv;
    const size_t lds = attn_lds_bytes(reps, a.hd, a.rdim);
    attn_decode_kernel<<<dim3(a.S, a.num_kv), dim3(kAttnThreads), lds, s>>>(a);
    LARQL_HIP_CHECK(hipGetLastError());
    // combine: S split weights + block-reduction scratch
    const size_t lds2 = sizeof(float) * (static_cast<size_t>(a.S) + 2 * kAttnThreads + kAttnThreads / 64);
    if (lds2 > 64 * 1024) fail(LARQL_HIP_ERR_UNSUPPORTED, "attention: too many position splits");
    attn_combine_kernel<<<dim3(a.num_q), dim3(kAttnThreads), lds2, s>>>(a);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
