// Decode step: single-query GQA attention over the fp16 KV cache, the KV cache
// itself, the device-resident decoder model and the per-token kernel sequence.
//
// Per layer (Llama, pre-norm, LI/src/attention/block.rs:52-157, LI/src/forward/layer.rs:50-94;
// op order of the reference GPU decode LC/src/metal/decode.rs:144-715):
//   1. qkv   = [Wq|Wk|Wv] . rms_norm(h, input_norm)          fused norm + matvec
//   2. attn  = softmax(RoPE(q) . RoPE(K)^T * scale) . V      split-K over T, this file
//              (the new K/V row is RoPE'd, rounded to fp16 and appended at pos)
//   3. h1    = h + Wo . attn                                  matvec + residual epilogue
//   4. act   = silu(Wg . n) * (Wu . n), n = rms_norm(h1)      fused norm + interleaved gate/up
//   5. h     = h1 + Wd . act                                  matvec + residual epilogue
// Five launches per layer; the final norm + head is one more.
#include "decode.h"
#include "matvec_common.h"

#include <cmath>
#include <vector>

namespace larql {

constexpr int kAttnThreads = 256;
constexpr int kAttnChunk = 64;   // positions per workgroup (= wave size: one score per lane)

// Split-half RoPE of element d of head vector x at the table's position
// (LI/src/attention/rope.rs:22-55): pairs (i, i + rdim/2), dims >= rdim untouched.
__device__ __forceinline__ float rope_elem(const float* x, int d, int half, const float* cs, const float* sn) {
    if (d < half) return x[d] * cs[d] - x[d + half] * sn[d];
    if (d < 2 * half) return x[d - half] * sn[d - half] + x[d] * cs[d - half];
    return x[d];
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
// num_q/num_kv query heads of kv head kvh (GQA: kv_h = h / reps, LI/src/attention/gqa.rs:53).
// Softmax partials are combined by the last workgroup of each kv head to finish.
__global__ __launch_bounds__(kAttnThreads) void attn_decode_kernel(AttnArgs a) {
    extern __shared__ float lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nw = kAttnThreads / 64;
    const int s = blockIdx.x, kvh = blockIdx.y;
    const int reps = a.num_q / a.num_kv;
    const int hd = a.hd, hd2 = hd / 2, half = a.rdim / 2;
    const int q_dim = a.num_q * hd, kv_dim = a.num_kv * hd;
    float* q_s = lds;                                               // reps * hd
    float* cs_s = q_s + reps * hd;                                  // half
    float* sn_s = cs_s + half;                                      // half
    uint32_t* k_s = reinterpret_cast<uint32_t*>(sn_s + half);       // chunk * (hd2 + 1), padded rows
    uint32_t* v_s = k_s + kAttnChunk * (hd2 + 1);                   // chunk * hd2
    float* p_s = reinterpret_cast<float*>(v_s + kAttnChunk * hd2);  // reps * chunk
    float* ml_s = p_s + reps * kAttnChunk;                          // reps * 2
    int* flag_s = reinterpret_cast<int*>(ml_s + 2 * reps);

    const int t0 = a.t_begin + s * kAttnChunk;
    const int t1 = min(a.T, t0 + kAttnChunk);
    const int nt = t1 - t0;
    const int pos = a.T - 1;

    // RoPE table for the new position, angles in f64 as the CPU path computes them.
    for (int i = tid; i < half; i += kAttnThreads) {
        const double inv_freq = 1.0 / pow(a.rope_base, 2.0 * i / static_cast<double>(a.rdim));
        const double th = static_cast<double>(pos) * inv_freq;
        cs_s[i] = static_cast<float>(cos(th));
        sn_s[i] = static_cast<float>(sin(th));
    }
    __syncthreads();
    for (int idx = tid; idx < reps * hd; idx += kAttnThreads) {
        const int g = idx / hd, d = idx - g * hd;
        q_s[idx] = rope_elem(a.qkv + static_cast<size_t>(kvh * reps + g) * hd, d, half, cs_s, sn_s);
    }
    // K/V tile into LDS (8 halves per thread-iteration).  The row at pos comes from the
    // fresh projections: RoPE'd, rounded to fp16 and appended to the cache by the one
    // workgroup that owns it.
    const int c8n = hd / 8;
    for (int idx = tid; idx < nt * c8n; idx += kAttnThreads) {
        const int tl = idx / c8n, c8 = idx - tl * c8n, t = t0 + tl;
        const size_t off = (static_cast<size_t>(t) * a.num_kv + kvh) * hd + c8 * 8;
        uint32_t kw[4], vw[4];
        if (t == pos) {
            const float* kh = a.qkv + q_dim + static_cast<size_t>(kvh) * hd;
            const float* vh = a.qkv + q_dim + kv_dim + static_cast<size_t>(kvh) * hd;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = c8 * 8 + 2 * j;
                kw[j] = f2_to_h2(rope_elem(kh, d, half, cs_s, sn_s), rope_elem(kh, d + 1, half, cs_s, sn_s));
                vw[j] = f2_to_h2(vh[d], vh[d + 1]);
            }
            *reinterpret_cast<uint4*>(a.kc + off) = make_uint4(kw[0], kw[1], kw[2], kw[3]);
            *reinterpret_cast<uint4*>(a.vc + off) = make_uint4(vw[0], vw[1], vw[2], vw[3]);
        } else {
            const uint4 kk = *reinterpret_cast<const uint4*>(a.kc + off);
            const uint4 vv = *reinterpret_cast<const uint4*>(a.vc + off);
            kw[0] = kk.x; kw[1] = kk.y; kw[2] = kk.z; kw[3] = kk.w;
            vw[0] = vv.x; vw[1] = vv.y; vw[2] = vv.z; vw[3] = vv.w;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            k_s[tl * (hd2 + 1) + c8 * 4 + j] = kw[j];
            v_s[tl * hd2 + c8 * 4 + j] = vw[j];
        }
    }
    __syncthreads();

    // Scores (one position per lane) and the chunk's softmax partials.
    for (int g = wave; g < reps; g += nw) {
        float sc = -INFINITY;
        if (lane < nt) {
            const uint32_t* kr = k_s + lane * (hd2 + 1);
            const float* qg = q_s + g * hd;
            float acc = 0.f;
            for (int j = 0; j < hd2; j++) {
                const float2 kf = h2_to_f2(kr[j]);
                acc = fmaf(kf.x, qg[2 * j], acc);
                acc = fmaf(kf.y, qg[2 * j + 1], acc);
            }
            sc = acc * a.scale;
        }
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
    // Unnormalised P.V for the chunk: lanes over dim pairs.
    for (int g = wave; g < reps; g += nw) {
        const int h = kvh * reps + g;
        float* dst = a.part + (static_cast<size_t>(h) * a.S + s) * (hd + 2);
        for (int j = lane; j < hd2; j += 64) {
            float ox = 0.f, oy = 0.f;
            for (int t = 0; t < nt; t++) {
                const float pt = p_s[g * kAttnChunk + t];
                const float2 v = h2_to_f2(v_s[t * hd2 + j]);
                ox = fmaf(pt, v.x, ox);
                oy = fmaf(pt, v.y, oy);
            }
            dst[2 * j] = ox;
            dst[2 * j + 1] = oy;
        }
        if (lane == 0) {
            dst[hd] = ml_s[2 * g];
            dst[hd + 1] = ml_s[2 * g + 1];
        }
    }
    // The last workgroup of this kv head to finish merges the S partials.
    __threadfence();
    __syncthreads();
    if (tid == 0) *flag_s = atomicAdd(&a.counter[kvh], 1) == a.S - 1;
    __syncthreads();
    if (!*flag_s) return;
    __threadfence();
    for (int g = wave; g < reps; g += nw) {
        const int h = kvh * reps + g;
        const volatile float* src = a.part + static_cast<size_t>(h) * a.S * (hd + 2);
        float M = -INFINITY;
        for (int s2 = lane; s2 < a.S; s2 += 64) M = fmaxf(M, src[s2 * (hd + 2) + hd]);
        M = wave_max(M);
        float L = 0.f;
        for (int s2 = lane; s2 < a.S; s2 += 64) L += src[s2 * (hd + 2) + hd + 1] * expf(src[s2 * (hd + 2) + hd] - M);
        L = wave_sum(L);
        const float invL = 1.0f / L;
        for (int d = lane; d < hd; d += 64) {
            float o = 0.f;
            for (int s2 = 0; s2 < a.S; s2++) o += src[s2 * (hd + 2) + d] * expf(src[s2 * (hd + 2) + hd] - M);
            a.out[static_cast<size_t>(h) * hd + d] = o * invL;
        }
    }
    if (tid == 0) a.counter[kvh] = 0;
}

size_t attn_lds_bytes(int reps, int hd, int rdim) {
    return sizeof(float) * (reps * hd + rdim) + sizeof(uint32_t) * (kAttnChunk * (hd / 2 + 1) + kAttnChunk * hd / 2) +
           sizeof(float) * (reps * kAttnChunk + 2 * reps) + 16;
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
}

}  // namespace larql
