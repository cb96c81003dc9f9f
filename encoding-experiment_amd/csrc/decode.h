// Attention kernel interface shared by decode.hip (kernel) and capi_decode.cpp (host).
#pragma once

#include "larql_hip_internal.h"

namespace larql {

struct AttnArgs {
    const float* qkv;  // pre-RoPE [q_dim | kv_dim | kv_dim]
    __half* kc;        // this layer's K cache [cap][num_kv][hd]
    __half* vc;        // this layer's V cache [cap / 8][num_kv][hd][8]
    float* out;        // [num_q * hd]
    float* part;       // [num_q][S][pst]: unnormalised o[hd], chunk max, chunk sum (attn_part_floats)
    int num_q, num_kv, hd, rdim;
    int T, t_begin, S;  // S is set by launch_attention
    int pst = 0;        // partial entry stride in floats (attn_partial_stride), set by launch_attention
    float scale;
    const float2* rope;  // [cap][rdim / 2] cos, sin (launch_rope_table)
    // Prompt mode (prefill): grid z = query position p of `batch`, T = T + p for query p,
    // the window start recomputed per query, qkv rows qkv_ld floats apart, every K/V row
    // (the query's own included) already in the cache, out rows num_q * hd apart and
    // partials [batch][num_q][S][pst] with S the largest query's split count.
    int batch = 0, window = 0, qkv_ld = 0;
    // Prompt-attention options of the reference's fused kernel (LC/src/metal/shaders/
    // fused_attention.rs:79-88, 132-137): qk_norm scales each RoPE'd query head by
    // 1 / sqrt(sum q^2 + 1e-6) (the cached K is not normed); softcap > 0 maps each scaled
    // score s to tanh(s / softcap) * softcap before the softmax.
    int qk_norm = 0;
    float softcap = 0.f;
};

void launch_attention(const AttnArgs& a, hipStream_t s);
// Position splits of one query (T positions from t_begin) and the most over a prompt's
// queries T0 .. T0 + batch - 1 (its partials stride).
int attn_splits(int T, int t_begin);
int attn_prompt_splits(int T0, int batch, int window);
// Floats per partial entry (o[hd], max, sum).  A partial buffer holds batch x num_q x S
// entries.
int attn_partial_stride(int hd);
inline size_t attn_part_floats(int num_q, int S, int hd, int batch = 1) {
    return static_cast<size_t>(batch) * num_q * S * attn_partial_stride(hd);
}
// cos/sin table for positions [0, cap): angle p * base^(-2i/rdim) in f64, as the CPU
// path computes it (LI/src/attention/rope.rs:22-55), rounded to f32.
void launch_rope_table(float2* cs, size_t cap, int rdim, double base, hipStream_t s);
// Head geometries the attention kernel takes: reps = num_q / num_kv in 1..8, hd a
// multiple of 32 up to 256.
bool attn_supported(int reps, int hd);
// K/V rows [seq][num_kv][hd] (f32 or fp16 bits) into the V cache layout.
void launch_v_to_cache(const void* src, bool src_f32, __half* dst, size_t seq, int num_kv, int hd, hipStream_t s);
void launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s);
// Row kernels of the batched prompt pass (prompt.hip).
// y = x / rms * (off + w) per row of n floats (w null: no weight).
void launch_rmsnorm_rows(const float* X, const float* w, float off, float* Y, size_t m, size_t n, double eps,
                         hipStream_t s);
// out = (h + v / rms(v) * (off + w)) * scale per row (the post-norm residual).
void launch_resid_norm_rows(const float* H, const float* V, const float* w, float off, float scale, float* out,
                            size_t m, size_t n, double eps, hipStream_t s);
// Parameter-free RMS norm of num_heads heads of hd floats, in place, in each of m rows ld apart.
void launch_vnorm_rows(float* X, size_t m, size_t ld, int num_heads, int hd, double eps, hipStream_t s);
void launch_rope_kv_rows(const float* QKV, size_t m, size_t p0, size_t q_dim, size_t kv_dim, int hd, int rdim,
                         const float2* rope, __half* kc, __half* vc, int num_kv, hipStream_t s);
void launch_add_rows(const float* a, const float* b, float* out, size_t n, hipStream_t s, float scale = 1.0f);
// act[i] = act(G[i]) * U[i] (separate gate and up buffers); kind 0 = SiLU, 1 = GELU-tanh.
void launch_gated_mul(const float* G, const float* U, float* act, size_t n, int kind, hipStream_t s);
// act[i] = act(GU[2i]) * GU[2i + 1]; kind 0 = SiLU, 1 = GELU-tanh.
void launch_gated_pair_rows(const float* GU, float* act, size_t n, int kind, hipStream_t s);
// Fused forms of the prompt pass, per row of n floats (n a multiple of 32, at most
// kFusedRowMax: the row is held in LDS), each value
// as the separate kernels compute it: hout = (hin + the projection row, its `splits`
// partial products summed in split order, pstride floats apart) * scale; then, with xn,
// xn = hout / rms(hout) * (off + w) and xn's GEMM row statistics into st.
constexpr int kFusedRowMax = 16384;
void launch_resid_norm_stats_rows(const float* P, size_t pstride, int splits, const float* hin, float scale,
                                  float* hout, const float* w, float off, float* xn, size_t m, size_t n, double eps,
                                  const GemmRowStats& st, hipStream_t s);
// act rows (m x n) as launch_gated_pair_rows, with their GEMM row statistics into st.
void launch_gated_pair_stats_rows(const float* GU, float* act, size_t m, size_t n, int kind, const GemmRowStats& st,
                                  hipStream_t s);
void launch_f32_to_f16(const float* src, __half* dst, size_t n, hipStream_t s);

}  // namespace larql
