// Attention kernel interface shared by decode.hip (kernel) and capi_decode.cpp (host).
#pragma once

#include "larql_hip_internal.h"

namespace larql {

struct AttnArgs {
    const float* qkv;  // pre-RoPE [q_dim | kv_dim | kv_dim]
    __half* kc;        // this layer's K cache [cap][num_kv][hd]
    __half* vc;        // this layer's V cache [cap / 8][num_kv][hd][8]
    float* out;        // [num_q * hd]
    float* part;       // [num_q][S][hd + 2]: unnormalised o, chunk max, chunk sum
    int num_q, num_kv, hd, rdim;
    int T, t_begin, S;  // S is set by launch_attention
    float scale;
    const float2* rope;  // [cap][rdim / 2] cos, sin (launch_rope_table)
};

void launch_attention(const AttnArgs& a, hipStream_t s);
// cos/sin table for positions [0, cap): angle p * base^(-2i/rdim) in f64, as the CPU
// path computes it (LI/src/attention/rope.rs:22-55), rounded to f32.
void launch_rope_table(float2* cs, size_t cap, int rdim, double base, hipStream_t s);
// Head geometries the attention kernel takes: reps = num_q / num_kv in 1..8, hd a
// multiple of 32 up to 256.
bool attn_supported(int reps, int hd);
// K/V rows [seq][num_kv][hd] (f32 or fp16 bits) into the V cache layout.
void launch_v_to_cache(const void* src, bool src_f32, __half* dst, size_t seq, int num_kv, int hd, hipStream_t s);
void launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s);
void launch_f32_to_f16(const float* src, __half* dst, size_t n, hipStream_t s);

}  // namespace larql
