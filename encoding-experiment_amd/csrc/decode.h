// Attention kernel interface shared by decode.hip (kernel) and capi_decode.cpp (host).
#pragma once

#include "larql_hip_internal.h"

namespace larql {

struct AttnArgs {
    const float* qkv;  // pre-RoPE [q_dim | kv_dim | kv_dim]
    __half* kc;        // this layer's cache [cap][num_kv][hd]
    __half* vc;
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
size_t attn_lds_bytes(int reps, int hd, int rdim);
void launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s);
void launch_f32_to_f16(const float* src, __half* dst, size_t n, hipStream_t s);

}  // namespace larql
