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
    int* counter;      // [num_kv], zero between launches
    int num_q, num_kv, hd, rdim;
    int T, t_begin, S;  // S is set by launch_attention
    float scale;
    double rope_base;
};

void launch_attention(const AttnArgs& a, hipStream_t s);
size_t attn_lds_bytes(int reps, int hd, int rdim);
void launch_copy_f32(const float* src, float* dst, size_t n, hipStream_t s);
void launch_f32_to_f16(const float* src, __half* dst, size_t n, hipStream_t s);

}  // namespace larql
