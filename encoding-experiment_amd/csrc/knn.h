// Gate-KNN kernel interface shared by knn.hip (kernels) and capi_knn.cpp (host).
#pragma once

#include "larql_hip_internal.h"

namespace larql {

constexpr int kMaxKnnLayers = LARQL_HIP_KNN_MAX_LAYERS;
constexpr int kTopkMaxK = LARQL_HIP_TOPK_MAX;

// Per-layer device pointers, passed by value in the kernel arguments.
struct KnnLayers {
    const void* p[kMaxKnnLayers];
};

// S[l][q][f] = G_l[f, :] . X[q, :], one fma chain over k from +0 per element.
void launch_gate_scores_f32(const KnnLayers& g, int n_layers, const float* X, float* S, int F, int K, int Q,
                            hipStream_t s);
// S[l][q][f] = sum_b (float)isum * (f16(scale) * XS[q][b]) in block order (Q4_0 x Q8).
// XA / XSP: work buffers of q4_xa_bytes / q4_xsp_bytes (the queries as MFMA operands).
void launch_gate_scores_q4(const KnnLayers& nibbles, const KnnLayers& scales, int n_layers, const int8_t* X8,
                           const float* XS, uint4* XA, float* XSP, float* S, int F, int K, int Q, hipStream_t s);
size_t q4_xa_bytes(int K, int Q);
size_t q4_xsp_bytes(int K, int Q);
// Top-k of `rows` rows of n scores (row stride row_stride floats), 1 <= k <= kTopkMaxK:
// min(k, n) entries per output row of k slots, the rest index 0xFFFFFFFF and score 0.
void launch_topk(const float* S, size_t rows, size_t row_stride, int n, int k, int signed_mode, uint32_t* idx,
                 float* val, hipStream_t s);

}  // namespace larql
