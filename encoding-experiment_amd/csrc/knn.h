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
// Top-k order key of a score: the f32 bit pattern of |s| (abs mode, SG false; -0 and +0
// equal), or an order-preserving map of s (signed mode); larger key = earlier, ties by
// ascending index.
template <bool SG>
__device__ __forceinline__ uint32_t order_key(float v) {
    uint32_t b = __float_as_uint(v);
    if constexpr (!SG) return b & 0x7FFFFFFFu;
    if ((b & 0x7FFFFFFFu) == 0) b = 0;  // -0 == +0
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Top-k of `rows` rows of n scores (row stride row_stride floats), 1 <= k <= kTopkMaxK:
// min(k, n) entries per output row of k slots, the rest index 0xFFFFFFFF and score 0.
// Rows longer than one selection kernel's registers run in chunks on many CUs when
// candidate buffers of topk_candidate_slots(rows, n, k) entries are given (else one
// workgroup streams each row).
void launch_topk(const float* S, size_t rows, size_t row_stride, int n, int k, int signed_mode, uint32_t* idx,
                 float* val, hipStream_t s, uint32_t* cand_idx = nullptr, float* cand_val = nullptr);
size_t topk_candidate_slots(size_t rows, int n, int k);
// The same order for any k >= 1 (topk_sort.hip): a stable segmented radix sort of every
// row's keys, descending, then the first min(k, n) of each row.  work: work_bytes of
// device memory, at least topk_sorted_work_bytes(rows, n); rows * n < 2^31.
size_t topk_sorted_work_bytes(size_t rows, int n);
void launch_topk_sorted(const float* S, size_t rows, size_t row_stride, int n, size_t k, int signed_mode,
                        uint32_t* idx, float* val, void* work, size_t work_bytes, hipStream_t s);

}  // namespace larql
