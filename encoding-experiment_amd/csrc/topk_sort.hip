// Top-k for k above the selection kernels' bound (LARQL_HIP_TOPK_MAX): the reference
// ranks a row with select_nth_unstable_by + sort_unstable_by and clamps k only to the row
// length (LV/src/index/gate.rs:307-316; range-filtered callers ask for top_k * 10,
// gate.rs:300).  Every row's order keys (order_key, knn.h) are sorted descending by a
// stable segmented radix sort (rocPRIM through hipCUB), each element carrying its index,
// so equal keys keep ascending index order: the order of the selection kernels.  The
// first min(k, n) of each row are gathered with their scores.
#include "knn.h"  // the HIP runtime headers first: hipCUB picks its rocPRIM backend from them

#include <hipcub/device/device_segmented_radix_sort.hpp>

namespace larql {

namespace {

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// keys[r][i] = order_key(S[r][i]), vals[r][i] = i, offs[r] = r n (r <= rows).
template <bool SG>
__global__ void topk_keys_kernel(const float* __restrict__ S, size_t rows, size_t stride, int n,
                                 uint32_t* __restrict__ keys, uint32_t* __restrict__ vals, int* __restrict__ offs) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i <= rows) offs[i] = static_cast<int>(i * n);
    if (i >= rows * n) return;
    const size_t r = i / n, j = i - r * n;
    keys[i] = order_key<SG>(S[r * stride + j]);
    vals[i] = static_cast<uint32_t>(j);
}

// The first min(k, n) sorted entries of each row and their scores; slots past n hold
// index 0xFFFFFFFF and score 0.
__global__ void topk_gather_kernel(const float* __restrict__ S, size_t rows, size_t stride, int n, size_t k,
                                   const uint32_t* __restrict__ sorted, uint32_t* __restrict__ idx,
                                   float* __restrict__ val) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i >= rows * k) return;
    const size_t r = i / k, j = i - r * k;
    if (j < static_cast<size_t>(n)) {
        const uint32_t t = sorted[r * n + j];
        idx[i] = t;
        val[i] = S[r * stride + t];
    } else {
        idx[i] = 0xFFFFFFFFu;
        val[i] = 0.f;
    }
}

size_t sort_temp_bytes(size_t rows, int n) {
    size_t tb = 0;
    LARQL_HIP_CHECK(hipcub::DeviceSegmentedRadixSort::SortPairsDescending(
        nullptr, tb, static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr),
        static_cast<const uint32_t*>(nullptr), static_cast<uint32_t*>(nullptr), static_cast<int>(rows * n),
        static_cast<int>(rows), static_cast<const int*>(nullptr), static_cast<const int*>(nullptr), 0, 32,
        static_cast<hipStream_t>(nullptr)));
    return tb;
}

}  // namespace

size_t topk_sorted_work_bytes(size_t rows, int n) {
    if (n < 1 || rows == 0 || rows * static_cast<size_t>(n) >= (size_t{1} << 31))
        fail(LARQL_HIP_ERR_INVALID, "top-k: rows x n must be below 2^31 for k above LARQL_HIP_TOPK_MAX");
    const size_t items = rows * static_cast<size_t>(n);
    return 4 * align256(items * sizeof(uint32_t)) + align256((rows + 1) * sizeof(int)) + sort_temp_bytes(rows, n);
}

void launch_topk_sorted(const float* S, size_t rows, size_t row_stride, int n, size_t k, int signed_mode,
                        uint32_t* idx, float* val, void* work, size_t work_bytes, hipStream_t s) {
    if (k < 1) fail(LARQL_HIP_ERR_INVALID, "top-k: k must be at least 1");
    if (rows == 0) return;
    const size_t need = topk_sorted_work_bytes(rows, n);
    if (!work || work_bytes < need) fail(LARQL_HIP_ERR_INVALID, "top-k: sort work buffer too small");
    const size_t items = rows * static_cast<size_t>(n);
    uint8_t* p = static_cast<uint8_t*>(work);
    uint32_t* keys_in = reinterpret_cast<uint32_t*>(p);
    uint32_t* keys_out = reinterpret_cast<uint32_t*>(p + align256(items * 4));
    uint32_t* vals_in = reinterpret_cast<uint32_t*>(p + 2 * align256(items * 4));
    uint32_t* vals_out = reinterpret_cast<uint32_t*>(p + 3 * align256(items * 4));
    int* offs = reinterpret_cast<int*>(p + 4 * align256(items * 4));
    void* temp = p + 4 * align256(items * 4) + align256((rows + 1) * sizeof(int));
    size_t tb = need - (4 * align256(items * 4) + align256((rows + 1) * sizeof(int)));
    const size_t nk = items > rows ? items : rows + 1;
    const dim3 g1(static_cast<unsigned>((nk + 255) / 256));
    if (signed_mode) topk_keys_kernel<true><<<g1, dim3(256), 0, s>>>(S, rows, row_stride, n, keys_in, vals_in, offs);
    else topk_keys_kernel<false><<<g1, dim3(256), 0, s>>>(S, rows, row_stride, n, keys_in, vals_in, offs);
    LARQL_HIP_CHECK(hipGetLastError());
    LARQL_HIP_CHECK(hipcub::DeviceSegmentedRadixSort::SortPairsDescending(
        temp, tb, keys_in, keys_out, vals_in, vals_out, static_cast<int>(items), static_cast<int>(rows), offs,
        offs + 1, 0, 32, s));
    const size_t no = rows * k;
    topk_gather_kernel<<<dim3(static_cast<unsigned>((no + 255) / 256)), dim3(256), 0, s>>>(S, rows, row_stride, n, k,
                                                                                         vals_out, idx, val);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
