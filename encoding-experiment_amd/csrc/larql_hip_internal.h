// Internal declarations shared by the HIP kernels and the C ABI of liblarql_hip.
//
// Device layouts ("dev layouts") are what a registered weight looks like in HBM.
// Every quantized format is repacked once, at registration, from the reference's
// byte layout (LC/src/cpu/ops/q4_common.rs) into structure-of-arrays form so the
// kernels issue 16-byte aligned, wave-contiguous loads:
//
//   Q4_K (148 B / 256 elems in the reference), tile-major over 16-row tiles:
//     qs  : u8 [rows/16][S][2][64][16]  nibble bytes: for row 16t + c, sub-block j of
//                                       super-block sb sits at [t][sb][j/4][16(j%4) + c],
//                                       16 bytes in reference order (element 2i low,
//                                       2i+1 high nibble of byte i)
//     hdr : u32x4 [rows/16][S][16]      {d|dmin<<16, sc[0..3], sc[4..7], min bytes}
//   so that one wave-wide 16-byte load of a (tile, super-block) reads 1 KB of
//   contiguous memory (the matrix-core matvec's B operand, one sub-block per lane).
//   Q6_K (210 B / 256), tile-major over 16-row tiles: one 3360-byte block per
//     (tile, super-block) holding its 16 rows' ql, regrouped qh, scales and d
//     (q6k_block below gives the block's offset and its internal layout)
//   Q4_0 (18 B / 32):
//     qs  : u8 [rows][B*16]       nibble bytes
//     d   : f16 [rows][B]         block scale
//   Q8_0 (trait form: i8 + separate f32 scales), tile-major over 16-row tiles and block
//     pairs (q8_piece / q8_scale_index below)
// where S = cols/256 and B = cols/32.  Rows are zero-padded to rows_pad (a multiple
// of 64) so matvec tiles load without row tests; padding rows decode to zero.
// The algorithmic byte count of every format stays the reference's; the Q4_K
// device layout drops the four unused scale bytes of each super-block (144 of
// 148 bytes are moved).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/larql_hip.h"

namespace larql {

// ── errors ──────────────────────────────────────────────────────────────
struct Error {
    int code;
    std::string msg;
};

#define LARQL_HIP_CHECK(expr)                                                        \
    do {                                                                             \
        hipError_t _e = (expr);                                                      \
        if (_e != hipSuccess)                                                        \
            throw ::larql::Error{LARQL_HIP_ERR_DEVICE,                               \
                                 std::string(#expr) + ": " + hipGetErrorString(_e)}; \
    } while (0)

[[noreturn]] inline void fail(int code, const std::string& msg) { throw Error{code, msg}; }

// ── device layouts ──────────────────────────────────────────────────────
struct DevWeight {
    int format = 0;          // larql_quant_format
    size_t rows = 0, cols = 0;
    size_t rows_pad = 0;     // rows rounded up to a multiple of 64
    void* base = nullptr;    // one device allocation holding all sub-arrays
    size_t bytes = 0;
    // sub-array pointers into `base`
    uint8_t* qs = nullptr;   // Q4_K/Q4_0 nibbles, Q6_K tile-major blocks (q6k_block), Q8_0 int8
    uint4* hdr = nullptr;    // Q4_K / Q4_KF headers
    int hf = 0;              // Q4_K-family header form: kHdr148, kHdrGguf or kHdrKf160
    void* d = nullptr;       // Q4_0 f16 scales, Q8_0 f32 scales
    // registry keys
    const void* host_ptr = nullptr;
    size_t host_len = 0;
    uint64_t host_fp = 0;    // sampled content fingerprint of the host bytes
    uint64_t handle = 0;
};

// FNV-1a over the whole buffer when it is small, else over 64 evenly spaced
// 64-byte samples: a cache hit on a reused host address with different bytes
// re-uploads instead of serving stale weights.
uint64_t host_fingerprint(const void* data, size_t len);

// Q4_K-family header forms in the device layout (DevWeight::hf):
//   kHdr148  : 148-byte Q4_K: uint4 {d | dmin << 16, sc 0..3, sc 4..7 (6-bit bytes),
//              min bytes m_j | m_{j+4} << 4}
//   kHdrGguf : 144-byte GGUF Q4_KF: the same uint4 with 6-bit mins, whose top two bits sit
//              in the top two bits of the scale bytes (m_j >> 4 above sc_j)
//   kHdrKf160: 160-byte Q4_KF: two uint4 {8 x f16 d*sc_j} {8 x f16 dmin*m_j} per row and
//              super-block
constexpr int kHdr148 = 0, kHdrGguf = 1, kHdrKf160 = 2;
// Bytes per 256-element block of a Q4_K-family header form in the reference layout.
inline size_t q4k_family_block_bytes(int hf) { return hf == kHdrKf160 ? 160 : hf == kHdrGguf ? 144 : 148; }
// Q4_KF carries two byte layouts (LC/src/pipeline.rs:15 says 160 bytes, the GPU decode
// kernels read 144, LC/src/metal/shaders/q4kf_qkv_proj.rs:46), told apart by length: a
// buffer of exactly rows x blocks x 160 bytes is the pre-baked form, exactly x 144 the GGUF
// form; any other length is ambiguous (a 160-byte buffer with slack would read as GGUF
// blocks) and is refused (q4kf_form_checked).
inline int q4kf_form(size_t len, size_t rows, size_t cols) {
    const size_t blocks = rows * (cols / 256);
    return len == blocks * 160 ? kHdrKf160 : len == blocks * 144 ? kHdrGguf : -1;
}
inline int q4kf_form_checked(size_t len, size_t rows, size_t cols) {
    const int hf = q4kf_form(len, rows, cols);
    if (hf < 0)
        fail(LARQL_HIP_ERR_INVALID, "Q4_KF buffer of " + std::to_string(len) + " bytes: must be exactly rows x " +
                                        std::to_string(cols / 256) + " blocks x 144 (GGUF) or x 160 (pre-baked)");
    return hf;
}
size_t ref_row_bytes(int format, size_t cols, int hf = kHdr148);   // bytes per row in the reference layout
// f32 gate rows on the device: cols rounded up to a multiple of 16 (the score kernel's
// k-stage), the extra columns -0.0; a query row is padded with +0.0 to match, so every
// padded term of a score's fma chain adds -0.0 (the additive identity) and the scores
// keep their bits.
inline size_t f32_row_stride(size_t cols) { return (cols + 15) & ~size_t(15); }
// dst[r][k] = src[r][k] for k < K, `pad` for K <= k < Kp (rows x Kp floats).
void launch_pad_rows_f32(const float* src, float* dst, size_t rows, size_t K, size_t Kp, float pad, hipStream_t s);
size_t dev_layout_bytes(int format, size_t rows_pad, size_t cols, int hf = kHdr148);
inline size_t pad_rows(size_t rows) { return (rows + 63) & ~size_t(63); }

// Q4_K tile-major layout: byte offset of sub-block j (0..7) of super-block sb of `row`
// in qs, and the index of its header in hdr (S = super-blocks per row).
__host__ __device__ inline size_t q4k_sub_offset(size_t row, size_t sb, int j, size_t S) {
    return ((((row >> 4) * S + sb) * 2 + static_cast<size_t>(j >> 2)) << 10) +
           ((16 * static_cast<size_t>(j & 3) + (row & 15)) << 4);
}
__host__ __device__ inline size_t q4k_hdr_index(size_t row, size_t sb, size_t S) {
    return ((row >> 4) * S + sb) * 16 + (row & 15);
}

// Q6_K device layout: one 3360-byte block per (16-row tile, super-block), in tile-major
// order (tile t, super-block sb at index t S + sb): [ql 2048][qh 1024][scales 256][d 32].
// Row c (0..15) of the tile, lane group g (0..3) = elements 64 g .. 64 g + 63:
//   ql bytes 32 g + 16 h .. + 15 (h = 0, 1)  at h * 1024 + (16 g + c) * 16,
//   qh group words 4 g .. 4 g + 3             at 2048 + (16 g + c) * 16
//     (word j: element 16 j + 8 w + 2 i + p at bits 8 i + 4 w + 2 p),
//   int8 scales 4 g .. 4 g + 3                at 3072 + (16 g + c) * 4,
//   f16 d                                     at 3328 + 2 c,
// so the load of one part by the 64 lanes (16 g + c) of a wave is one contiguous span.
constexpr size_t kQ6Block = 3360;
constexpr size_t kQ6Qh = 2048, kQ6Sc = 3072, kQ6D = 3328;
__host__ __device__ inline size_t q6k_block(size_t row, size_t sb, size_t S) {
    return ((row >> 4) * S + sb) * kQ6Block;
}

// Q8_0 device layout: one 1 KB chunk per (16-row tile t, block pair p) at (t P + p) * 1024,
// P = ceil(B / 2): piece g (0, 1 = block 2p bytes 0-15, 16-31; 2, 3 = block 2p + 1) of
// row c of the tile at g * 256 + c * 16, so one wave-wide 16-byte load of a chunk (lane
// 16 g + c) or of four pieces (16 rows each) reads contiguous runs of 256 bytes or more.
// Scales: the pair {d[2p], d[2p + 1]} of row c at float ((t P + p) * 16 + c) * 2.  The
// second block of a pair past an odd block count is zeros.
__host__ __device__ inline size_t q8_pairs(size_t nb) { return (nb + 1) / 2; }
__host__ __device__ inline size_t q8_piece(size_t row, size_t blk, int half, size_t P) {
    return (((row >> 4) * P + (blk >> 1)) << 10) + ((((blk & 1) * 2 + static_cast<size_t>(half)) * 16 + (row & 15)) << 4);
}
__host__ __device__ inline size_t q8_scale_index(size_t row, size_t blk, size_t P) {
    return (((row >> 4) * P + (blk >> 1)) * 16 + (row & 15)) * 2 + (blk & 1);
}

// Compute units of the current device (queried once per device, then cached).
int current_device_cus();
void dev_layout_carve(DevWeight& w);              // set sub-array pointers from base

// Repack reference-layout bytes already on the device (`raw`, src_rows rows; 0 = w.rows)
// into `w`, source row r landing in destination row row0 + r*stride.
void launch_repack(const DevWeight& w, const uint8_t* raw, const float* q8_scales, hipStream_t s,
                   size_t src_rows = 0, size_t row0 = 0, size_t stride = 1);

// ── KV cache ────────────────────────────────────────────────────────────
// cos / sin of the split-half RoPE angles for positions [0, cap): float2 [cap][rdim/2].
struct RopeTable {
    double base = 0.0;
    int rdim = 0;
    size_t cap = 0;
    float2* cs = nullptr;
};

struct KVCache {
    size_t num_layers = 0, max_seq = 0;
    size_t current_len = 0;
    std::vector<__half*> k, v;   // per layer: K [max_seq][num_kv][head_dim], V [max_seq / 8][num_kv][head_dim][8]
    std::vector<size_t> num_kv, head_dim;  // per layer (layers may differ, LC/src/metal/ops/kv_cache.rs:12-19)
    std::vector<RopeTable> rope;  // one per (rope_base, rdim) in use, cap >= max_seq
};

// ── context ─────────────────────────────────────────────────────────────
struct DeviceBuf {
    void* p = nullptr;
    size_t n = 0;
};

}  // namespace larql

struct larql_hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::recursive_mutex mu;
    std::string last_error;
    std::string device_name;
    int num_cus = 0;
    uint64_t next_handle = 1;
    std::unordered_map<uint64_t, larql::DevWeight> weights;
    std::map<std::pair<const void*, size_t>, uint64_t> by_host;
    // reusable device staging buffers for host-pointer calls
    larql::DeviceBuf stage_in, stage_in2, stage_out, stage_raw, scratch;
    // gate-KNN work buffers: scores [layers][nq][features], quantized queries, f32 queries
    // padded to the gate row stride
    larql::DeviceBuf knn_scores, knn_q8, knn_q8s, knn_idx, knn_val, knn_handles, knn_xa, knn_xsp, knn_xpad, knn_sort, knn_cand;
    // q4_vecmat chunk partials; pair-batch quantized activations
    larql::DeviceBuf vecmat_part, pair_q8, pair_q8s;
    // prefill GEMM: X as fp16 MFMA operands
    larql::DeviceBuf gemm_x16;
    larql::KVCache kv;
    // the cache-less full pipeline (full_pipeline_q4) runs its positions against this one,
    // leaving the decode cache `kv` untouched
    larql::KVCache kv_aside;
    // multi_layer_q4_ffn work buffer
    larql::DeviceBuf ffn_work;
    // model built by the last host-pointer decode_token (re-used while its key matches)
    larql_hip_model* trait_model = nullptr;
};

namespace larql {
// Records this device's address of the allocation-free entry points' fixed device array
// (capi_knn.cpp); run once per device by context creation, with the device current.
void noalloc_scratch_init(int device);
}  // namespace larql

// Frees the decode-side state of a context (trait model, KV cache).
void larql_hip_decode_release(larql_hip_ctx* c);

namespace larql {

void* ensure(larql_hip_ctx* c, DeviceBuf& b, size_t bytes);
const DevWeight& lookup(larql_hip_ctx* c, uint64_t handle);
// Find or create a device copy of reference-layout host bytes (Metal-style cache
// keyed by host pointer and length, LC/src/metal/buffers.rs:37-85).
const DevWeight& cached_weight(larql_hip_ctx* c, int format, const void* data, size_t len,
                               const float* q8_scales, size_t rows, size_t cols);

// ── kernel launchers (device pointers; enqueue only) ───────────────────
// m > 1 runs the prefill GEMM and needs `ws` of q4k_gemm_ws_bytes(m, cols) bytes.
void launch_q4k_matvec(const DevWeight& w, const float* x, float* out, size_t m, void* ws, hipStream_t s);
void launch_q6k_matvec(const DevWeight& w, const float* x, float* out, size_t m, hipStream_t s);
// Plain-read floor of a Q4_K-family weight: its device bytes read once by `groups`
// workgroups of `threads` (both 0: the matvec's launch shape), one XOR fold per
// workgroup into out[0 .. groups).
void launch_q4k_read_floor(const DevWeight& w, uint32_t* out, size_t out_words, unsigned groups, unsigned threads,
                           int num_cus, hipStream_t s);
// C[m][n] = A[m][k] . B (B [k][n], or [n][k] transposed), f32 fma chains in k order
// (f32_gemm.hip).
void launch_f32_matmul(const float* A, const float* B, float* C, size_t m, size_t k, size_t n, bool transpose_b,
                       hipStream_t s);
// Y[m][rows] = X[m][cols] . deq(W)^T, Q4_K, on MFMA (prefill.hip); ws holds X as fp16
// MFMA operands.
size_t q4k_gemm_ws_bytes(size_t m, size_t cols);
void launch_q4k_gemm(const DevWeight& w, const float* X, float* Y, size_t m, void* ws, hipStream_t s);
// The same product from f32 X at f32 accuracy (fp16 operand pairs, three products each,
// X rows scaled into range by per-token powers of two): ~1e-6 instead of ~1e-4, for
// chains of projections (the batched prompt pass).  `part` is the workspace (floats:
// q4k_gemm_f32_part_floats): the m row exponents, and the partial products when small
// grids split K over up to four workgroups per tile (summed in split order).
size_t q4k_gemm_f32_part_floats(const DevWeight& w, size_t m);
// Row statistics of an f32-accuracy GEMM input (row exponents; the scaled sub-block sums
// that Q4_K weights use, m x cols / 32 floats from a 16-byte boundary), computed by a
// caller that fuses them into the kernel producing the input: the floats of workspace
// for m rows of `cols`, their place in it, and the standalone computation.
struct GemmRowStats {
    int* xe;
    float* xs;
};
size_t gemm_row_stats_floats(size_t m, size_t cols);
GemmRowStats gemm_row_stats_at(float* ws, size_t m, size_t cols);
void launch_gemm_row_stats(const float* X, size_t m, size_t cols, const GemmRowStats& st, hipStream_t s);
// K-split partial products left to the caller to sum in split order (splits 1: part null,
// Y was written): split z of row r at part + (z m + r) rows.
struct GemmSplits {
    const float* part;
    int splits;
};
// Q4_K or Q6_K weights.  Y rows are ldy floats apart (0: w.rows), so a projection can
// fill a column slice.  pre: X's row statistics, already computed (for Q4_K weights with
// the sub-block sums).  defer: leave the split partial products unsummed (ldy = w.rows).
void launch_q4k_gemm_f32(const DevWeight& w, const float* X, float* Y, size_t m, float* part, size_t part_floats,
                         hipStream_t s, size_t ldy = 0, const GemmRowStats* pre = nullptr,
                         GemmSplits* defer = nullptr);
void launch_q4_0_matvec(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out,
                        size_t m, hipStream_t s);
// Two Q4_0 matrices of one shape times the same Q8 rows, in one launch per pass.
void launch_q4_0_matvec_pair(const DevWeight& w1, const DevWeight& w2, const int8_t* q8x, const float* q8s,
                             float* out1, float* out2, size_t m, hipStream_t s);
void launch_q8_matvec(const DevWeight& w, const int8_t* q8x, const float* q8s, float* out,
                      size_t m, hipStream_t s);
// Q4_0 weights x f32 activation (one row of x), the reference GPU's q4_f32_matvec.
void launch_q4_0_f32_matvec(const DevWeight& w, const float* x, float* out, hipStream_t s);
void launch_quantize_q8(const float* x, size_t n, size_t m, int8_t* q8, float* scales, hipStream_t s);
// q4_vecmat: chunks of rows per partial (q4_vecmat_chunks) and the two-pass launch;
// part holds chunks x cols floats.
size_t q4_vecmat_chunks(size_t inter, size_t hidden);
void launch_q4_vecmat(const DevWeight& w, const float* act, float* out, float* part, size_t chunks, hipStream_t s);
void launch_quantize_weights(int format, const float* x, size_t n, void* out, float* q8_scales, hipStream_t s);

}  // namespace larql
