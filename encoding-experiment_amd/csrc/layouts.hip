// Registration-time repack: reference byte layouts -> device SoA layouts.
//
// Reference layouts (LC/src/cpu/ops/q4_common.rs):
//   Q4_0  18 B / 32  : [f16 scale][16 B nibbles]                              (:50-81)
//   Q4_K 148 B / 256 : [f16 d][f16 dmin][12 B sc (0..7 used)][4 B mins][128 B]  (:104-170)
//   Q6_K 210 B / 256 : [128 B ql][64 B qh][16 x i8 scales][f16 d]              (:179-239)
//                      (device: 3360-byte blocks per 16-row tile and super-block, q6k_block)
//   Q8_0 trait form  : i8 [rows*cols] + f32 scales [rows*cols/32]          (LC/src/pipeline.rs:22-27)
//                      (device: 1 KB chunks per 16-row tile and block pair, q8_piece)
//   Q4_KF 144 B / 256: llama.cpp GGUF block [f16 d][f16 dmin][12 B packed 6-bit scales and
//                      mins][128 B: chunk c of 32 bytes = sub-block 2c low, 2c+1 high
//                      nibbles]            (LC/src/metal/shaders/q4kf_qkv_proj.rs:87-119)
//   Q4_KF 160 B / 256: [8 x f16 d*sc_j][8 x f16 dmin*m_j][128 B nibbles as Q4_K] (q4_common.rs:370-413)
// Both Q4_KF forms land in the Q4_K tile-major nibble layout (sub-blocks in the 148-byte
// nibble order), so one matvec kernel reads all three, templated on the header form.
#include "larql_hip_internal.h"

namespace larql {

size_t ref_row_bytes(int format, size_t cols, int hf) {
    switch (format) {
        case LARQL_Q4_0: return cols / 32 * 18;
        case LARQL_Q4_K: return cols / 256 * 148;
        case LARQL_Q4_KF: return cols / 256 * q4k_family_block_bytes(hf);
        case LARQL_Q6_K: return cols / 256 * 210;
        case LARQL_Q8_0: return cols;
        case LARQL_F32: return cols * 4;
        default: return 0;
    }
}

static size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

size_t dev_layout_bytes(int format, size_t rows, size_t cols, int hf) {
    switch (format) {
        case LARQL_Q4_0: return align256(rows * cols / 2) + align256(rows * (cols / 32) * 2);
        case LARQL_Q4_K: return align256(rows * cols / 2) + align256(rows * (cols / 256) * 16);
        case LARQL_Q4_KF: return align256(rows * cols / 2) + align256(rows * (cols / 256) * (hf == kHdrKf160 ? 32 : 16));
        case LARQL_Q6_K: return align256(rows * (cols / 256) * 210);  // rows % 16 == 0: kQ6Block per tile
        case LARQL_Q8_0:  // rows % 16 == 0: q8_piece / q8_scale_index
            return align256(rows / 16 * q8_pairs(cols / 32) * 1024) + align256(rows / 16 * q8_pairs(cols / 32) * 128);
        case LARQL_F32: return align256(rows * f32_row_stride(cols) * 4);
        default: return 0;
    }
}

__global__ void pad_rows_f32_kernel(const float* __restrict__ src, float* __restrict__ dst, size_t rows, size_t K,
                                    size_t Kp, float pad) {
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i >= rows * Kp) return;
    const size_t r = i / Kp, k = i - r * Kp;
    dst[i] = k < K ? src[r * K + k] : pad;
}

void launch_pad_rows_f32(const float* src, float* dst, size_t rows, size_t K, size_t Kp, float pad, hipStream_t s) {
    const size_t n = rows * Kp;
    if (n == 0) return;
    pad_rows_f32_kernel<<<dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s>>>(src, dst, rows, K, Kp, pad);
    LARQL_HIP_CHECK(hipGetLastError());
}

void dev_layout_carve(DevWeight& w) {
    uint8_t* p = static_cast<uint8_t*>(w.base);
    const size_t R = w.rows_pad, K = w.cols;
    switch (w.format) {
        case LARQL_Q4_0:
            w.qs = p; p += align256(R * K / 2);
            w.d = p;
            break;
        case LARQL_Q4_K:
        case LARQL_Q4_KF:
            w.qs = p; p += align256(R * K / 2);
            w.hdr = reinterpret_cast<uint4*>(p);
            break;
        case LARQL_Q6_K:  // tile-major blocks (q6k_block)
            w.qs = p;
            break;
        case LARQL_Q8_0:
            w.qs = p; p += align256(R / 16 * q8_pairs(K / 32) * 1024);
            w.d = p;
            break;
        case LARQL_F32:
            w.qs = p;
            break;
        default: break;
    }
}

// One thread per Q4_K super-block.  Source blocks sit at 148-byte offsets, so they
// are 4-byte aligned whenever the raw buffer is.
// Source row r lands in destination row row0 + r*stride (concatenated or interleaved
// fused weights); bpr = blocks per row.
__device__ __forceinline__ size_t dst_block(size_t b, size_t bpr, size_t row0, size_t stride) {
    const size_t r = b / bpr;
    return (row0 + r * stride) * bpr + (b - r * bpr);
}

__global__ void repack_q4k_kernel(const uint32_t* __restrict__ raw, uint8_t* __restrict__ qs,
                                  uint4* __restrict__ hdr, size_t nblocks, size_t bpr, size_t row0, size_t stride) {
    size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint32_t* s = raw + b * 37;
    const size_t o = dst_block(b, bpr, row0, stride);
    const size_t row = o / bpr, sb = o - row * bpr;
    hdr[q4k_hdr_index(row, sb, bpr)] = make_uint4(s[0], s[1], s[2], s[4]);
#pragma unroll
    for (int j = 0; j < 8; j++)
        *reinterpret_cast<uint4*>(qs + q4k_sub_offset(row, sb, j, bpr)) =
            make_uint4(s[5 + 4 * j], s[6 + 4 * j], s[7 + 4 * j], s[8 + 4 * j]);
}

// One thread per GGUF (144-byte, llama.cpp layout) super-block: scales and 6-bit mins
// unpacked (get_scale_min_k4: j < 4: sc = q[j] & 63, m = q[j+4] & 63; j >= 4: sc =
// (q[j+4] & 15) | (q[j-4] >> 6) << 4, m = (q[j+4] >> 4) | (q[j] >> 6) << 4) into the kHdrGguf
// header, nibbles of sub-block j = 2c + h (nibble h of bytes 32c .. 32c + 31) regrouped into
// the 148-byte order (element 2i low, 2i + 1 high nibble of byte i).
__global__ void repack_q4kf_gguf_kernel(const uint32_t* __restrict__ raw, uint8_t* __restrict__ qs,
                                        uint4* __restrict__ hdr, size_t nblocks, size_t bpr, size_t row0,
                                        size_t stride) {
    size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint32_t* s = raw + b * 36;
    const size_t o = dst_block(b, bpr, row0, stride);
    const size_t row = o / bpr, sb = o - row * bpr;
    uint8_t q[12];
#pragma unroll
    for (int i = 0; i < 3; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) q[4 * i + k] = static_cast<uint8_t>(s[1 + i] >> (8 * k));
    uint32_t scw[2] = {0u, 0u}, mnw = 0u;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t sc = j < 4 ? (q[j] & 63u) : ((q[j + 4] & 15u) | ((q[j - 4] >> 6) << 4));
        const uint32_t mn = j < 4 ? (q[j + 4] & 63u) : ((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
        scw[j >> 2] |= (sc | ((mn >> 4) << 6)) << (8 * (j & 3));
        mnw |= (mn & 15u) << (8 * (j & 3) + 4 * (j >> 2));
    }
    hdr[q4k_hdr_index(row, sb, bpr)] = make_uint4(s[0], scw[0], scw[1], mnw);
    const uint8_t* n = reinterpret_cast<const uint8_t*>(s + 4);
    for (int j = 0; j < 8; j++) {
        const int c = j >> 1, sh = 4 * (j & 1);
        uint32_t d4[4];
        for (int w = 0; w < 4; w++) {
            uint32_t v = 0;
            for (int k = 0; k < 4; k++) {
                const int i = 4 * w + k;  // output byte i = elements 2i, 2i + 1 of the sub-block
                const uint32_t lo = (n[32 * c + 2 * i] >> sh) & 15u, hi = (n[32 * c + 2 * i + 1] >> sh) & 15u;
                v |= (lo | (hi << 4)) << (8 * k);
            }
            d4[w] = v;
        }
        *reinterpret_cast<uint4*>(qs + q4k_sub_offset(row, sb, j, bpr)) = make_uint4(d4[0], d4[1], d4[2], d4[3]);
    }
}

// One thread per 160-byte Q4_KF super-block: the two f16 octets (d*sc_j, dmin*m_j) as the
// kHdrKf160 header pair, nibbles (148-byte order) as Q4_K.
__global__ void repack_q4kf160_kernel(const uint32_t* __restrict__ raw, uint8_t* __restrict__ qs,
                                      uint4* __restrict__ hdr, size_t nblocks, size_t bpr, size_t row0,
                                      size_t stride) {
    size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint32_t* s = raw + b * 40;
    const size_t o = dst_block(b, bpr, row0, stride);
    const size_t row = o / bpr, sb = o - row * bpr;
    const size_t h = q4k_hdr_index(row, sb, bpr) * 2;
    hdr[h] = make_uint4(s[0], s[1], s[2], s[3]);
    hdr[h + 1] = make_uint4(s[4], s[5], s[6], s[7]);
#pragma unroll
    for (int j = 0; j < 8; j++)
        *reinterpret_cast<uint4*>(qs + q4k_sub_offset(row, sb, j, bpr)) =
            make_uint4(s[8 + 4 * j], s[9 + 4 * j], s[10 + 4 * j], s[11 + 4 * j]);
}

// One thread per Q6_K super-block (210-byte stride: 2-byte aligned source) into its row
// of the tile-major block (q6k_block).  The 64 qh bytes (element e at byte e/4, bits
// 2*(e%4)) are regrouped into 16 words, one per 16-element group j: element 16j + 8w +
// 2i + p goes to bits 8i + 4w + 2p.
__global__ void repack_q6k_kernel(const uint16_t* __restrict__ raw, uint8_t* __restrict__ blocks,
                                  size_t nblocks, size_t bpr, size_t row0, size_t stride) {
    size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint16_t* s = raw + b * 105;
    const size_t o = dst_block(b, bpr, row0, stride);
    const size_t row = o / bpr, sb = o - row * bpr, c = row & 15;
    uint8_t* blk = blocks + q6k_block(row, sb, bpr);
    for (int g = 0; g < 4; g++)
        for (int h = 0; h < 2; h++) {
            uint16_t* l = reinterpret_cast<uint16_t*>(blk + h * 1024 + (16 * g + c) * 16);
            for (int i = 0; i < 8; i++) l[i] = s[16 * g + 8 * h + i];
        }
    for (int j = 0; j < 16; j++) {
        // source: 16 elements = 4 bytes = u16 words s[64 + 2j] and s[64 + 2j + 1]
        const uint32_t src = static_cast<uint32_t>(s[64 + 2 * j]) | (static_cast<uint32_t>(s[64 + 2 * j + 1]) << 16);
        uint32_t dst = 0;
        for (int e = 0; e < 16; e++) {
            const uint32_t v = (src >> (2 * e)) & 3u;
            const int w = e >> 3, i = (e & 7) >> 1, p = e & 1;
            dst |= v << (8 * i + 4 * w + 2 * p);
        }
        *reinterpret_cast<uint32_t*>(blk + kQ6Qh + (16 * (j >> 2) + c) * 16 + 4 * (j & 3)) = dst;
    }
    for (int k = 0; k < 8; k++)  // scales 2k, 2k + 1
        *reinterpret_cast<uint16_t*>(blk + kQ6Sc + (16 * (k >> 1) + c) * 4 + 2 * (k & 1)) = s[96 + k];
    *reinterpret_cast<uint16_t*>(blk + kQ6D + 2 * c) = s[104];
}

// One thread per 16-byte piece (source row r, pair p, piece g) of a Q8_0 weight in the
// trait form (i8 [rows][cols], f32 scales [rows][B]) into the tile-major layout; the
// thread of piece 0 also moves the pair's two scales.  Byte loads: the source may sit at
// any offset.
__global__ void repack_q8_0_kernel(const int8_t* __restrict__ raw, const float* __restrict__ sc,
                                   uint8_t* __restrict__ qs, float* __restrict__ d, size_t src_rows, size_t nb,
                                   size_t row0) {
    const size_t P = q8_pairs(nb);
    const size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (i >= src_rows * P * 4) return;
    const int g = static_cast<int>(i & 3);
    const size_t p = (i >> 2) % P, r = (i >> 2) / P, row = row0 + r;
    const size_t blk = 2 * p + (g >> 1);
    uint32_t v[4] = {0, 0, 0, 0};
    if (blk < nb) {
        const int8_t* src = raw + r * nb * 32 + blk * 32 + (g & 1) * 16;
#pragma unroll
        for (int k = 0; k < 16; k++) v[k >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(src[k])) << (8 * (k & 3));
    }
    *reinterpret_cast<uint4*>(qs + q8_piece(row, blk, g & 1, P)) = make_uint4(v[0], v[1], v[2], v[3]);
    if (g == 0) {
        float* dst = d + q8_scale_index(row, 2 * p, P);
        dst[0] = sc[r * nb + 2 * p];
        dst[1] = 2 * p + 1 < nb ? sc[r * nb + 2 * p + 1] : 0.0f;
    }
}

// One thread per Q4_0 block (18-byte stride: 2-byte aligned source).
__global__ void repack_q4_0_kernel(const uint16_t* __restrict__ raw, uint8_t* __restrict__ qs,
                                   uint16_t* __restrict__ d, size_t nblocks, size_t bpr, size_t row0, size_t stride) {
    size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    const uint16_t* s = raw + b * 9;
    const size_t o = dst_block(b, bpr, row0, stride);
    d[o] = s[0];
    uint16_t* q = reinterpret_cast<uint16_t*>(qs + o * 16);
#pragma unroll
    for (int i = 0; i < 8; i++) q[i] = s[1 + i];
}

void launch_repack(const DevWeight& w, const uint8_t* raw, const float* q8_scales, hipStream_t s,
                   size_t src_rows, size_t row0, size_t stride) {
    const int T = 256;
    if (src_rows == 0) src_rows = w.rows;
    if (row0 + (src_rows - 1) * stride >= w.rows) fail(LARQL_HIP_ERR_INVALID, "repack: rows out of range");
    switch (w.format) {
        case LARQL_Q4_K: {
            const size_t bpr = w.cols / 256, nb = src_rows * bpr;
            repack_q4k_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(
                reinterpret_cast<const uint32_t*>(raw), w.qs, w.hdr, nb, bpr, row0, stride);
            break;
        }
        case LARQL_Q4_KF: {
            const size_t bpr = w.cols / 256, nb = src_rows * bpr;
            if (w.hf == kHdrKf160)
                repack_q4kf160_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(
                    reinterpret_cast<const uint32_t*>(raw), w.qs, w.hdr, nb, bpr, row0, stride);
            else
                repack_q4kf_gguf_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(
                    reinterpret_cast<const uint32_t*>(raw), w.qs, w.hdr, nb, bpr, row0, stride);
            break;
        }
        case LARQL_Q6_K: {
            const size_t bpr = w.cols / 256, nb = src_rows * bpr;
            repack_q6k_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(
                reinterpret_cast<const uint16_t*>(raw), w.qs, nb, bpr, row0, stride);
            break;
        }
        case LARQL_Q4_0: {
            const size_t bpr = w.cols / 32, nb = src_rows * bpr;
            repack_q4_0_kernel<<<dim3((nb + T - 1) / T), dim3(T), 0, s>>>(
                reinterpret_cast<const uint16_t*>(raw), w.qs, static_cast<uint16_t*>(w.d), nb, bpr, row0, stride);
            break;
        }
        case LARQL_Q8_0: {
            if (stride != 1) fail(LARQL_HIP_ERR_UNSUPPORTED, "repack: interleaved Q8_0");
            const size_t nb = w.cols / 32, n = src_rows * q8_pairs(nb) * 4;
            repack_q8_0_kernel<<<dim3(static_cast<unsigned>((n + T - 1) / T)), dim3(T), 0, s>>>(
                reinterpret_cast<const int8_t*>(raw), q8_scales, w.qs, static_cast<float*>(w.d), src_rows, nb, row0);
            break;
        }
        case LARQL_F32: {
            if (stride != 1) fail(LARQL_HIP_ERR_UNSUPPORTED, "repack: interleaved f32");
            const size_t Kp = f32_row_stride(w.cols);
            if (Kp == w.cols)
                LARQL_HIP_CHECK(hipMemcpyAsync(w.qs + row0 * w.cols * 4, raw, src_rows * w.cols * 4,
                                               hipMemcpyDeviceToDevice, s));
            else
                launch_pad_rows_f32(reinterpret_cast<const float*>(raw), reinterpret_cast<float*>(w.qs) + row0 * Kp,
                                    src_rows, w.cols, Kp, -0.0f, s);
            break;
        }
        default: fail(LARQL_HIP_ERR_UNSUPPORTED, "repack: unsupported format");
    }
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
