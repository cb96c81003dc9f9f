// Q4_0 vector x matrix: out[hidden] = act[inter] . deq(W[inter, hidden]), the trait's
// q4_vecmat (LC/src/backend.rs:56-60 -> LC/src/cpu/ops/q4_vecmat.rs:8-18 ->
// LC/csrc/q4_dot.c:201-232; ARM :130-164).
//
// Reference semantics: rows whose activation lies in (-1e-10, 1e-10) are skipped, and
// each term is (nib - 8) * (f16(d) * act).  The reference adds the rows into each
// output in row order, one long serial chain per column (and its ARM build contracts
// the add into an fma, so its two builds already disagree in the last bits); here each
// lane forms sum(nib * s) with fmas and subtracts 8 * sum(s) once, the rows are summed
// in chunks — sequentially within a wave, the four waves of a workgroup in order, then
// the chunk partials in a fixed grouping — so the result is deterministic and within
// f32 rounding of the reference (the bar is relative, 1e-3).
//
// Pass 1 (q4_vecmat_part_kernel): workgroup (tile, chunk) = 512 output columns x one
// chunk of rows, four waves each owning a quarter of the chunk's rows.  Lane l holds
// dword l % 4 of block l / 4 of the tile (8 outputs), so one row is a 256-byte
// contiguous read per wave.  The row's activation is wave-uniform (a scalar load),
// which makes the skip a uniform branch.
// Pass 2 (q4_vecmat_sum_kernel): out[k] = sum over chunks of part[chunk][k], chunk
// groups in parallel and their totals added in a fixed order.
#include "device_common.h"
#include "larql_hip_internal.h"


namespace larql {

namespace {

constexpr int kVmThreads = 256;
constexpr int kVmWaves = kVmThreads / 64;
constexpr int kVmTileCols = 512;   // 64 lanes x 8 outputs
constexpr int kVmRowsPerWave = 32;  // rows in flight per wave (all loaded before any arithmetic)

// Grid (ceil(hidden / 512), chunks).  part: [chunks][hidden].
__global__ __launch_bounds__(kVmThreads) void q4_vecmat_part_kernel(const uint32_t* __restrict__ qs,
                                                                    const uint16_t* __restrict__ dsc,
                                                                    const float* __restrict__ act,
                                                                    float* __restrict__ part, int inter, int hidden,
                                                                    int rows_per_chunk) {
    __shared__ float red[kVmWaves - 1][8][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = hidden >> 5;
    const int col0 = blockIdx.x * kVmTileCols + 8 * lane;  // first output of this lane
    const bool active = col0 < hidden;
    const int blk = min(col0, hidden - 8) >> 5;            // block column
    const int dw = (min(col0, hidden - 8) >> 3) & 3;       // dword within the block's 16 bytes
    // rows of this wave: a contiguous quarter of the chunk
    const int c0 = blockIdx.y * rows_per_chunk;
    const int c1 = min(inter, c0 + rows_per_chunk);
    const int per = (c1 - c0 + kVmWaves - 1) / kVmWaves;
    const int r0 = min(c1, c0 + wave * per), r1 = min(c1, r0 + per);

    float acc[8], ssum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    for (int rb = r0; rb < r1; rb += kVmRowsPerWave) {
        uint32_t q[kVmRowsPerWave];
        uint32_t d[kVmRowsPerWave];
        float a[kVmRowsPerWave];
#pragma unroll
        for (int k = 0; k < kVmRowsPerWave; k++) {
            const int row = min(rb + k, r1 - 1);
            const size_t b = static_cast<size_t>(row) * nb + blk;
            q[k] = qs[b * 4 + dw];
            d[k] = dsc[b];
            a[k] = act[row];
        }
#pragma unroll
        for (int k = 0; k < kVmRowsPerWave; k++) {
            const float av = a[k];
            if (rb + k >= r1 || (av > -1e-10f && av < 1e-10f)) continue;  // wave-uniform
            const float scale = h2f(d[k]) * av;
            // sum((nib - 8) * scale) as fma(nib, scale, acc) and 8 * sum(scale) once
            const uint32_t lo4 = q[k] & 0x0F0F0F0Fu, hi4 = (q[k] >> 4) & 0x0F0F0F0Fu;
            acc[0] = __builtin_fmaf(ubyte0(lo4), scale, acc[0]);
            acc[1] = __builtin_fmaf(ubyte0(hi4), scale, acc[1]);
            acc[2] = __builtin_fmaf(ubyte1(lo4), scale, acc[2]);
            acc[3] = __builtin_fmaf(ubyte1(hi4), scale, acc[3]);
            acc[4] = __builtin_fmaf(ubyte2(lo4), scale, acc[4]);
            acc[5] = __builtin_fmaf(ubyte2(hi4), scale, acc[5]);
            acc[6] = __builtin_fmaf(ubyte3(lo4), scale, acc[6]);
            acc[7] = __builtin_fmaf(ubyte3(hi4), scale, acc[7]);
            ssum = ssum + scale;
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = __builtin_fmaf(-8.0f, ssum, acc[i]);
    // the four waves' sums in wave order
    if (wave > 0) {
#pragma unroll
        for (int i = 0; i < 8; i++) red[wave - 1][i][lane] = acc[i];
    }
    __syncthreads();
    if (wave == 0 && active) {
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float v = acc[i];
#pragma unroll
            for (int w = 0; w < kVmWaves - 1; w++) v = v + red[w][i][lane];
            o[i] = v;
        }
        float4* dst = reinterpret_cast<float4*>(part + static_cast<size_t>(blockIdx.y) * hidden + col0);
        dst[0] = make_float4(o[0], o[1], o[2], o[3]);
        dst[1] = make_float4(o[4], o[5], o[6], o[7]);
    }
}

// out[k] = sum over chunks of part[c][k]: workgroup = 16 columns x 16 chunk groups;
// group g sums chunks g, g + 16, ... (eight loads in flight at a time), then the 16
// group totals are added in group order.
constexpr int kSumCols = 16, kSumGroups = 16;
__global__ __launch_bounds__(256) void q4_vecmat_sum_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                           int hidden, int chunks) {
    __shared__ float red[kSumGroups][kSumCols];
    const int col = threadIdx.x & (kSumCols - 1), g = threadIdx.x / kSumCols;
    const int k = blockIdx.x * kSumCols + col;
    const int kc = min(k, hidden - 1);
    float s = 0.0f;
    for (int c0 = g; c0 < chunks; c0 += 8 * kSumGroups) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = part[static_cast<size_t>(min(c0 + u * kSumGroups, chunks - 1)) * hidden + kc];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (c0 + u * kSumGroups < chunks) s = s + v[u];
    }
    red[g][col] = s;
    __syncthreads();
    if (g == 0 && k < hidden) {
        float t = red[0][col];
#pragma unroll
        for (int i = 1; i < kSumGroups; i++) t = t + red[i][col];
        out[k] = t;
    }
}

}  // namespace

// Chunks: two workgroups per CU (about 8 waves per CU) without letting the partials
// (4 bytes x chunks x hidden, written and read once) pass ~1/8 of the weight bytes
// (18/32 bytes per weight).  Measured on [10240 x 2560]: 14.0 / 10.9 / 12.5 us for one,
// two and four workgroups per CU.
size_t q4_vecmat_chunks(size_t inter, size_t hidden) {
    const size_t tiles = (hidden + kVmTileCols - 1) / kVmTileCols;
    const size_t want = std::max<size_t>(1, (static_cast<size_t>(current_device_cus()) * 2 + tiles - 1) / tiles);
    const size_t cap = std::max<size_t>(1, inter * 18 / (32 * 4 * 8));  // partials <= weights / 8
    return std::max<size_t>(1, std::min({want, cap, (inter + kVmWaves - 1) / kVmWaves}));
}

void launch_q4_vecmat(const DevWeight& w, const float* act, float* out, float* part, size_t chunks, hipStream_t s) {
    if (w.format != LARQL_Q4_0) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_vecmat: Q4_0 weights only");
    if (w.cols % 32 || w.cols == 0 || w.rows == 0) fail(LARQL_HIP_ERR_INVALID, "q4_vecmat: shape");
    if (w.rows > 0x7FFFFFFF / (w.cols / 32)) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_vecmat: matrix too large");
    const int inter = static_cast<int>(w.rows), hidden = static_cast<int>(w.cols);
    const int rows_per_chunk = static_cast<int>((w.rows + chunks - 1) / chunks);
    const int nch = (inter + rows_per_chunk - 1) / rows_per_chunk;
    const dim3 g1(static_cast<unsigned>((hidden + kVmTileCols - 1) / kVmTileCols), static_cast<unsigned>(nch));
    q4_vecmat_part_kernel<<<g1, dim3(kVmThreads), 0, s>>>(reinterpret_cast<const uint32_t*>(w.qs),
                                                          static_cast<const uint16_t*>(w.d), act, part, inter, hidden,
                                                          rows_per_chunk);
    LARQL_HIP_CHECK(hipGetLastError());
    q4_vecmat_sum_kernel<<<dim3(static_cast<unsigned>((hidden + kSumCols - 1) / kSumCols)), dim3(256), 0, s>>>(
        part, out, hidden, nch);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
