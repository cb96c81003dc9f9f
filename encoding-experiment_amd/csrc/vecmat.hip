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
// Pass 1 (q4_vecmat_part_kernel): workgroup (tile, chunk) = the output columns of 8
// blocks (256 outputs) x one chunk of rows.  Thread (g, b) owns block b of the tile (16
// bytes, 32 outputs) in rows g, g + G, g + 2 G, ... of the chunk, so a load instruction
// reads one whole 128-byte line of each of 8 rows.  Rows whose activation is skipped
// contribute a zero scale.  The G lane sums of each column are added in row-group order
// through LDS.  Narrow tiles keep the partials small (chunks x hidden floats, written and
// read once): whole-row workgroups need several times the chunks to fill the GPU, and at
// [10240 x 2560] their partials cost more than the row pieces save (14.4 us against 11.0).
// Pass 2 (q4_vecmat_sum_kernel): out[k] = sum over chunks of part[chunk][k], chunk
// groups in parallel and their totals added in a fixed order.  Folding it into pass 1
// (the last workgroup of a tile sums the tile, found by a device counter) measured
// slower: 14.9 us, the counter and the partial loads adding round trips after the last
// partial lands.
#include "device_common.h"
#include "larql_hip_internal.h"


namespace larql {

namespace {

constexpr int kVmTileBlocks = 8;     // blocks (of 32 columns) per tile
constexpr int kVmThreadsWant = 256;  // threads per workgroup
constexpr int kVmMaxThreads = 512;
constexpr int kVmR = 8;              // rows in flight per thread

// Tile width and row groups for a row of nb blocks; the LDS partial sums (G x 33 x tile
// floats) stay within 64 KB.
struct VmShape {
    int tb, groups, threads;
};
VmShape vecmat_shape(int nb) {
    VmShape v;
    v.tb = std::min(nb, kVmTileBlocks);
    v.groups = std::max(1, std::min(kVmThreadsWant / v.tb, 496 / v.tb));
    v.threads = (v.tb * v.groups + 63) / 64 * 64;
    return v;
}

// Grid tiles x chunks (one dimension), vecmat_shape threads.  part: [chunks][hidden].
// Workgroup i runs on XCD i % 8; with the chunk count a multiple of 8 every tile of a
// chunk runs on one XCD (chunk x + 8 k on XCD x), so the rows' scale lines, which the
// tiles of a row share (160 bytes per [.. x 2560] row), are fetched into one L2 instead
// of up to eight.
__global__ __launch_bounds__(kVmMaxThreads) void q4_vecmat_part_kernel(const uint4* __restrict__ qs,
                                                                       const uint16_t* __restrict__ dsc,
                                                                       const float* __restrict__ act,
                                                                       float* __restrict__ part, int inter, int hidden,
                                                                       int rows_per_chunk, int tb, int groups,
                                                                       int tiles, int nch) {
    extern __shared__ float red[];  // [groups][33 tb]: block b's 32 sums at 33 b
    const int t = threadIdx.x;
    const int nb = hidden >> 5;
    const int b = t % tb, g = t / tb;
    const int wg = static_cast<int>(blockIdx.x);
    int tile, chunk;
    if (nch % 8 == 0) {
        const int x = wg & 7, slot = wg >> 3;
        chunk = x + 8 * (slot / tiles);
        tile = slot % tiles;
    } else {
        chunk = wg / tiles;
        tile = wg % tiles;
    }
    const int blk = min(tile * tb + b, nb - 1);  // past the edge: a real block, unused
    const int c0 = chunk * rows_per_chunk;
    const int c1 = min(inter, c0 + rows_per_chunk);

    if (g < groups) {
        float acc[32], ssum = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; i++) acc[i] = 0.0f;
        for (int rb = c0 + g; rb < c1; rb += groups * kVmR) {
            uint4 q[kVmR];
            uint32_t d[kVmR];
            float a[kVmR];
#pragma unroll
            for (int k = 0; k < kVmR; k++) {
                const int row = min(rb + k * groups, c1 - 1);
                const size_t bi = static_cast<size_t>(row) * nb + blk;
                q[k] = qs[bi];
                d[k] = dsc[bi];
                a[k] = act[row];
            }
#pragma unroll
            for (int k = 0; k < kVmR; k++) {
                const float av = a[k];
                const bool use = rb + k * groups < c1 && !(av > -1e-10f && av < 1e-10f);
                const float scale = use ? h2f(d[k]) * av : 0.0f;
                const uint32_t w4[4] = {q[k].x, q[k].y, q[k].z, q[k].w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t lo4 = w4[i] & 0x0F0F0F0Fu, hi4 = (w4[i] >> 4) & 0x0F0F0F0Fu;
                    // opaque to the compiler: with the masks known it extracts bytes 1-3 with a
                    // v_bfe_u32 before each conversion instead of v_cvt_f32_ubyte1..3
                    asm volatile("" : "+v"(lo4), "+v"(hi4));
                    acc[8 * i + 0] = __builtin_fmaf(ubyte0(lo4), scale, acc[8 * i + 0]);
                    acc[8 * i + 1] = __builtin_fmaf(ubyte0(hi4), scale, acc[8 * i + 1]);
                    acc[8 * i + 2] = __builtin_fmaf(ubyte1(lo4), scale, acc[8 * i + 2]);
                    acc[8 * i + 3] = __builtin_fmaf(ubyte1(hi4), scale, acc[8 * i + 3]);
                    acc[8 * i + 4] = __builtin_fmaf(ubyte2(lo4), scale, acc[8 * i + 4]);
                    acc[8 * i + 5] = __builtin_fmaf(ubyte2(hi4), scale, acc[8 * i + 5]);
                    acc[8 * i + 6] = __builtin_fmaf(ubyte3(lo4), scale, acc[8 * i + 6]);
                    acc[8 * i + 7] = __builtin_fmaf(ubyte3(hi4), scale, acc[8 * i + 7]);
                }
                ssum = ssum + scale;
            }
        }
        float* my = red + static_cast<size_t>(g) * 33 * tb + 33 * b;
#pragma unroll
        for (int i = 0; i < 32; i++) my[i] = __builtin_fmaf(-8.0f, ssum, acc[i]);
    }
    __syncthreads();
    // column c of the tile (block c / 32, element c % 32): its row groups' sums in order
    const int ncol = min(32 * tb, hidden - tile * 32 * tb);
    for (int c = t; c < ncol; c += blockDim.x) {
        const int li = 33 * (c >> 5) + (c & 31);
        float v = red[li];
        for (int r = 1; r < groups; r++) v = v + red[static_cast<size_t>(r) * 33 * tb + li];
        part[static_cast<size_t>(chunk) * hidden + static_cast<size_t>(tile) * 32 * tb + c] = v;
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

// Chunks: a multiple of 8 (one XCD per chunk), the most that keep every CU at two
// workgroups or fewer (a CU holding a third finishes last: [10240 x 2560] with 10 tiles,
// 48 chunks 8.7 us, 56 9.4, 80 10.4; 40 8.8, 32 10.7, where a thread's 10 rows take two
// load rounds), each at least one row per row group, the partials at most 1/8 of the
// weight bytes.
size_t q4_vecmat_chunks(size_t inter, size_t hidden) {
    const VmShape v = vecmat_shape(static_cast<int>(hidden / 32));
    const size_t tiles = (hidden / 32 + v.tb - 1) / v.tb;
    const size_t want = std::max<size_t>(8, static_cast<size_t>(current_device_cus()) * 2 / tiles / 8 * 8);
    const size_t cap = std::max<size_t>(1, inter * 18 / (32 * 4 * 8));  // partials <= weights / 8
    return std::max<size_t>(1, std::min({want, cap, inter / static_cast<size_t>(v.groups)}));
}

void launch_q4_vecmat(const DevWeight& w, const float* act, float* out, float* part, size_t chunks, hipStream_t s) {
    if (w.format != LARQL_Q4_0) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_vecmat: Q4_0 weights only");
    if (w.cols % 32 || w.cols == 0 || w.rows == 0) fail(LARQL_HIP_ERR_INVALID, "q4_vecmat: shape");
    if (w.rows > 0x7FFFFFFF / (w.cols / 32)) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4_vecmat: matrix too large");
    const int inter = static_cast<int>(w.rows), hidden = static_cast<int>(w.cols);
    const VmShape v = vecmat_shape(hidden / 32);
    const int rows_per_chunk = static_cast<int>((w.rows + chunks - 1) / chunks);
    const int nch = (inter + rows_per_chunk - 1) / rows_per_chunk;
    const int tiles = (hidden / 32 + v.tb - 1) / v.tb;
    const dim3 g1(static_cast<unsigned>(tiles * nch));
    const size_t lds = static_cast<size_t>(v.groups) * 33 * v.tb * sizeof(float);
    q4_vecmat_part_kernel<<<g1, dim3(v.threads), lds, s>>>(reinterpret_cast<const uint4*>(w.qs),
                                                           static_cast<const uint16_t*>(w.d), act, part, inter, hidden,
                                                           rows_per_chunk, v.tb, v.groups, tiles, nch);
    LARQL_HIP_CHECK(hipGetLastError());
    q4_vecmat_sum_kernel<<<dim3(static_cast<unsigned>((hidden + kSumCols - 1) / kSumCols)), dim3(256), 0, s>>>(
        part, out, hidden, nch);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
