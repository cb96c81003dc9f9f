// Q4_K x f32 matvec: out[n] = sum_k deq(W[n,k]) * x[k]   (148-byte Q4_K, reference
// semantics LC/src/cpu/ops/q4k_matvec.rs:31-90; trait method LC/src/backend.rs:126-130).
//
// Mapping (gfx950, wave64): a "row slot" is `wpr` waves whose 64*wpr lanes cover the
// K dimension, one 32-element sub-block (16 nibble bytes) per lane per pass.  Each
// lane keeps its x sub-blocks in registers for the whole launch, so x is read from
// L2 once per workgroup and every nibble byte is read from HBM exactly once, with
// wave-contiguous 16-byte loads (64 lanes x 16 B = 1 KB per instruction).
// Per sub-block the lane computes  sc*sum(q*x) - mn*sum(x)  (the Metal kernel's
// factorisation, LC/src/metal/shaders/q4k_matvec.rs:13-79), sum(x) being fixed per lane.
// Row partials are combined with a transposed butterfly (log2(RB) halving steps then
// a plain butterfly), then across the wpr waves of the slot through LDS.
#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

// Reduce RB per-lane partials over the 64 lanes of a wave.  On return lane
// (r << (6 - log2(RB))) holds the total of row r.
template <int RB>
__device__ __forceinline__ float multi_row_reduce(float (&v)[RB], int lane) {
    int n = RB;
    int mask = 32;
#pragma unroll
    for (int step = 0; step < 6; step++) {
        if (n > 1) {
            const bool upper = (lane & mask) != 0;
            const int half = n >> 1;
#pragma unroll
            for (int i = 0; i < RB / 2; i++) {
                if (i < half) {
                    float keep = upper ? v[i + half] : v[i];
                    float send = upper ? v[i] : v[i + half];
                    v[i] = keep + __shfl_xor(send, mask, 64);
                }
            }
            n = half;
        } else {
            v[0] += __shfl_xor(v[0], mask, 64);
        }
        mask >>= 1;
    }
    return v[0];
}

template <int RB>
__device__ __forceinline__ constexpr int log2_rb() { return RB == 1 ? 0 : RB == 2 ? 1 : RB == 4 ? 2 : 3; }

template <int SBL, int RB>
__global__ __launch_bounds__(512) void q4k_matvec_kernel(const uint8_t* __restrict__ qs,
                                                         const uint4* __restrict__ hdr,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ out, int rows, int cols,
                                                         int wpr, int steps) {
    extern __shared__ float red[];  // [2][waves][RB]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    const int slot = wave / wpr;
    const int wslot = wave - slot * wpr;
    const int nslots = nwaves / wpr;
    const int C = wpr * 64;
    const int cl = wslot * 64 + lane;
    const int nsub = cols >> 5;
    const int S = cols >> 8;
    const size_t rowq = static_cast<size_t>(cols) >> 1;

    float xe[SBL][16], xo[SBL][16], xs[SBL];
    int scw[SBL], scsh[SBL], msh[SBL];
    bool valid[SBL];
#pragma unroll
    for (int i = 0; i < SBL; i++) {
        const int c = cl + i * C;
        valid[i] = c < nsub;
        float s = 0.f;
        const float4* xp = reinterpret_cast<const float4*>(x + static_cast<size_t>(c) * 32);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            float4 v = valid[i] ? xp[k] : make_float4(0.f, 0.f, 0.f, 0.f);
            xe[i][2 * k] = v.x;
            xo[i][2 * k] = v.y * 0.0625f;
            xe[i][2 * k + 1] = v.z;
            xo[i][2 * k + 1] = v.w * 0.0625f;
            s += v.x;
            s += v.y;
            s += v.z;
            s += v.w;
        }
        xs[i] = s;
        const int j = c & 7;
        scw[i] = j < 4 ? 1 : 2;
        scsh[i] = 8 * (j & 3);
        msh[i] = 8 * (j & 3) + (j < 4 ? 0 : 4);
    }

    for (int t = 0; t < steps; t++) {
        const int row0 = ((blockIdx.x * steps + t) * nslots + slot) * RB;
        float acc[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) {
            acc[r] = 0.f;
            const int row = row0 + r;
            if (row < rows) {
#pragma unroll
                for (int i = 0; i < SBL; i++) {
                    if (valid[i]) {
                        const int c = cl + i * C;
                        const uint4 q = *reinterpret_cast<const uint4*>(qs + row * rowq + c * 16);
                        const uint4 h = hdr[static_cast<size_t>(row) * S + (c >> 3)];
                        const float d = h2f(h.x);
                        const float dmin = h2f(h.x >> 16);
                        const uint32_t sw = scw[i] == 1 ? h.y : h.z;
                        const float sc = d * static_cast<float>((sw >> scsh[i]) & 0x3Fu);
                        const float mn = dmin * static_cast<float>((h.w >> msh[i]) & 0xFu);
                        float dl = 0.f, dh = 0.f;
                        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                        for (int w = 0; w < 4; w++) {
                            const uint32_t lo = qw[w] & 0x0F0F0F0Fu;
                            const uint32_t hi = qw[w] & 0xF0F0F0F0u;  // 16*hi per byte; x odd pre-scaled by 1/16
                            dl = fmaf(ubyte0(lo), xe[i][4 * w + 0], dl);
                            dh = fmaf(ubyte0(hi), xo[i][4 * w + 0], dh);
                            dl = fmaf(ubyte1(lo), xe[i][4 * w + 1], dl);
                            dh = fmaf(ubyte1(hi), xo[i][4 * w + 1], dh);
                            dl = fmaf(ubyte2(lo), xe[i][4 * w + 2], dl);
                            dh = fmaf(ubyte2(hi), xo[i][4 * w + 2], dh);
                            dl = fmaf(ubyte3(lo), xe[i][4 * w + 3], dl);
                            dh = fmaf(ubyte3(hi), xo[i][4 * w + 3], dh);
                        }
                        acc[r] = fmaf(sc, dl + dh, fmaf(-mn, xs[i], acc[r]));
                    }
                }
            }
        }
        const float tot = multi_row_reduce<RB>(acc, lane);
        const int rsh = 6 - log2_rb<RB>();
        const bool owner = (lane & ((1 << rsh) - 1)) == 0;
        const int r = lane >> rsh;
        if (wpr == 1) {
            if (owner && row0 + r < rows) out[row0 + r] = tot;
        } else {
            float* buf = red + (t & 1) * nwaves * RB;
            if (owner) buf[wave * RB + r] = tot;
            __syncthreads();
            if (wslot == 0 && lane < RB && row0 + lane < rows) {
                float s = 0.f;
                for (int w = 0; w < wpr; w++) s += buf[(slot * wpr + w) * RB + lane];
                out[row0 + lane] = s;
            }
        }
    }
}

struct MvCfg {
    int wpr, nslots, sbl;
};

static MvCfg q4k_cfg(size_t cols) {
    const size_t nsub = cols / 32;
    // Lanes per row slot must cover K with 1 or 2 sub-blocks per lane.
    size_t waves1 = (nsub + 63) / 64;
    if (waves1 <= 8) {
        MvCfg c{static_cast<int>(waves1), 1, 1};
        while (c.wpr * c.nslots * 2 <= 4) c.nslots *= 2;  // keep >= 256 threads where possible
        return c;
    }
    size_t waves2 = (nsub + 127) / 128;
    return MvCfg{static_cast<int>(waves2), 1, 2};
}

void launch_q4k_matvec(const DevWeight& w, const float* x, float* out, size_t m, hipStream_t s) {
    if (m != 1) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4k_matvec: batch > 1 not supported");
    constexpr int RB = 4;
    const MvCfg c = q4k_cfg(w.cols);
    if (c.wpr > 8) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4k_matvec: hidden too large");
    const int threads = 64 * c.wpr * c.nslots;
    const size_t rows_per_step = static_cast<size_t>(c.nslots) * RB;
    const size_t total_steps = (w.rows + rows_per_step - 1) / rows_per_step;
    const size_t target = 1024;
    const int steps = static_cast<int>((total_steps + target - 1) / target);
    const size_t grid = (total_steps + steps - 1) / steps;
    const size_t shmem = 2 * (threads / 64) * RB * sizeof(float);
    if (c.sbl == 1)
        q4k_matvec_kernel<1, RB><<<dim3(grid), dim3(threads), shmem, s>>>(
            w.qs, w.hdr, x, out, static_cast<int>(w.rows), static_cast<int>(w.cols), c.wpr, steps);
    else
        q4k_matvec_kernel<2, RB><<<dim3(grid), dim3(threads), shmem, s>>>(
            w.qs, w.hdr, x, out, static_cast<int>(w.rows), static_cast<int>(w.cols), c.wpr, steps);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
