// Q6_K x f32 matvec (210-byte Q6_K; reference semantics LC/src/cpu/ops/q6k_matvec.rs:31-90,
// trait method LC/src/backend.rs:133-137).  Element e of a super-block:
//   lo4 = nibble e of ql (byte e/2, low for even e), hi2 = qh bits at byte e/4, shift 2*(e%4),
//   value = d * sc[e/16] * ((lo4 + 16*hi2) - 32).
// Mapping as in the Q4_K kernel: one 32-element chunk (two scale groups) per lane, x in
// registers, wave-contiguous loads of the ql (16 B), qh (8 B) and scale (2 B) arrays.
#include "device_common.h"
#include "larql_hip_internal.h"

namespace larql {

template <int RB>
__device__ __forceinline__ float q6_multi_row_reduce(float (&v)[RB], int lane) {
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

template <int SBL, int RB>
__global__ __launch_bounds__(512) void q6k_matvec_kernel(const uint8_t* __restrict__ ql,
                                                         const uint8_t* __restrict__ qh,
                                                         const int8_t* __restrict__ scl,
                                                         const uint16_t* __restrict__ dd,
                                                         const float* __restrict__ x,
                                                         float* __restrict__ out, int rows, int cols,
                                                         int wpr, int steps) {
    extern __shared__ float red[];
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
    const size_t rowl = static_cast<size_t>(cols) >> 1;
    const size_t rowh = static_cast<size_t>(cols) >> 2;
    const size_t rows_s = static_cast<size_t>(cols) >> 4;

    float xv[SBL][32], xs0[SBL], xs1[SBL];
    bool valid[SBL];
#pragma unroll
    for (int i = 0; i < SBL; i++) {
        const int c = cl + i * C;
        valid[i] = c < nsub;
        const float4* xp = reinterpret_cast<const float4*>(x + static_cast<size_t>(c) * 32);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            float4 v = valid[i] ? xp[k] : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[i][4 * k + 0] = v.x;
            xv[i][4 * k + 1] = v.y;
            xv[i][4 * k + 2] = v.z;
            xv[i][4 * k + 3] = v.w;
            if (k < 4) { s0 += v.x; s0 += v.y; s0 += v.z; s0 += v.w; }
            else { s1 += v.x; s1 += v.y; s1 += v.z; s1 += v.w; }
        }
        xs0[i] = s0;
        xs1[i] = s1;
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
                        const uint4 l = *reinterpret_cast<const uint4*>(ql + row * rowl + c * 16);
                        const uint2 h = *reinterpret_cast<const uint2*>(qh + row * rowh + c * 8);
                        const uint32_t s2 = *reinterpret_cast<const uint16_t*>(scl + row * rows_s + c * 2);
                        const float d = h2f(dd[static_cast<size_t>(row) * S + (c >> 3)]);
                        const uint32_t lw[4] = {l.x, l.y, l.z, l.w};
                        float g0 = 0.f, g1 = 0.f;
#pragma unroll
                        for (int w = 0; w < 4; w++) {
                            const uint32_t H = ((w < 2 ? h.x : h.y) >> (16 * (w & 1))) & 0xFFFFu;
                            float gd = 0.f;
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                const uint32_t le = (lw[w] >> (8 * j)) & 0xFu;
                                const uint32_t lo = (lw[w] >> (8 * j + 4)) & 0xFu;
                                const uint32_t he = (H >> (4 * j)) & 0x3u;
                                const uint32_t ho = (H >> (4 * j + 2)) & 0x3u;
                                gd = fmaf(static_cast<float>(le | (he << 4)), xv[i][8 * w + 2 * j], gd);
                                gd = fmaf(static_cast<float>(lo | (ho << 4)), xv[i][8 * w + 2 * j + 1], gd);
                            }
                            if (w < 2) g0 += gd; else g1 += gd;
                        }
                        const float sc0 = d * static_cast<float>(static_cast<int8_t>(s2 & 0xFFu));
                        const float sc1 = d * static_cast<float>(static_cast<int8_t>(s2 >> 8));
                        acc[r] = fmaf(sc0, fmaf(-32.f, xs0[i], g0), acc[r]);
                        acc[r] = fmaf(sc1, fmaf(-32.f, xs1[i], g1), acc[r]);
                    }
                }
            }
        }
        const float tot = q6_multi_row_reduce<RB>(acc, lane);
        constexpr int rsh = RB == 1 ? 6 : RB == 2 ? 5 : RB == 4 ? 4 : 3;
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

void launch_q6k_matvec(const DevWeight& w, const float* x, float* out, size_t m, hipStream_t s) {
    if (m != 1) fail(LARQL_HIP_ERR_UNSUPPORTED, "q6k_matvec: batch > 1 not supported");
    constexpr int RB = 4;
    const size_t nsub = w.cols / 32;
    int wpr, nslots = 1, sbl;
    size_t waves1 = (nsub + 63) / 64;
    if (waves1 <= 8) {
        wpr = static_cast<int>(waves1);
        sbl = 1;
        while (wpr * nslots * 2 <= 4) nslots *= 2;
    } else {
        wpr = static_cast<int>((nsub + 127) / 128);
        sbl = 2;
        if (wpr > 8) fail(LARQL_HIP_ERR_UNSUPPORTED, "q6k_matvec: hidden too large");
    }
    const int threads = 64 * wpr * nslots;
    const size_t rows_per_step = static_cast<size_t>(nslots) * RB;
    const size_t total_steps = (w.rows + rows_per_step - 1) / rows_per_step;
    const size_t target = 1024;
    const int steps = static_cast<int>((total_steps + target - 1) / target);
    const size_t grid = (total_steps + steps - 1) / steps;
    const size_t shmem = 2 * (threads / 64) * RB * sizeof(float);
    const uint16_t* dd = static_cast<const uint16_t*>(w.d);
    if (sbl == 1)
        q6k_matvec_kernel<1, RB><<<dim3(grid), dim3(threads), shmem, s>>>(
            w.qs, w.qh, w.sc, dd, x, out, static_cast<int>(w.rows), static_cast<int>(w.cols), wpr, steps);
    else
        q6k_matvec_kernel<2, RB><<<dim3(grid), dim3(threads), shmem, s>>>(
            w.qs, w.qh, w.sc, dd, x, out, static_cast<int>(w.rows), static_cast<int>(w.cols), wpr, steps);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
