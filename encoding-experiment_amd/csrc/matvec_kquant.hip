// Q6_K x f32 matvec (tiled form for tall or very long matrices) with fused RMSNorm
// prologue and decode epilogues, and the matvec dispatch for both K-quant formats
// (Q4_K goes to the matrix-core kernel of matvec_q4k_mfma.hip).
//
//   Q6_K (210-byte layout): LC/src/cpu/ops/q6k_matvec.rs:31-90, backend.rs:133-137.
//
// Mapping (gfx950, wave64): a "row slot" is `wpr` waves whose 64*wpr lanes cover K,
// one 32-element sub-block per lane per pass (SBL passes).  Every weight byte is read
// from HBM exactly once with wave-contiguous 16-byte loads; each workgroup issues the
// loads of its whole RB-row tile before any arithmetic.
//
// Arithmetic: the dot of 4-bit / 6-bit integer codes with x is done in exact int32
// with v_dot4.  Each lane turns its x sub-block once into 23-bit fixed point
// T = 65536 a + 256 b + c (three byte planes, x ~= s' T, error <= 1.2e-7 max|x|), so
//   sum(q * x) = s' * (65536 I_a + 256 I_b + I_c)
// with I_a = sdot4(q, a) and I_b, I_c = udot4(q, b|c) exact integer dots.
// The per-sub-block scale and min are applied in f32 as in the Metal kernel's
// factorisation  sc*sum(q*x) - mn*sum(x)  (LC/src/metal/shaders/q4k_matvec.rs:13-79),
// sum(x) being the f32 sum of the lane's (normalised) x.
#include "kquant_levels.h"
#include "matvec_common.h"

namespace larql {

// Shared prologue: x sub-blocks into registers (optionally RMS-normalised), then
// their int8 level images.
template <int SBL>
__device__ __forceinline__ void prologue_levels(const MvArgs& a, int cl, int C, int nsub, double* dscratch,
                                                int wave, int slot, int lane, XLevels (&L)[SBL],
                                                const bool (&valid)[SBL]) {
    float xv[SBL][32];
#pragma unroll
    for (int i = 0; i < SBL; i++) load_slice<32>(a.x, (cl + i * C) * 32, valid[i], xv[i]);
    if (a.norm_w) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < SBL; i++)
#pragma unroll
            for (int k = 0; k < 32; k++) ss += static_cast<double>(xv[i][k]) * static_cast<double>(xv[i][k]);
        const double tot = slot_sum_d(ss, dscratch, wave, slot, a.wpr, lane);
        // rms as the CPU path rounds it (LI/src/residual.rs:24); x * (1/rms) differs from
        // x / rms by at most one f32 rounding.
        const float rms = static_cast<float>(sqrt(tot / static_cast<double>(a.cols) + a.eps));
        const float inv_rms = 1.0f / rms;
#pragma unroll
        for (int i = 0; i < SBL; i++) {
            float wv[32];
            load_slice<32>(a.norm_w, (cl + i * C) * 32, valid[i], wv);
#pragma unroll
            for (int k = 0; k < 32; k++) xv[i][k] = (xv[i][k] * inv_rms) * (a.norm_offset + wv[k]);
        }
    }
#pragma unroll
    for (int i = 0; i < SBL; i++) make_levels(xv[i], L[i]);
}

template <int RB>
__device__ __forceinline__ void finish_rows(const MvArgs& a, float (&acc)[RB], float* red, int t, int lane, int wave,
                                            int nwaves, int slot, int wslot, int row0) {
    const float tot = multi_row_reduce<RB>(acc, lane);
    if (a.wpr == 1) {
        epilogue_wave<RB>(a, tot, lane, row0);
    } else {
        constexpr int rsh = rb_shift<RB>();
        const bool owner = (lane & ((1 << rsh) - 1)) == 0;
        float* buf = red + (t & 1) * nwaves * RB;
        if (owner) buf[wave * RB + (lane >> rsh)] = tot;
        __syncthreads();
        if (wslot == 0) {
            float s = 0.f;
            if (lane < RB)
                for (int w = 0; w < a.wpr; w++) s += buf[(slot * a.wpr + w) * RB + lane];
            epilogue_lanes(a, s, lane, row0, RB);
        }
    }
}

// ── Q6_K ────────────────────────────────────────────────────────────────
// Device layout per 32-element chunk: ql 16 B (reference order), qh 8 B rearranged at
// registration so that for ql dword w (elements 8w..8w+7), word qh[w/2] holds the
// 2-bit high part of element 8w + 2j + p at byte j, bits 4*(w&1) + 2p.  Then the q6
// bytes of the even / odd elements are  lo4 | (((qh >> s) & 0x03030303) << 4).
template <int SBL, int RB, bool FULL>
__global__ __launch_bounds__(512) void q6k_mv_kernel(MvArgs a) {
    extern __shared__ double dyn_lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar row addresses
    const int nwaves = blockDim.x >> 6;
    const int slot = wave / a.wpr;
    const int wslot = wave - slot * a.wpr;
    const int nslots = nwaves / a.wpr;
    const int C = a.wpr * 64;
    const int cl = wslot * 64 + lane;
    const int nsub = a.cols >> 5;
    const int S = a.cols >> 8;
    const size_t rowl = static_cast<size_t>(a.cols) >> 1;
    const size_t rowh = static_cast<size_t>(a.cols) >> 2;
    const size_t rows_s = static_cast<size_t>(a.cols) >> 4;
    double* dscratch = dyn_lds;
    float* red = reinterpret_cast<float*>(dyn_lds + nwaves);

    bool valid[SBL];
    int cc[SBL];
#pragma unroll
    for (int i = 0; i < SBL; i++) {
        valid[i] = cl + i * C < nsub;
        cc[i] = FULL ? cl + i * C : min(cl + i * C, nsub - 1);
    }
    struct Tile {
        uint4 l[RB][SBL];
        uint2 h[RB][SBL];
        uint32_t s[RB][SBL], d[RB][SBL];
    };
    Tile ta, tb;
    auto load_tile = [&](Tile& T, int tile) __attribute__((always_inline)) {
        const int row0 = (tile * nslots + slot) * RB;
#pragma unroll
        for (int r = 0; r < RB; r++)
#pragma unroll
            for (int i = 0; i < SBL; i++) {
                const size_t row = static_cast<size_t>(row0 + r);
                const uint32_t c = static_cast<uint32_t>(cc[i]);
                T.l[r][i] = *reinterpret_cast<const uint4*>(a.qs + row * rowl + c * 16u);
                T.h[r][i] = *reinterpret_cast<const uint2*>(a.qh + row * rowh + c * 8u);
                T.s[r][i] = *reinterpret_cast<const uint16_t*>(a.sc + row * rows_s + c * 2u);
                T.d[r][i] = a.d[row * S + (c >> 3)];
            }
    };
    XLevels L[SBL];
    auto compute_tile = [&](const Tile& T, int t, int tile) __attribute__((always_inline)) {
        float acc[RB];
#pragma unroll
        for (int r = 0; r < RB; r++) {
            acc[r] = 0.f;
#pragma unroll
            for (int i = 0; i < SBL; i++) {
                const uint4 l = T.l[r][i];
                const uint32_t lw[4] = {l.x, l.y, l.z, l.w};
                const uint32_t hw[2] = {T.h[r][i].x, T.h[r][i].y};
                int ga[2] = {0, 0};
                uint32_t gb[2] = {0u, 0u}, gc[2] = {0u, 0u};
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    const uint32_t H = hw[w >> 1];
                    const int sh = 4 * (w & 1);
                    const uint32_t qe = (lw[w] & 0x0F0F0F0Fu) | (((H >> sh) & 0x03030303u) << 4);
                    const uint32_t qo = ((lw[w] >> 4) & 0x0F0F0F0Fu) | (((H >> (sh + 2)) & 0x03030303u) << 4);
                    const int h2 = w >> 1;
                    ga[h2] = sdot4(qe, L[i].ev[0][w], ga[h2]);
                    ga[h2] = sdot4(qo, L[i].od[0][w], ga[h2]);
                    gb[h2] = udot4(qe, L[i].ev[1][w], gb[h2]);
                    gb[h2] = udot4(qo, L[i].od[1][w], gb[h2]);
                    gc[h2] = udot4(qe, L[i].ev[2][w], gc[h2]);
                    gc[h2] = udot4(qo, L[i].od[2][w], gc[h2]);
                }
                const float d = h2f(T.d[r][i]);
                const uint32_t s2 = T.s[r][i];
                float sc0 = d * static_cast<float>(static_cast<int8_t>(s2 & 0xFFu));
                float sc1 = d * static_cast<float>(static_cast<int8_t>(s2 >> 8));
                if (!FULL && !valid[i]) { sc0 = 0.f; sc1 = 0.f; }
                // value = sc * (q6 - 32): group sum = sc * (sum(q6 * x) - 32 * sum(x))
                acc[r] = fmaf(sc0, fmaf(-32.f, L[i].xs0, combine(ga[0], gb[0], gc[0], L[i].sp)), acc[r]);
                acc[r] = fmaf(sc1, fmaf(-32.f, L[i].xs1, combine(ga[1], gb[1], gc[1], L[i].sp)), acc[r]);
            }
        }
        finish_rows<RB>(a, acc, red, t, lane, wave, nwaves, slot, wslot, (tile * nslots + slot) * RB);
    };
    const int g = static_cast<int>(gridDim.x);
    load_tile(ta, blockIdx.x);
    prologue_levels<SBL>(a, cl, C, nsub, dscratch, wave, slot, lane, L, valid);
    for (int t = 0; t < a.steps; t += 2) {
        const int t0 = blockIdx.x + t * g, t1 = t0 + g, t2 = t1 + g;
        if (t + 1 < a.steps && t1 < a.tiles) load_tile(tb, t1);
        if (t0 < a.tiles) compute_tile(ta, t, t0);
        if (t + 1 < a.steps) {
            if (t + 2 < a.steps && t2 < a.tiles) load_tile(ta, t2);
            if (t1 < a.tiles) compute_tile(tb, t + 1, t1);
        }
    }
}

// ── launch ──────────────────────────────────────────────────────────────
template <int SBL, int RB>
static void launch_mv_t(const DevWeight& w, MvArgs a, hipStream_t s, int nslots, bool full) {
    const int threads = 64 * a.wpr * nslots;
    const size_t rows_per_tile = static_cast<size_t>(nslots) * RB;
    if (w.rows_pad % rows_per_tile) fail(LARQL_HIP_ERR_INVALID, "matvec: device rows not padded to the tile");
    const size_t tiles = w.rows_pad / rows_per_tile;
    // About two workgroups per CU; each loops over its share of the tiles.
    const size_t target = 2 * static_cast<size_t>(a.num_cus);
    a.tiles = static_cast<int>(tiles);
    a.steps = static_cast<int>((tiles + target - 1) / target);
    const size_t grid = (tiles + a.steps - 1) / a.steps;
    const int nwaves = threads / 64;
    const size_t shmem = nwaves * sizeof(double) + 2 * nwaves * RB * sizeof(float);
    const dim3 g(static_cast<unsigned>(grid)), b(threads);
    {
        a.qs = w.qs;
        a.qh = w.qh;
        a.sc = w.sc;
        a.d = static_cast<const uint16_t*>(w.d);
        if (full) q6k_mv_kernel<SBL, RB, true><<<g, b, shmem, s>>>(a);
        else q6k_mv_kernel<SBL, RB, false><<<g, b, shmem, s>>>(a);
    }
    LARQL_HIP_CHECK(hipGetLastError());
}

void launch_mv(const DevWeight& w, MvArgs a, hipStream_t s) {
    if (w.format == LARQL_Q4_K || w.format == LARQL_Q4_KF) return launch_q4k_mfma(w, a, s);
    if (w.format != LARQL_Q6_K) fail(LARQL_HIP_ERR_UNSUPPORTED, "launch_mv: format");
    if (a.num_cus <= 0) a.num_cus = current_device_cus();
    if (stream_mv_supported(w)) return launch_mv_stream(w, a, s);
    a.rows = static_cast<int>(w.rows);
    a.cols = static_cast<int>(w.cols);
    if (a.epi == EPI_GATED_PAIR && (w.rows & 1)) fail(LARQL_HIP_ERR_INVALID, "gated pair epilogue needs even rows");
    const size_t nsub = w.cols / 32;
    const size_t waves1 = (nsub + 63) / 64;
    if (waves1 <= 8) {
        // one sub-block per lane; >= 256 threads per workgroup where possible
        a.wpr = static_cast<int>(waves1);
        int nslots = 1;
        while (a.wpr * nslots * 2 <= 4) nslots *= 2;
        launch_mv_t<1, 8>(w, a, s, nslots, static_cast<size_t>(64) * a.wpr == nsub);
    } else {
        a.wpr = static_cast<int>((nsub + 127) / 128);
        if (a.wpr > 8) fail(LARQL_HIP_ERR_UNSUPPORTED, "matvec: hidden too large (max 32768)");
        launch_mv_t<2, 4>(w, a, s, 1, static_cast<size_t>(128) * a.wpr == nsub);
    }
}

void launch_q4k_matvec(const DevWeight& w, const float* x, float* out, size_t m, void* ws, hipStream_t s) {
    if (m > 1) {  // prefill: m tokens on the matrix cores (148-byte Q4_K)
        if (w.format != LARQL_Q4_K) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4k matmul: Q4_K weights only");
        return launch_q4k_gemm(w, x, out, m, ws, s);
    }
    MvArgs a;
    a.x = x;
    a.out = out;
    launch_mv(w, a, s);
}

void launch_q6k_matvec(const DevWeight& w, const float* x, float* out, size_t m, hipStream_t s) {
    if (m != 1) fail(LARQL_HIP_ERR_UNSUPPORTED, "q6k_matvec: batch > 1 not supported");
    MvArgs a;
    a.x = x;
    a.out = out;
    launch_mv(w, a, s);
}

}  // namespace larql
