// Q4_K x f32 matvec with the integer block dots on the matrix cores.
//
//   Reference semantics: LC/src/cpu/ops/q4k_matvec.rs:31-90 (trait method
//   LC/src/backend.rs:126-130): out[n] = sum_sb sum_j sum_i (d*sc_j*q - dmin*m_j) * x,
//   computed here in the factorised form sc * sum(q x) - mn * sum(x) per 32-element
//   sub-block (LC/src/metal/shaders/q4k_matvec.rs:13-79).  The two Q4_KF byte layouts
//   (144-byte GGUF and 160-byte pre-baked, LC/src/pipeline.rs:15) arrive in the same
//   device nibble layout and differ only in how a header gives the scales and mins.
//
// Work split.  A workgroup owns T tiles of 16 consecutive weight rows; its KS waves
// split the super-blocks of the rows into contiguous parts of P = UR * R super-blocks
// (wave w takes [wP, wP + P) of every tile), walked in R rounds of UR.  A round's loads
// are its x slice, then UR units per tile of two 1 KB nibble loads and one 256 B header
// load: with R = 1 every weight byte is requested within the first microsecond or two of
// the launch and the arithmetic of every wave overlaps the streaming of all the others.
// The weights are stored tile-major (layouts.hip), so each of those loads reads
// contiguous memory, and they are non-temporal (each byte is used once).
//
// Per unit (one super-block of the 16 rows), lane (g, c) = lane 16 g + c holds
// sub-blocks g and g + 4 of row c.  Four v_mfma_i32_16x16x64_i8 take the nibbles
// (unpacked to bytes) as B, column c = row c, and the activation as A, with A row
// 4 s + p = digit plane p of the x sub-block held by k-group s (zero in the other
// k-groups).  Result lane 16 g + c, register p, is then exactly the int32 dot of plane p
// of x with sub-block g (first accumulator) or g + 4 (second) of row c: no cross-lane
// traffic until the end of the row.
//
// x digit planes: per 32-element sub-block, T = rint(x * (2^22 - 1) / max|x|) is split
// into balanced signed bytes T = 65536 a + 256 b + c (a, b, c in [-128, 127]) taken from
// the bytes of T + 0x808080 with their top bits flipped.  |x - s' T| <= s'/2 with
// s' = max|x| / (2^22 - 1): the size of one f32 rounding of the sub-block's largest
// element.  Each wave builds the planes of its own part in its own LDS area (no
// workgroup barrier before the loop); a fused RMSNorm adds one barrier for sum(x^2).
#include <type_traits>

#include "kquant_levels.h"
#include "matvec_common.h"
#include "mfma_planes.h"


namespace larql {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// Within a unit, sub-block j's planes (mfma_planes.h) sit in slot 2 (j % 4) + j / 4, so
// the two sub-blocks of a lane (g and g + 4) are adjacent; the slot's float4 is
// {s', 65536 s', sum x, 0}.
constexpr int kZeroBytes = 256;  // per-wave zero area read by the idle A lanes (offsets < 176)
constexpr int kMaxKS = 16;

template <int UR>
__host__ __device__ constexpr int wave_lds_bytes() {
    return kZeroBytes + 8 * UR * static_cast<int>(sizeof(PlSlot));
}

// Nibble dword (element 2i in the low, 2i + 1 in the high nibble of byte i) -> bytes of
// its even / odd elements.
__device__ __forceinline__ int lo_nib(uint32_t w) { return static_cast<int>(w & 0x0F0F0F0Fu); }
__device__ __forceinline__ int hi_nib(uint32_t w) { return static_cast<int>((w >> 4) & 0x0F0F0F0Fu); }

// UR: super-blocks per round (2 or 4); T: 16-row tiles per workgroup (rows
// 16 T blockIdx.x ...), all sharing the wave's x planes; a.steps = R rounds;
// KS = blockDim.x / 64 waves.
template <int UR, int T>
constexpr int max_waves() {
    return UR * T >= 8 ? kMaxKS / 2 : kMaxKS;  // 8 units in flight need more than 128 VGPRs
}

// Scales and mins of sub-blocks g and g + 4 of one row from its header (HF: the header
// form, kHdr148 / kHdrGguf / kHdrKf160; h2 is the second uint4 of a kHdrKf160 pair).
template <int HF>
__device__ __forceinline__ void q4k_scale_min(const uint4& h, const uint4& h2, int g, float& sc0, float& sc1,
                                              float& mn0, float& mn1) {
    const int scsh = 8 * g;
    if constexpr (HF == kHdrKf160) {
        const uint32_t s0 = (g < 2 ? h.x : h.y) >> (16 * (g & 1)), s1 = (g < 2 ? h.z : h.w) >> (16 * (g & 1));
        const uint32_t m0 = (g < 2 ? h2.x : h2.y) >> (16 * (g & 1)), m1 = (g < 2 ? h2.z : h2.w) >> (16 * (g & 1));
        sc0 = h2f(s0);
        sc1 = h2f(s1);
        mn0 = h2f(m0);
        mn1 = h2f(m1);
    } else {
        const float d = h2f(h.x), dmin = h2f(h.x >> 16);
        sc0 = d * static_cast<float>((h.y >> scsh) & 0x3Fu);
        sc1 = d * static_cast<float>((h.z >> scsh) & 0x3Fu);
        uint32_t q0 = (h.w >> scsh) & 0xFu, q1 = (h.w >> (scsh + 4)) & 0xFu;
        if constexpr (HF == kHdrGguf) {  // 6-bit mins: bits 4..5 above the 6-bit scales
            q0 |= ((h.y >> (scsh + 6)) & 3u) << 4;
            q1 |= ((h.z >> (scsh + 6)) & 3u) << 4;
        }
        mn0 = dmin * static_cast<float>(q0);
        mn1 = dmin * static_cast<float>(q1);
    }
}

// PRE: units whose loads are issued with x, before the planes are built (the rest after);
// XB: every wave's x loads are issued before any wave of the workgroup issues a weight
// load (a bare s_barrier between them), so x is not queued behind the workgroup's weights.
template <int UR, int T, bool NORM, int HF, int PRE, bool XB>
__global__ __launch_bounds__((64 * max_waves<UR, T>())) void q4k_mfma_kernel(MvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int EL = 4 * UR;  // x elements per lane and round
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KS = blockDim.x >> 6;
    const int R = a.steps;
    const int S = a.cols >> 8;
    const int sb0 = wave * UR * R;                  // first super-block of this wave
    const int nsb = max(0, min(UR * R, S - sb0));   // super-blocks of this wave
    const int g = lane >> 4, c = lane & 15;
    const size_t tile0 = static_cast<size_t>(blockIdx.x) * T;  // < rows_pad / 16: the grid is rows_pad / (16 T)
    const uint8_t* tq = a.qs + tile0 * S * 2048 + lane * 16;
    constexpr int HW = HF == kHdrKf160 ? 2 : 1;  // uint4 header words per row and super-block
    const uint4* th = a.hdr + (tile0 * S * 16 + c) * HW;

    uint8_t* wl = lds + wave * wave_lds_bytes<UR>();
    PlSlot* slots = reinterpret_cast<PlSlot*>(wl + kZeroBytes);
    float* red = reinterpret_cast<float*>(lds + KS * wave_lds_bytes<UR>());  // [KS][16 T], then NORM scratch

    float xv[EL], wv[NORM ? EL : 1];
    uint4 n0[T][UR], n1[T][UR], hd[T][UR], hd2[HF == kHdrKf160 ? T : 1][HF == kHdrKf160 ? UR : 1];
    // Loads of round r: this lane's x slice (element e0), then the units' weights
    // (super-block indices clamped: a short last round re-reads a real block).  The
    // first PRE units are issued with x; the rest after the planes are built, so that a
    // wave held up issuing loads into a full memory system has its planes ready when
    // its data arrives.
    auto load_x = [&](int r) __attribute__((always_inline)) {
        const int e0 = (sb0 + r * UR) * 256 + lane * EL;
        load_slice<EL>(a.x, min(e0, a.cols - EL), true, xv);
        if constexpr (NORM) load_slice<EL>(a.norm_w, min(e0, a.cols - EL), true, wv);
    };
    // units are numbered t * UR + u (tile t, super-block u of the round)
    auto load_units = [&](int r, int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int u = 0; u < UR; u++) {
                if (t * UR + u < i0 || t * UR + u >= i1) continue;
                const size_t sb = static_cast<size_t>(t) * S + min(sb0 + r * UR + u, S - 1);
                const uint8_t* q = tq + sb * 2048;
                n0[t][u] = load_nt(q);
                n1[t][u] = load_nt(q + 1024);
                hd[t][u] = load_nt(th + sb * 16 * HW);
                if constexpr (HF == kHdrKf160) hd2[t][u] = load_nt(th + sb * 32 + 1);
            }
    };
    load_x(0);
    if constexpr (XB) __builtin_amdgcn_s_barrier();
    load_units(0, 0, PRE);
    // Loaded now, used at the end (so the epilogue waits on no memory): the producer's
    // partial sums of squares of a prenormed x, and wave 0's residual and out2 weight rows.
    double ps0 = 0.0, ps1 = 0.0;
    float rv_pre = 0.f, w2_pre = 0.f;
    if constexpr (!NORM) {
        if (a.x_psum) {
            const int i0 = static_cast<int>(threadIdx.x), i1 = i0 + static_cast<int>(blockDim.x);
            if (i0 < a.x_npsum) ps0 = a.x_psum[i0];
            if (i1 < a.x_npsum) ps1 = a.x_psum[i1];
        }
        const int row = static_cast<int>(tile0 * 16) + lane;
        if (wave == 0 && lane < 16 * T && row < a.rows) {
            if (a.epi == EPI_RESID || a.epi == EPI_GATED_MUL) rv_pre = a.resid[row];
            if (a.out2) w2_pre = a.out2_w[row];
        }
    }

    // Fused RMSNorm (LI/src/residual.rs:17-33): sum(x^2) over all of x, in f64.
    float inv_rms = 1.f;
    if constexpr (NORM) {
        double part[2] = {0.0, 0.0};
        for (int r = 0; r < R; r++) {
            float xs[EL];
            const int e0 = (sb0 + r * UR) * 256 + lane * EL;
            if (r == 0) {
#pragma unroll
                for (int k = 0; k < EL; k++) xs[k] = xv[k];
            } else {
                load_slice<EL>(a.x, min(e0, a.cols - EL), true, xs);
            }
            if (e0 < sb0 * 256 + nsb * 256) {
#pragma unroll
                for (int k = 0; k < EL; k++)
                    part[k & 1] = fma(static_cast<double>(xs[k]), static_cast<double>(xs[k]), part[k & 1]);
            }
        }
        const double v = wave_sum_d(part[0] + part[1]);
        double* dscr = reinterpret_cast<double*>(red + KS * 16);
        if (lane == 0) dscr[wave] = v;
        __syncthreads();
        double tot = 0.0;
        for (int w = 0; w < KS; w++) tot += dscr[w];
        // rms as the CPU path rounds it (LI/src/residual.rs:24); x * (1/rms) differs from
        // x / rms by at most one f32 rounding.
        const float rms = static_cast<float>(sqrt(tot / static_cast<double>(a.cols) + a.eps));
        inv_rms = 1.0f / rms;
    }

    // A lane (g, i): A row i = 4 s + p is live in k-group g iff s == g and p < 3; the
    // others read the zero area (same immediate offsets, all inside it).
    const int ia = lane & 15;
    const bool alive = (ia >> 2) == g && (ia & 3) < 3;
    const uint32_t abase = alive ? static_cast<uint32_t>(kZeroBytes + 2 * g * sizeof(PlSlot) + (ia & 3) * 16) : 0u;
    const uint32_t astep = alive ? 8u * sizeof(PlSlot) : 0u;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.f;

    for (int r = 0; r < R; r++) {
        const int nr = min(UR, nsb - r * UR);  // units of this round (wave-uniform)
        if (nr <= 0) break;
        if (r > 0) {
            load_x(r);
            load_units(r, 0, PRE);
        }
        // Digit planes of this lane's EL elements (one sub-block of 32 spans 32 / EL lanes).
        {
            if constexpr (NORM) {
#pragma unroll
                for (int k = 0; k < EL; k++) xv[k] = (xv[k] * inv_rms) * (a.norm_offset + wv[k]);
            }
            float m = tree_max_abs<EL>(xv);
            float s = tree_sum<EL>(xv);
            m = fmaxf(m, dpp_f<DPP_QUAD_1032>(m));
            s = s + dpp_f<DPP_QUAD_1032>(s);
            if constexpr (UR == 2) {
                m = fmaxf(m, dpp_f<DPP_QUAD_2301>(m));
                s = s + dpp_f<DPP_QUAD_2301>(s);
            }
            const float inv = m > 0.f ? kLevelScale / m : 0.f;
            uint32_t u[EL];
#pragma unroll
            for (int k = 0; k < EL; k++)
                u[k] = __float_as_uint(fmaf(xv[k], inv, 12582912.0f)) + (0x808080u - 0x4B400000u);
            const int sub = (lane * EL) >> 5;  // sub-block within the round: unit sub / 8, j = sub % 8
            const int ofs = (lane * EL) & 31;  // first element of the lane within it
            if (sub < 8 * nr) {
                const int j = sub & 7;
                PlSlot& sl = slots[(sub & ~7) + 2 * (j & 3) + (j >> 2)];
                const int hm = ofs >> 4;
                const int dw0 = (ofs & 15) >> 2;  // first dword of the half this lane fills (0 or 2)
#pragma unroll
                for (int q8 = 0; q8 < EL / 8; q8++) {
                    uint32_t pe[3], po[3];
                    pack_planes(u[8 * q8 + 0], u[8 * q8 + 2], u[8 * q8 + 4], u[8 * q8 + 6], pe);
                    pack_planes(u[8 * q8 + 1], u[8 * q8 + 3], u[8 * q8 + 5], u[8 * q8 + 7], po);
#pragma unroll
                    for (int p = 0; p < 3; p++) {
                        uint32_t* d = reinterpret_cast<uint32_t*>(&sl.pl[hm][p]) + dw0 + 2 * q8;
                        *reinterpret_cast<uint2*>(d) = make_uint2(pe[p], po[p]);
                    }
                }
                if (ofs == 0) sl.s = make_float4(m / kLevelScale, m * (65536.0f / kLevelScale), s, 0.f);
            }
            if (r == 0 && lane < kZeroBytes / 16) reinterpret_cast<uint4*>(wl)[lane] = make_uint4(0, 0, 0, 0);
        }
        load_units(r, PRE, T * UR);
        // the wave reads what its own lanes wrote: keep the LDS accesses in program order
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
        for (int u = 0; u < UR; u++) {
            if (u < nr) {
                const uint8_t* ab = wl + abase + u * astep;
                const uint4 a0 = *reinterpret_cast<const uint4*>(ab);
                const uint4 a1 = *reinterpret_cast<const uint4*>(ab + 48);
                const uint4 a2 = *reinterpret_cast<const uint4*>(ab + sizeof(PlSlot));
                const uint4 a3 = *reinterpret_cast<const uint4*>(ab + sizeof(PlSlot) + 48);
                const v4i A0 = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w};
                const v4i A1 = {(int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                const v4i A2 = {(int)a2.x, (int)a2.y, (int)a2.z, (int)a2.w};
                const v4i A3 = {(int)a3.x, (int)a3.y, (int)a3.z, (int)a3.w};
                const v4i B0 = {lo_nib(n0[t][u].x), hi_nib(n0[t][u].x), lo_nib(n0[t][u].y), hi_nib(n0[t][u].y)};
                const v4i B1 = {lo_nib(n0[t][u].z), hi_nib(n0[t][u].z), lo_nib(n0[t][u].w), hi_nib(n0[t][u].w)};
                const v4i B2 = {lo_nib(n1[t][u].x), hi_nib(n1[t][u].x), lo_nib(n1[t][u].y), hi_nib(n1[t][u].y)};
                const v4i B3 = {lo_nib(n1[t][u].z), hi_nib(n1[t][u].z), lo_nib(n1[t][u].w), hi_nib(n1[t][u].w)};
                v4i Da = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, v4i{0, 0, 0, 0}, 0, 0, 0);
                v4i Db = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, B2, v4i{0, 0, 0, 0}, 0, 0, 0);
                Da = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, Da, 0, 0, 0);
                Db = __builtin_amdgcn_mfma_i32_16x16x64_i8(A3, B3, Db, 0, 0, 0);
                // scales of sub-blocks g and g + 4 of row c
                const PlSlot* sl = slots + 8 * u + 2 * g;
                const float4 sa = sl[0].s, sb = sl[1].s;
                float sc0, sc1, mn0, mn1;
                if constexpr (HF == kHdrKf160) q4k_scale_min<HF>(hd[t][u], hd2[t][u], g, sc0, sc1, mn0, mn1);
                else q4k_scale_min<HF>(hd[t][u], hd[t][u], g, sc0, sc1, mn0, mn1);
                // s' (65536 a + 256 b + c): 256 b + c is exact in int32 and in f32 (< 2^24)
                const float dot0 = fmaf(static_cast<float>(Da[2]), sa.y, sa.x * static_cast<float>(Da[1] * 256 + Da[0]));
                const float dot1 = fmaf(static_cast<float>(Db[2]), sb.y, sb.x * static_cast<float>(Db[1] * 256 + Db[0]));
                acc[t] = fmaf(sc0, dot0, fmaf(-mn0, sa.z, acc[t]));
                acc[t] = fmaf(sc1, dot1, fmaf(-mn1, sb.z, acc[t]));
            }
        }
        if (r + 1 < R) {
            // the next round rewrites the planes this round's MFMA operands came from
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }

    // Row totals: over the four k-groups of the wave, then over the waves in order.
#pragma unroll
    for (int t = 0; t < T; t++) {
        float v = swap32_add(acc[t], acc[t]);
        v = swap16_add(v, v);
        if (lane < 16) red[(wave * T + t) * 16 + lane] = v;
    }
    double* xsq = reinterpret_cast<double*>(red + KS * 16 * T);  // prenormed input: per-wave sums
    if (!NORM && a.x_psum) {
        const double v = wave_sum_d(ps0 + ps1);
        if (lane == 0) xsq[wave] = v;
    }
    __syncthreads();
    if (wave == 0) {
        const int row = static_cast<int>(tile0 * 16) + lane;
        float tot = 0.f;
        if (lane < 16 * T) {
            tot = red[lane];
            for (int w = 1; w < KS; w++) tot += red[w * 16 * T + lane];
        }
        if (!NORM && a.x_psum) {
            double sq = 0.0;
            for (int w = 0; w < KS; w++) sq += xsq[w];
            // rms as the CPU path rounds it (LI/src/residual.rs:24)
            const float rms = static_cast<float>(sqrt(sq / static_cast<double>(a.cols) + a.eps));
            tot *= 1.0f / rms;
        }
        if (a.epi == EPI_GATED_PAIR) {
            const float up = __shfl_down(tot, 1, 64);  // rows 2i, 2i + 1 sit in adjacent lanes of one tile
            if (lane < 16 * T && (lane & 1) == 0 && row < a.rows) a.out[row >> 1] = gated_act(a.act, tot, up);
        } else {
            const bool live = lane < 16 * T && row < a.rows;
            const float rv = a.epi == EPI_STORE ? 0.f : (NORM ? (live ? a.resid[row] : 0.f) : rv_pre);
            const float v = live ? epi_value(a, rv, tot) : 0.f;
            if (live) a.out[row] = v;
            if (!NORM && a.out2 && live) a.out2[row] = v * (a.out2_off + w2_pre);
            if (!NORM && a.psum) {
                const double q = wave_sum_d(static_cast<double>(v) * static_cast<double>(v));
                if (lane == 0) a.psum[blockIdx.x] = q;
            }
        }
    }
}



template <int UR, int T, int HF, int PRE, bool XB>
void launch_q4k_mfma_t(const DevWeight& w, MvArgs a, int R, hipStream_t s) {
    const int S = static_cast<int>(w.cols / 256);
    const int KS = (S + UR * R - 1) / (UR * R);
    a.steps = R;
    if (KS > max_waves<UR, T>()) fail(LARQL_HIP_ERR_UNSUPPORTED, "q4k matvec: row too long for this split");
    const size_t shmem = static_cast<size_t>(KS) * (wave_lds_bytes<UR>() + 16 * T * sizeof(float)) +
                         (a.norm_w || a.x_psum ? kMaxKS * sizeof(double) : 0);
    if (a.x_psum && (a.norm_w || a.x_npsum > 2 * 64 * KS))
        fail(LARQL_HIP_ERR_INVALID, "q4k matvec: prenormed input with a norm, or too many partial sums");
    if ((a.out2 || a.psum) && (a.epi != EPI_RESID || a.norm_w))
        fail(LARQL_HIP_ERR_INVALID, "q4k matvec: out2 / psum need EPI_RESID and no fused norm");
    const dim3 grid(static_cast<unsigned>(w.rows_pad / (16 * T))), block(64 * KS);
    if (a.norm_w) q4k_mfma_kernel<UR, T, true, HF, PRE, XB><<<grid, block, shmem, s>>>(a);
    else q4k_mfma_kernel<UR, T, false, HF, PRE, XB><<<grid, block, shmem, s>>>(a);
    LARQL_HIP_CHECK(hipGetLastError());
}

// The launch split of a Q4_K-family weight: ur super-blocks per round, t tiles per
// workgroup, pre units issued with x, xb the x-first barrier, R rounds.
struct Q4kSplit {
    int ur, t, pre;
    bool xb;
    int R;
};

// Measured on MI355X (256 CUs, rotating weight copies, back-to-back launches): rows of
// <= 16 super-blocks with 1.5 .. 8 tiles per CU take two super-blocks per wave and two
// tiles per workgroup, the first two units' loads issued with x ([14336 x 4096] 7.2 us,
// against 7.73 with four tiles per workgroup; [6144 x 4096] 4.76 us; [28672 x 4096], 7
// tiles per CU: 12.30 us standalone against 12.15 with the split below, but in the 8B
// decode step, where it is the fused gate|up, 1.5368 against 1.5394 ms per step, five
// medians of 30 steps each way on one box, spread 0.001 ms); longer tile counts at <= 16 super-blocks take four super-blocks
// per wave, one tile per workgroup and four units issued with x, and the rest ([4096 x
// 4096] 3.9 us, [4096 x 14336] 7.5 us, against 8.1 with the loads of one unit issued
// with x) four super-blocks per wave, one tile per workgroup, x issued by every wave
// before any weight load.  Rows longer than 16 waves x 4 super-blocks (K > 16384) take
// several rounds.  The per-wave phases explain the spread: a wave cannot build its x
// planes before its x loads return, and those queue behind weight loads already in
// flight (planes ready 0.7 .. 5.8 us into a 7.5 us launch).
Q4kSplit pick_q4k_split(const DevWeight& w, int num_cus) {
    const size_t S = w.cols / 256;
    const size_t tiles = w.rows_pad / 16, cus = static_cast<size_t>(num_cus);
    const int R4 = static_cast<int>((S + 4 * kMaxKS - 1) / (4 * kMaxKS));
    if (S <= 16 && 2 * tiles >= 3 * cus && tiles < 8 * cus && w.rows_pad % 32 == 0) return {2, 2, 2, false, 1};
    if (S <= 16 && tiles >= 6 * cus) return {4, 1, 4, true, R4};
    return {4, 1, 2, true, R4};
}

}  // namespace

void launch_q4k_mfma(const DevWeight& w, MvArgs a, hipStream_t s) {
    if ((w.format != LARQL_Q4_K && w.format != LARQL_Q4_KF) || w.cols % 256 != 0 || w.cols == 0 || w.rows_pad % 16 != 0 ||
        w.cols > (size_t{1} << 24) || w.rows_pad / 16 > 0x7FFFFFFFu)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "q4k matvec: shape");
    if (a.num_cus <= 0) a.num_cus = current_device_cus();
    a.rows = static_cast<int>(w.rows);
    a.cols = static_cast<int>(w.cols);
    a.rows_pad = static_cast<int>(w.rows_pad);
    a.qs = w.qs;
    a.hdr = w.hdr;
    if (a.epi == EPI_GATED_PAIR && (w.rows & 1)) fail(LARQL_HIP_ERR_INVALID, "gated pair epilogue needs even rows");
    const Q4kSplit sp = pick_q4k_split(w, a.num_cus);
    auto go = [&](auto hf) {
        constexpr int HF = decltype(hf)::value;
        if (sp.ur == 2) launch_q4k_mfma_t<2, 2, HF, 2, false>(w, a, sp.R, s);
        else if (sp.pre == 4) launch_q4k_mfma_t<4, 1, HF, 4, true>(w, a, sp.R, s);
        else launch_q4k_mfma_t<4, 1, HF, 2, true>(w, a, sp.R, s);
    };
    if (w.format == LARQL_Q4_KF && w.hf == kHdrKf160) go(std::integral_constant<int, kHdrKf160>{});
    else if (w.format == LARQL_Q4_KF) go(std::integral_constant<int, kHdrGguf>{});
    else go(std::integral_constant<int, kHdr148>{});
}

int q4k_mfma_groups(const DevWeight& w, int num_cus) {
    if (num_cus <= 0) num_cus = current_device_cus();
    return static_cast<int>(w.rows_pad / (16 * pick_q4k_split(w, num_cus).t));
}

Q4kShape q4k_mfma_shape(const DevWeight& w, int num_cus) {
    if ((w.format != LARQL_Q4_K && w.format != LARQL_Q4_KF) || w.cols % 256 != 0 || w.cols == 0 || w.rows_pad % 16 != 0)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "q4k launch shape: not a Q4_K-family weight");
    if (num_cus <= 0) num_cus = current_device_cus();
    const Q4kSplit sp = pick_q4k_split(w, num_cus);
    const size_t S = w.cols / 256;
    const unsigned waves = static_cast<unsigned>((S + sp.ur * sp.R - 1) / (sp.ur * sp.R));
    return Q4kShape{sp.ur, sp.t, sp.pre, sp.xb ? 1 : 0, sp.R, static_cast<unsigned>(w.rows_pad / (16 * sp.t)),
                    64 * waves};
}

int q4k_mfma_max_psum(const DevWeight& w, int num_cus) {
    if (num_cus <= 0) num_cus = current_device_cus();
    const Q4kSplit sp = pick_q4k_split(w, num_cus);
    const size_t S = w.cols / 256;
    return static_cast<int>(2 * 64 * ((S + sp.ur * sp.R - 1) / (sp.ur * sp.R)));
}

namespace {

// Every byte of the weight's device allocation loaded once (16 B non-temporal loads,
// eight in flight per lane), XOR-folded to one word per workgroup: no arithmetic on the
// values, so its time is what memory alone allows for these bytes in this launch shape.
__global__ __launch_bounds__(64 * kMaxKS) void q4k_read_floor_kernel(const uint4* __restrict__ p, size_t n16,
                                                                      uint32_t* __restrict__ out) {
    const size_t G = static_cast<size_t>(gridDim.x) * blockDim.x;
    size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 7 * G < n16; i += 8 * G) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = load_nt(p + i + u * G);
#pragma unroll
        for (int u = 0; u < 8; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += G) {
        const uint4 v = load_nt(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc ^= static_cast<uint32_t>(__shfl_xor(static_cast<int>(acc), m));
    __shared__ uint32_t wv[kMaxKS];
    if ((threadIdx.x & 63) == 0) wv[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t f = 0;
        for (unsigned w = 0; w < blockDim.x / 64; w++) f ^= wv[w];
        out[blockIdx.x] = f;
    }
}

}  // namespace

void launch_q4k_read_floor(const DevWeight& w, uint32_t* out, size_t out_words, unsigned groups, unsigned threads,
                           int num_cus, hipStream_t s) {
    if (w.bytes % 16 != 0 || w.bytes == 0) fail(LARQL_HIP_ERR_UNSUPPORTED, "read floor: weight size");
    if (num_cus <= 0) num_cus = current_device_cus();
    if (groups == 0 && threads == 0) {
        if ((w.format != LARQL_Q4_K && w.format != LARQL_Q4_KF) || w.cols % 256 != 0 || w.rows_pad % 16 != 0)
            fail(LARQL_HIP_ERR_UNSUPPORTED, "read floor: the matvec launch shape is known for Q4_K-family weights only");
        const Q4kSplit sp = pick_q4k_split(w, num_cus);
        const size_t S = w.cols / 256;
        groups = static_cast<unsigned>(w.rows_pad / (16 * sp.t));
        threads = static_cast<unsigned>(64 * ((S + sp.ur * sp.R - 1) / (sp.ur * sp.R)));
    }
    if (groups == 0 || threads == 0 || threads % 64 != 0 || threads > 64 * kMaxKS)
        fail(LARQL_HIP_ERR_INVALID, "read floor: workgroup size must be 64 .. 1024 in steps of 64");
    if (out_words < groups) fail(LARQL_HIP_ERR_INVALID, "read floor: out holds fewer words than workgroups");
    q4k_read_floor_kernel<<<dim3(groups), dim3(threads), 0, s>>>(static_cast<const uint4*>(w.base), w.bytes / 16, out);
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace larql
