// Q6_K x f32 matvec with the integer sub-block dots on the matrix cores.
//
//   Reference semantics: LC/src/cpu/ops/q6k_matvec.rs:31-90 (trait method
//   LC/src/backend.rs:133-137): out[n] = sum over 16-element sub-blocks j of
//   d * sc_j * sum_i (q_i - 32) * x_i, q_i = (ql nibble) + 16 (qh bits), computed here as
//   (d sc_j) * (sum(q x) - 32 sum(x)) per sub-block (the factorisation of the Metal kernel,
//   LC/src/metal/shaders/q4k_matvec.rs:13-79).
//
// Work split and x digit planes as in the Q4_K kernel (matvec_q4k_mfma.hip): a workgroup
// owns T tiles of 16 consecutive rows; its KS waves split the super-blocks into parts of
// P = UR * R (wave w takes [wP, wP + P) of every tile), walked in R rounds of UR; each wave
// builds the digit planes (mfma_planes.h) of its own x slice in its own LDS area.
//
// Per unit (one super-block of one tile), lane (g, c) = lane 16 g + c takes row c,
// elements 64 g .. 64 g + 63 (sub-blocks 4 g .. 4 g + 3) from the tile-major device block
// (q6k_block, larql_hip_internal.h): 32 ql bytes (two 16-byte loads), the four qh group
// words 4 g .. 4 g + 3 (element 16 j + 8 w + 2 i + p at bits 8 i + 4 w + 2 p of word j),
// four int8 scales and the f16 d — each of those loads one contiguous span for the wave
// (the row-major layout spread each load over 16 rows: 13.5 against 9.7 us on
// [14336 x 4096]).  MFMA m (m = 0..3) takes sub-block 4 g + m of every lane as B — the
// 6-bit codes as bytes, even elements then odd ones — and as A row 4 s + p the digit
// plane p of x elements 64 s + 16 m .. + 15 in k-group s (zero in the other k-groups).
// Result lane 16 g + c, register p, is then the exact int32 dot of plane p with sub-block
// 4 g + m of row c: no cross-lane traffic until the end of the row.
#include <type_traits>

#include "kquant_levels.h"
#include "matvec_common.h"
#include "mfma_planes.h"

namespace larql {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// Slot k of a round holds the k-th 32-element x sub-block of the round's super-blocks;
// its float4 is {s', 65536 s', sum of elements 0..15, sum of elements 16..31}.
constexpr int kZeroBytes = 256;  // per-wave zero area read by the idle A lanes (offsets < 160)
constexpr int kMaxKS = 16;

template <int UR>
__host__ __device__ constexpr int q6_wave_lds_bytes() {
    return kZeroBytes + 8 * UR * static_cast<int>(sizeof(PlSlot));
}

// 8 units in flight, or 4 with the fused norm's x and norm-weight registers, need more
// than the 128 VGPRs of a 16-wave workgroup.
template <int UR, int T, bool NORM>
constexpr int q6_max_waves() {
    return UR * T >= (NORM ? 4 : 8) ? kMaxKS / 2 : kMaxKS;
}

// One unit's weight registers of a lane.
struct Q6Unit {
    uint4 l0, l1;  // ql bytes 32 g .. 32 g + 31
    uint4 h;       // qh words 4 g .. 4 g + 3
    uint32_t s;    // int8 scales of sub-blocks 4 g .. 4 g + 3
    uint32_t d;    // f16 d (low half)
};

// B operand of MFMA m: the 16 codes of sub-block 4 g + m, from ql dwords (2m, 2m + 1) and
// qh word m: {even elements 0..6, odd 1..7, even 8..14, odd 9..15}, code = nibble | hi2 << 4.
__device__ __forceinline__ v4i q6_codes(uint32_t l0, uint32_t l1, uint32_t H) {
    const uint32_t e0 = (l0 & 0x0F0F0F0Fu) | ((H << 4) & 0x30303030u);
    const uint32_t o0 = ((l0 >> 4) & 0x0F0F0F0Fu) | ((H << 2) & 0x30303030u);
    const uint32_t e1 = (l1 & 0x0F0F0F0Fu) | (H & 0x30303030u);
    const uint32_t o1 = ((l1 >> 4) & 0x0F0F0F0Fu) | ((H >> 2) & 0x30303030u);
    return v4i{static_cast<int>(e0), static_cast<int>(o0), static_cast<int>(e1), static_cast<int>(o1)};
}

// PRE: units whose loads are issued with x, before the planes are built (the rest after);
// XB: every wave's x loads are issued before any wave of the workgroup issues a weight
// load (a bare s_barrier between them).
template <int UR, int T, bool NORM, int PRE, bool XB>
__global__ __launch_bounds__((64 * q6_max_waves<UR, T, NORM>())) void q6k_mfma_kernel(MvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int EL = 4 * UR;  // x elements per lane and round
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KS = blockDim.x >> 6;
    const int R = a.steps;
    const int S = a.cols >> 8;
    const int sb0 = wave * UR * R;                 // first super-block of this wave
    const int nsb = max(0, min(UR * R, S - sb0));  // super-blocks of this wave
    const int g = lane >> 4, c = lane & 15;
    const size_t tile0 = static_cast<size_t>(blockIdx.x) * T;  // < rows_pad / 16: the grid is rows_pad / (16 T)
    const uint8_t* qb = a.qs + tile0 * S * kQ6Block;

    uint8_t* wl = lds + wave * q6_wave_lds_bytes<UR>();
    PlSlot* slots = reinterpret_cast<PlSlot*>(wl + kZeroBytes);
    float* red = reinterpret_cast<float*>(lds + KS * q6_wave_lds_bytes<UR>());  // [KS][16 T], then NORM scratch

    float xv[EL], wv[NORM ? EL : 1];
    Q6Unit un[T][UR];
    auto load_x = [&](int r) __attribute__((always_inline)) {
        const int e0 = (sb0 + r * UR) * 256 + lane * EL;
        load_slice<EL>(a.x, min(e0, a.cols - EL), true, xv);
        if constexpr (NORM) load_slice<EL>(a.norm_w, min(e0, a.cols - EL), true, wv);
    };
    // units are numbered t * UR + u (tile t, super-block u of the round); super-block
    // indices clamped: a short last round re-reads a real block
    auto load_units = [&](int r, int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int u = 0; u < UR; u++) {
                if (t * UR + u < i0 || t * UR + u >= i1) continue;
                const uint8_t* blk = qb + (static_cast<size_t>(t) * S + min(sb0 + r * UR + u, S - 1)) * kQ6Block;
                Q6Unit& q = un[t][u];
                q.l0 = load_nt(blk + lane * 16);
                q.l1 = load_nt(blk + 1024 + lane * 16);
                q.h = load_nt(blk + kQ6Qh + lane * 16);
                q.s = *reinterpret_cast<const uint32_t*>(blk + kQ6Sc + lane * 4);
                q.d = *reinterpret_cast<const uint16_t*>(blk + kQ6D + c * 2);
            }
    };
    load_x(0);
    if constexpr (XB) __builtin_amdgcn_s_barrier();
    load_units(0, 0, PRE);
    // Loaded now, used at the end (so the epilogue waits on no memory): wave 0's residual rows.
    float rv_pre = 0.f;
    if constexpr (!NORM) {
        const int row = static_cast<int>(blockIdx.x) * T * 16 + lane;
        if (wave == 0 && lane < 16 * T && row < a.rows && (a.epi == EPI_RESID || a.epi == EPI_GATED_MUL))
            rv_pre = a.resid[row];
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
        double* dscr = reinterpret_cast<double*>(red + KS * 16 * T);
        if (lane == 0) dscr[wave] = v;
        __syncthreads();
        double tot = 0.0;
        for (int w = 0; w < KS; w++) tot += dscr[w];
        // rms as the CPU path rounds it (LI/src/residual.rs:24); x * (1/rms) differs from
        // x / rms by at most one f32 rounding.
        const float rms = static_cast<float>(sqrt(tot / static_cast<double>(a.cols) + a.eps));
        inv_rms = 1.0f / rms;
    }

    // A lane (g, i): A row i = 4 s + p is live in k-group g iff s == g and p < 3; it reads
    // plane p of slot 2 g + m / 2 (of the unit), half m % 2.  The others read the zero area
    // (same immediate offsets, all inside it).
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
            float other;  // (lane of element 0) the sum of elements 16..31
            if constexpr (UR == 2) {
                m = fmaxf(m, dpp_f<DPP_QUAD_2301>(m));
                s = s + dpp_f<DPP_QUAD_1032>(s);  // a half: lanes of elements 0..15 or 16..31
                other = dpp_f<DPP_QUAD_2301>(s);
            } else {
                other = dpp_f<DPP_QUAD_1032>(s);  // a lane holds a half
            }
            const float inv = m > 0.f ? kLevelScale / m : 0.f;
            uint32_t u[EL];
#pragma unroll
            for (int k = 0; k < EL; k++)
                u[k] = __float_as_uint(fmaf(xv[k], inv, 12582912.0f)) + (0x808080u - 0x4B400000u);
            const int sub = (lane * EL) >> 5;  // x sub-block within the round (slot)
            const int ofs = (lane * EL) & 31;  // first element of the lane within it
            if (sub < 8 * nr) {
                PlSlot& sl = slots[sub];
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
                if (ofs == 0) sl.s = make_float4(m / kLevelScale, m * (65536.0f / kLevelScale), s, other);
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
                const Q6Unit& q = un[t][u];
                const uint8_t* ab = wl + abase + u * astep;
                const uint32_t lq[8] = {q.l0.x, q.l0.y, q.l0.z, q.l0.w, q.l1.x, q.l1.y, q.l1.z, q.l1.w};
                const uint32_t hq[4] = {q.h.x, q.h.y, q.h.z, q.h.w};
                v4i D[4];
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const uint4 av = *reinterpret_cast<const uint4*>(ab + (m >> 1) * sizeof(PlSlot) + (m & 1) * 48);
                    const v4i A = {(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                    D[m] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, q6_codes(lq[2 * m], lq[2 * m + 1], hq[m]),
                                                                 v4i{0, 0, 0, 0}, 0, 0, 0);
                }
                // sub-block 4 g + m: x slot 8 u + 2 g + m / 2, half m % 2
                const PlSlot* sl = slots + 8 * u + 2 * g;
                const float d = h2f(q.d);
#pragma unroll
                for (int m = 0; m < 4; m++) {
                    const float4 sv = sl[m >> 1].s;
                    const float xsum = (m & 1) ? sv.w : sv.z;
                    // s' (65536 a + 256 b + c): 256 b + c is exact in int32 and in f32 (< 2^24)
                    const float dot = fmaf(static_cast<float>(D[m][2]), sv.y, sv.x * static_cast<float>(D[m][1] * 256 + D[m][0]));
                    const float sc = d * static_cast<float>(static_cast<int8_t>((q.s >> (8 * m)) & 0xFFu));
                    acc[t] = fmaf(sc, fmaf(-32.f, xsum, dot), acc[t]);
                }
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
    __syncthreads();
    if (wave == 0) {
        const int row = static_cast<int>(blockIdx.x) * T * 16 + lane;
        float tot = 0.f;
        if (lane < 16 * T) {
            tot = red[lane];
            for (int w = 1; w < KS; w++) tot += red[w * 16 * T + lane];
        }
        if (a.epi == EPI_GATED_PAIR) {
            const float up = __shfl_down(tot, 1, 64);  // rows 2i, 2i + 1 sit in adjacent lanes of one tile
            if (lane < 16 * T && (lane & 1) == 0 && row < a.rows) a.out[row >> 1] = gated_act(a.act, tot, up);
        } else {
            const bool live = lane < 16 * T && row < a.rows;
            const float rv = a.epi == EPI_STORE ? 0.f : (NORM ? (live ? a.resid[row] : 0.f) : rv_pre);
            if (live) a.out[row] = epi_value(a, rv, tot);
        }
    }
}

// R rounds: the fewest that keep the waves within the kernel's limit.
template <int UR, int T, int PRE, bool XB>
void launch_q6k_mfma_t(const DevWeight& w, MvArgs a, hipStream_t s) {
    const int S = static_cast<int>(w.cols / 256);
    auto go = [&](auto norm) {
        constexpr bool NORM = decltype(norm)::value;
        constexpr int MW = q6_max_waves<UR, T, NORM>();
        const int R = (S + UR * MW - 1) / (UR * MW);
        const int KS = (S + UR * R - 1) / (UR * R);
        a.steps = R;
        const size_t shmem = static_cast<size_t>(KS) * (q6_wave_lds_bytes<UR>() + 16 * T * sizeof(float)) +
                             (NORM ? kMaxKS * sizeof(double) : 0);
        const dim3 grid(static_cast<unsigned>(w.rows_pad / (16 * T))), block(64 * KS);
        q6k_mfma_kernel<UR, T, NORM, PRE, XB><<<grid, block, shmem, s>>>(a);
    };
    if (a.norm_w) go(std::true_type{});
    else go(std::false_type{});
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace

bool q6k_mfma_supported(const DevWeight& w) {
    return w.format == LARQL_Q6_K && w.cols % 256 == 0 && w.cols > 0 && w.cols <= (size_t{1} << 16) &&
           w.rows_pad % 32 == 0 && w.rows_pad * (w.cols / 256) < (size_t{1} << 31);
}

// The launch split, as for the Q4_K kernel: rows of <= 16 super-blocks with 1.5 .. 6 tiles
// per CU take two super-blocks per wave and two tiles per workgroup, the first two units'
// loads issued with x; the others four super-blocks per wave, one tile per workgroup, x
// issued by every wave before any weight load; rows longer than 16 waves x 4 super-blocks
// take several rounds.
void launch_q6k_mfma(const DevWeight& w, MvArgs a, hipStream_t s) {
    if (!q6k_mfma_supported(w)) fail(LARQL_HIP_ERR_UNSUPPORTED, "q6k matvec: shape");
    if (a.x_psum || a.out2 || a.psum) fail(LARQL_HIP_ERR_INVALID, "q6k matvec: no prenormed input or second output");
    if (a.num_cus <= 0) a.num_cus = current_device_cus();
    a.rows = static_cast<int>(w.rows);
    a.cols = static_cast<int>(w.cols);
    a.rows_pad = static_cast<int>(w.rows_pad);
    a.qs = w.qs;
    if (a.epi == EPI_GATED_PAIR && (w.rows & 1)) fail(LARQL_HIP_ERR_INVALID, "gated pair epilogue needs even rows");
    const size_t S = w.cols / 256;
    const size_t tiles = w.rows_pad / 16, cus = static_cast<size_t>(a.num_cus);
    if (S <= 16 && 2 * tiles >= 3 * cus && tiles < 6 * cus) launch_q6k_mfma_t<2, 2, 2, false>(w, a, s);
    else if (S <= 16 && tiles >= 6 * cus) launch_q6k_mfma_t<4, 1, 4, true>(w, a, s);
    else launch_q6k_mfma_t<4, 1, 2, true>(w, a, s);
}

}  // namespace larql
