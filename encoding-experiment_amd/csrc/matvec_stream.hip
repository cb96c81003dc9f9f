// Streaming Q6_K x f32 matvec: the decode-time weight sweep.
//
//   Q6_K (210-byte layout): LC/src/cpu/ops/q6k_matvec.rs:31-90, backend.rs:133-137.
//
// Shape of the launch (gfx950): a persistent grid of a few 256-thread workgroups per
// CU.  Each workgroup first builds the fixed-point image of the whole activation
// (optionally RMS-normalised) in LDS, 112 bytes per 32-element sub-block, while the
// first weight loads are already in flight.  Row groups (RB rows) are dealt to the
// waves grid-strided, and each wave sweeps its groups in "units" of one row group x
// 64 sub-blocks (one per lane).  Units stream through a ring of D
// register buffers: the loads of unit u + D - 1 are issued before unit u's arithmetic,
// so every wave keeps D - 1 units of weight bytes in flight at all times.  Each
// weight byte is read from HBM once, with wave-contiguous 16-byte loads from a
// wave-uniform row base.
//
// Arithmetic per lane and row: exact int32 v_dot4 of the 6-bit codes with the three
// x byte planes, then the f32 sub-block scale / min as in the reference factorisation
// sc * sum(q x) - mn * sum(x)  (LC/src/metal/shaders/q4k_matvec.rs:13-79).  Row sums
// over lanes use the permlane-swap transposing reduction; the epilogue is fused.
#include "kquant_levels.h"
#include "matvec_common.h"

#include <algorithm>

namespace larql {

namespace {

constexpr int kMaxWaves = 16;  // 1024-thread workgroups at most

// One sub-block's levels in LDS: three byte planes (even / odd element dwords) and
// {s', sum x, sum x[0:16], sum x[16:32]}.
struct LvSlot {
    uint4 e[3], o[3];
    float4 s;
};
static_assert(sizeof(LvSlot) == 112, "LDS level slot");

// Sum of a double over the workgroup (all threads get the total).
__device__ __forceinline__ double block_sum_d(double v, double* scratch) {
    v = wave_sum_d(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    double s = 0.0;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); w++) s += scratch[w];
    __syncthreads();
    return s;
}

// Per-unit weight registers of one row.
template <int FMT>
struct RowRegs;
template <>
struct RowRegs<LARQL_Q6_K> {
    uint4 l;      // 16 low-nibble bytes
    uint2 h;      // 8 high-bit bytes (regrouped at registration)
    uint32_t sd;  // int8 scales of the two 16-element groups | f16 super-block scale << 16
};

// One ring slot: RB rows x one pass, plus the residual of the lane's epilogue row
// (loaded with the unit so that no load is issued behind the ring).
template <int FMT, int RB>
struct Unit {
    RowRegs<FMT> r[RB];
    float rs;
};

// Epilogue with the residual already in a register: `tot` and `rv` are valid in lane
// (r << rsh) for row row0 + r.
template <int RB>
__device__ __forceinline__ void epilogue_rv(const MvArgs& a, float tot, float rv, int lane, int row0) {
    constexpr int rsh = rb_shift<RB>();
    const int r = lane >> rsh;
    const bool owner = (lane & ((1 << rsh) - 1)) == 0;
    const int row = row0 + r;
    if (a.epi == EPI_GATED_PAIR) {
        const float up = __shfl_down(tot, 1 << rsh, 64);
        if (owner && (r & 1) == 0 && row < a.rows) a.out[row >> 1] = gated_act(a.act, tot, up);
    } else if (owner && row < a.rows) {
        a.out[row] = epi_value(a, rv, tot);
    }
}

// Levels of R x 8-element slices, four lanes (a DPP quad) per 32-element sub-block:
// slice sl is quarter sl & 3 (elements 8q..8q+7) of sub-block sl >> 2.  The result is
// bit-identical to make_levels on the whole sub-block: the max is exact, and the sums
// keep its tree (sum of 8, plus the neighbour's 8 for the half, plus the other half).
template <int R>
__device__ __forceinline__ void store_levels_quads(float (&xv)[R][8], int nsl, int nt, LvSlot* lv) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int sl = static_cast<int>(threadIdx.x) + nt * r;
        float m = tree_max_abs<8>(xv[r]);
        m = fmaxf(m, dpp_f<DPP_QUAD_1032>(m));
        m = fmaxf(m, dpp_f<DPP_QUAD_2301>(m));
        const float sl8 = tree_sum<8>(xv[r]);
        const float half = sl8 + dpp_f<DPP_QUAD_1032>(sl8);    // elements 0..15 (q < 2) or 16..31
        const float other = dpp_f<DPP_QUAD_2301>(half);
        const float inv = m > 0.f ? kLevelScale / m : 0.f;
        uint32_t T[8];
#pragma unroll
        for (int k = 0; k < 8; k++) T[k] = __float_as_uint(fmaf(xv[r][k], inv, 12582912.0f)) - 0x4B400000u;
        if (sl < nsl) {
            const int q = sl & 3;
            LvSlot* slot = lv + (sl >> 2);
#pragma unroll
            for (int l = 0; l < 3; l++) {
                reinterpret_cast<uint32_t*>(&slot->e[l])[q] = gather_byte(T[0], T[2], T[4], T[6], 2 - l);
                reinterpret_cast<uint32_t*>(&slot->o[l])[q] = gather_byte(T[1], T[3], T[5], T[7], 2 - l);
            }
            if (q == 0) slot->s = make_float4(m / kLevelScale, half + other, half, other);
        }
    }
}

// Memory-op discipline (what keeps D - 1 units in flight): every global load in the
// main loop is unconditional and issued in program order (unit indices are clamped in
// scalar code), and no load is issued whose value is needed before older loads return,
// so the compiler's waits are vmcnt(N) with N = the loads issued after the one needed.
// R = 8-element x slices per thread (4 nsub <= R NT); NORM: fused RMSNorm of x.
template <int FMT, int RB, int D, int NT, int OCC, int R, bool NORM>
__global__ __launch_bounds__(NT, OCC) void kq_stream_kernel(MvArgs a) {
    extern __shared__ double dyn_lds[];
    double* scratch = dyn_lds;                                    // kMaxWaves doubles
    LvSlot* lv = reinterpret_cast<LvSlot*>(dyn_lds + kMaxWaves);  // nsub slots
    constexpr int rsh = rb_shift<RB>();

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsub = a.cols >> 5;
    const int nsl = 4 * nsub;      // 8-element x slices, <= R * NT
    const int npass = (nsub + 63) >> 6;
    const int S = a.cols >> 8;
    const int gw = blockIdx.x * (NT / 64) + wave;
    const int W = gridDim.x * (NT / 64);
    // Row groups are dealt out grid-strided: wave gw takes super-groups gw, gw + W, ...
    // (a super-group is `pairs` consecutive RB-row groups; with RB == 1 and the gate/up
    // pair epilogue a pair never straddles two waves).  At any moment the requests in
    // flight over the whole GPU then cover one contiguous window of the weights, which
    // HBM serves far better than one separate stream per wave (measured: 33 MB in
    // ~7 us instead of ~9 us at the same depth).
    const int pairs = (RB == 1 && a.epi == EPI_GATED_PAIR) ? 2 : 1;
    const int NSG = a.rows_pad / (RB * pairs);
    const int nsg = gw < NSG ? (NSG - gw + W - 1) / W : 0;
    const int U = nsg * pairs * npass;

    // 1. x (and the norm weights) of this thread's slices: issued first, spread evenly
    // over the workgroup (two 16-byte loads per slice).
    float xv[R][8], wv[NORM ? R : 1][8];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const int sl = min(static_cast<int>(threadIdx.x) + NT * r, nsl - 1);
        load_slice<8>(a.x, sl * 8, true, xv[r]);
        if constexpr (NORM) load_slice<8>(a.norm_w, sl * 8, true, wv[r]);
    }

    // 2. The first D - 1 units.
    const float* rsrc = a.resid ? a.resid : a.x;

    Unit<FMT, RB> buf[D];
    // next unit to load (clamped to the last one; a wave without units loads from a
    // valid super-group and computes nothing) and next unit to compute
    int lu = 0, lsg = min(gw, NSG - 1), lgi = 0, lp = 0;
    int csg = lsg, cgi = 0, cp = 0;
    float acc[RB];
#pragma unroll
    for (int r = 0; r < RB; r++) acc[r] = 0.f;
    float gate_tot = 0.f;  // RB == 1 gate/up pairs

    auto load_unit = [&](Unit<FMT, RB>& B) __attribute__((always_inline)) {
        const uint32_t c = static_cast<uint32_t>(min(lp * 64 + lane, nsub - 1));
#pragma unroll
        for (int r = 0; r < RB; r++) {
            const size_t row = static_cast<size_t>(lsg * pairs + lgi) * RB + r;
            {
                const uint8_t* lrow = a.qs + row * (static_cast<size_t>(a.cols) >> 1);
                const uint8_t* hrow = a.qh + row * (static_cast<size_t>(a.cols) >> 2);
                const int8_t* srow = a.sc + row * (static_cast<size_t>(a.cols) >> 4);
                // weights are read once per launch: non-temporal loads keep them from
                // displacing x and the scales in the caches
                typedef uint32_t nt4 __attribute__((ext_vector_type(4)));
                typedef uint32_t nt2 __attribute__((ext_vector_type(2)));
                const nt4 lv = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(lrow + c * 16u));
                const nt2 hv = __builtin_nontemporal_load(reinterpret_cast<const nt2*>(hrow + c * 8u));
                B.r[r].l = make_uint4(lv.x, lv.y, lv.z, lv.w);
                B.r[r].h = make_uint2(hv.x, hv.y);
                const uint32_t s2 = *reinterpret_cast<const uint16_t*>(srow + c * 2u);
                const uint32_t d = (a.d + row * S)[c >> 3];
                B.r[r].sd = s2 | (d << 16);
            }
        }
        const int rrow = a.resid ? min((lsg * pairs + lgi) * RB + (lane >> rsh), a.rows - 1) : 0;
        B.rs = rsrc[rrow];
        if (lu < U - 1) {
            ++lu;
            if (++lp == npass) {
                lp = 0;
                if (++lgi == pairs) { lgi = 0; lsg += W; }
            }
        }
    };

#pragma unroll
    for (int d = 0; d < D - 1; d++) load_unit(buf[d]);

    // 3. Levels of the (normalised, LI/src/residual.rs:17-33) activation into LDS.
    if constexpr (NORM) {
        double part[2] = {0.0, 0.0};  // two chains: latency, not order
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (static_cast<int>(threadIdx.x) + NT * r < nsl) {
#pragma unroll
                for (int k = 0; k < 8; k++)
                    part[k & 1] = fma(static_cast<double>(xv[r][k]), static_cast<double>(xv[r][k]), part[k & 1]);
            }
        }
        const double tot = block_sum_d(part[0] + part[1], scratch);
        // rms as the CPU path rounds it (LI/src/residual.rs:24); x * (1/rms) differs from
        // x / rms by at most one f32 rounding.
        const float rms = static_cast<float>(sqrt(tot / static_cast<double>(a.cols) + a.eps));
        const float inv_rms = 1.0f / rms;
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int k = 0; k < 8; k++) xv[r][k] = (xv[r][k] * inv_rms) * (a.norm_offset + wv[r][k]);
    }
    store_levels_quads<R>(xv, nsl, NT, lv);
    __syncthreads();

    // 4. Stream the units.
    auto compute_unit = [&](const Unit<FMT, RB>& B) __attribute__((always_inline)) {
        const int c = cp * 64 + lane;
        const bool valid = c < nsub;
        const LvSlot& L = lv[valid ? c : nsub - 1];
        uint32_t ev[3][4], od[3][4];
#pragma unroll
        for (int l = 0; l < 3; l++) {
            const uint4 e = L.e[l], o = L.o[l];
            ev[l][0] = e.x; ev[l][1] = e.y; ev[l][2] = e.z; ev[l][3] = e.w;
            od[l][0] = o.x; od[l][1] = o.y; od[l][2] = o.z; od[l][3] = o.w;
        }
        const float4 st = L.s;
        // Integer dots first, rows interleaved and each level split over two
        // accumulators: 6 * RB independent chains of length 4.
        {
            int ga[RB][2];
            uint32_t gb[RB][2], gc[RB][2];
#pragma unroll
            for (int r = 0; r < RB; r++)
#pragma unroll
                for (int p = 0; p < 2; p++) ga[r][p] = 0, gb[r][p] = 0u, gc[r][p] = 0u;
#pragma unroll
            for (int w = 0; w < 4; w++) {
#pragma unroll
                for (int r = 0; r < RB; r++) {
                    const uint4 l = B.r[r].l;
                    const uint32_t lw = w == 0 ? l.x : w == 1 ? l.y : w == 2 ? l.z : l.w;
                    const uint32_t H = (w >> 1) ? B.r[r].h.y : B.r[r].h.x;
                    const int sh = 4 * (w & 1);
                    const uint32_t qe = (lw & 0x0F0F0F0Fu) | (((H >> sh) & 0x03030303u) << 4);
                    const uint32_t qo = ((lw >> 4) & 0x0F0F0F0Fu) | (((H >> (sh + 2)) & 0x03030303u) << 4);
                    const int h2 = w >> 1;  // 16-element group
                    ga[r][h2] = sdot4(qe, ev[0][w], ga[r][h2]);
                    gb[r][h2] = udot4(qe, ev[1][w], gb[r][h2]);
                    gc[r][h2] = udot4(qe, ev[2][w], gc[r][h2]);
                    ga[r][h2] = sdot4(qo, od[0][w], ga[r][h2]);
                    gb[r][h2] = udot4(qo, od[1][w], gb[r][h2]);
                    gc[r][h2] = udot4(qo, od[2][w], gc[r][h2]);
                }
            }
#pragma unroll
            for (int r = 0; r < RB; r++) {
                const uint32_t sd = B.r[r].sd;
                const float d = h2f(sd >> 16);
                float sc0 = d * static_cast<float>(static_cast<int8_t>(sd & 0xFFu));
                float sc1 = d * static_cast<float>(static_cast<int8_t>((sd >> 8) & 0xFFu));
                if (!valid) { sc0 = 0.f; sc1 = 0.f; }
                // value = sc * (q6 - 32): group sum = sc * (sum(q6 * x) - 32 * sum(x))
                const float g0v = fmaf(-32.f, st.z, combine(ga[r][0], gb[r][0], gc[r][0], st.x));
                const float g1v = fmaf(-32.f, st.w, combine(ga[r][1], gb[r][1], gc[r][1], st.x));
                acc[r] = fmaf(sc0, g0v, fmaf(sc1, g1v, acc[r]));
            }
        }
        if (++cp == npass) {
            const int cg = csg * pairs + cgi;
            const float tot = multi_row_reduce<RB>(acc, lane);
            if constexpr (RB == 1) {
                // single-row groups: the gate row's total waits in a register for its up row
                if (a.epi == EPI_GATED_PAIR) {
                    if ((cg & 1) == 0) gate_tot = tot;
                    else if (lane == 0 && cg < a.rows) a.out[cg >> 1] = gated_act(a.act, gate_tot, tot);
                } else {
                    epilogue_rv<1>(a, tot, B.rs, lane, cg);
                }
            } else {
                epilogue_rv<RB>(a, tot, B.rs, lane, cg * RB);
            }
#pragma unroll
            for (int r = 0; r < RB; r++) acc[r] = 0.f;
            cp = 0;
            if (++cgi == pairs) { cgi = 0; csg += W; }
        }
    };

    for (int u0 = 0; u0 < U; u0 += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            load_unit(buf[(d + D - 1) % D]);
            if (u0 + d < U) compute_unit(buf[d]);
        }
    }
}

template <int FMT, int RB, int D, int NT, int OCC>
void launch_stream_t(const DevWeight& w, MvArgs a, hipStream_t s, int wg_per_cu) {
    const size_t ng = w.rows_pad / RB;
    const size_t cus = static_cast<size_t>(a.num_cus);
    // at least one row group per wave
    size_t grid = std::min(cus * static_cast<size_t>(wg_per_cu), (ng + NT / 64 - 1) / (NT / 64));
    if (grid == 0) grid = 1;
    const size_t shmem = kMaxWaves * sizeof(double) + (w.cols / 32) * sizeof(LvSlot);
    const size_t nsl = w.cols / 8;
    const dim3 g(static_cast<unsigned>(grid)), b(NT);
    const bool norm = a.norm_w != nullptr;
    if (nsl <= NT) {
        if (norm) kq_stream_kernel<FMT, RB, D, NT, OCC, 1, true><<<g, b, shmem, s>>>(a);
        else kq_stream_kernel<FMT, RB, D, NT, OCC, 1, false><<<g, b, shmem, s>>>(a);
    } else if (nsl <= 2 * NT) {
        if (norm) kq_stream_kernel<FMT, RB, D, NT, OCC, 2, true><<<g, b, shmem, s>>>(a);
        else kq_stream_kernel<FMT, RB, D, NT, OCC, 2, false><<<g, b, shmem, s>>>(a);
    } else {
        if (nsl > 4 * NT) fail(LARQL_HIP_ERR_UNSUPPORTED, "stream matvec: hidden too large for the workgroup");
        if (norm) kq_stream_kernel<FMT, RB, D, NT, OCC, 4, true><<<g, b, shmem, s>>>(a);
        else kq_stream_kernel<FMT, RB, D, NT, OCC, 4, false><<<g, b, shmem, s>>>(a);
    }
    LARQL_HIP_CHECK(hipGetLastError());
}

}  // namespace

// Largest K the streaming kernel takes (LDS holds 112 bytes per 32 columns).
constexpr size_t kStreamMaxCols = 16384;

static_assert(kStreamMaxCols / 8 <= 4 * 512, "prologue: at most four 8-element slices per thread of 512");

// Very tall matrices (a vocabulary head) stream faster through the tiled kernel, whose
// many small workgroups keep more rows in flight (measured: 128256 x 4096 Q6_K,
// 77 us tiled vs 86 us streaming).
constexpr size_t kStreamMaxRows = 65536;

bool stream_mv_supported(const DevWeight& w) {
    return w.format == LARQL_Q6_K && w.cols % 256 == 0 && w.cols <= kStreamMaxCols &&
           w.rows_pad % 8 == 0 && w.rows_pad < kStreamMaxRows;
}

void launch_mv_stream(const DevWeight& w, MvArgs a, hipStream_t s) {
    if (!stream_mv_supported(w)) fail(LARQL_HIP_ERR_UNSUPPORTED, "stream matvec: shape");
    if (a.num_cus <= 0) a.num_cus = current_device_cus();
    a.rows = static_cast<int>(w.rows);
    a.cols = static_cast<int>(w.cols);
    a.rows_pad = static_cast<int>(w.rows_pad);
    if (a.epi == EPI_GATED_PAIR && (w.rows & 1)) fail(LARQL_HIP_ERR_INVALID, "gated pair epilogue needs even rows");
    a.qs = w.qs;
    a.qh = w.qh;
    a.sc = w.sc;
    a.d = static_cast<const uint16_t*>(w.d);
    // One workgroup per CU, two rows per unit, four units in the ring.  The workgroup
    // has 8, 7 or 6 waves, whichever deals the row groups out most evenly (every wave
    // finishes with the last one): e.g. 7168 groups (14336 rows) -> 7 waves per CU,
    // four groups each; 3072 (a fused Q|K|V of 6144 rows) -> 6 waves, two each.
    // Measured (on the 4-bit form of this kernel, [14336 x 4096]): 9.2 us with 7 waves
    // vs 9.6 us with 8.
    const long long ng = static_cast<long long>(w.rows_pad) / 2;  // RB = 2: a group holds a gate/up pair
    int best_nt = 512;
    long long best_slots = 0;
    for (int nt : {512, 448, 384}) {
        if (w.cols / 8 > static_cast<size_t>(4 * nt)) continue;  // prologue: <= 4 x slices per thread
        const long long W = static_cast<long long>(a.num_cus) * (nt / 64);
        const long long slots = (ng + W - 1) / W * W;  // group slots incl. idle ones
        if (best_slots == 0 || slots < best_slots) best_slots = slots, best_nt = nt;
    }
    {
        if (best_nt == 448) launch_stream_t<LARQL_Q6_K, 2, 4, 448, 1>(w, a, s, 1);
        else if (best_nt == 384) launch_stream_t<LARQL_Q6_K, 2, 4, 384, 1>(w, a, s, 1);
        else launch_stream_t<LARQL_Q6_K, 2, 4, 512, 2>(w, a, s, 1);
    }
}

}  // namespace larql
