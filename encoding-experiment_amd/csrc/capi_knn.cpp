// Gate-KNN entry points (vindex code in the reference, not trait methods):
// VectorIndex::gate_knn / gate_knn_batch / gate_knn_q4 / top_k_from_scores,
// LV/src/index/gate.rs:14-29, 108-134, 307-316, 500-537, 711-731.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>
#include <vector>

#include "capi_util.h"
#include "knn.h"

using larql::DevWeight;
using larql::fail;

namespace {

struct KnnPlan {
    int format = 0;
    int F = 0, K = 0;
    larql::KnnLayers a{}, b{};  // f32: a = rows; Q4_0: a = nibbles, b = f16 scales
};

KnnPlan plan_layers(larql_hip_ctx* c, const uint64_t* handles, size_t n_layers) {
    if (!handles || n_layers == 0) fail(LARQL_HIP_ERR_INVALID, "gate KNN: no layers");
    if (n_layers > static_cast<size_t>(larql::kMaxKnnLayers))
        fail(LARQL_HIP_ERR_INVALID, "gate KNN: more than LARQL_HIP_KNN_MAX_LAYERS layers in one call");
    KnnPlan p;
    for (size_t l = 0; l < n_layers; l++) {
        const DevWeight& w = larql::lookup(c, handles[l]);
        if (w.format != LARQL_F32 && w.format != LARQL_Q4_0)
            fail(LARQL_HIP_ERR_UNSUPPORTED, "gate KNN: gate weights must be LARQL_F32 or LARQL_Q4_0");
        if (l == 0) {
            p.format = w.format;
            p.F = static_cast<int>(w.rows);
            p.K = static_cast<int>(w.cols);
        } else if (w.format != p.format || static_cast<int>(w.rows) != p.F || static_cast<int>(w.cols) != p.K) {
            fail(LARQL_HIP_ERR_INVALID, "gate KNN: layers differ in format or shape");
        }
        p.a.p[l] = w.qs;
        p.b.p[l] = w.d;
    }
    if (p.format == LARQL_Q4_0 && p.K % 64) fail(LARQL_HIP_ERR_INVALID, "gate KNN: Q4_0 hidden must be a multiple of 64");
    return p;
}

// Scores [n_layers][nq][F] into `scores` (device).
void run_scores(larql_hip_ctx* c, const KnnPlan& p, size_t n_layers, const float* queries, size_t nq, float* scores,
                hipStream_t s) {
    if (!queries || !scores || nq == 0) fail(LARQL_HIP_ERR_INVALID, "gate KNN: null queries/scores or nq == 0");
    if (nq > 0x7FFFFFFF / static_cast<size_t>(p.K)) fail(LARQL_HIP_ERR_INVALID, "gate KNN: too many queries");
    const int Q = static_cast<int>(nq);
    if (p.format == LARQL_F32) {
        // rows of the device gate are f32_row_stride(K) apart; queries are padded to match
        const size_t Kp = larql::f32_row_stride(static_cast<size_t>(p.K));
        const float* X = queries;
        if (Kp != static_cast<size_t>(p.K)) {
            float* xp = static_cast<float*>(larql::ensure(c, c->knn_xpad, nq * Kp * sizeof(float)));
            larql::launch_pad_rows_f32(queries, xp, nq, static_cast<size_t>(p.K), Kp, 0.0f, s);
            X = xp;
        }
        larql::launch_gate_scores_f32(p.a, static_cast<int>(n_layers), X, scores, p.F, static_cast<int>(Kp), Q, s);
    } else {
        int8_t* q8 = static_cast<int8_t*>(larql::ensure(c, c->knn_q8, nq * p.K));
        float* q8s = static_cast<float*>(larql::ensure(c, c->knn_q8s, nq * (p.K / 32) * sizeof(float)));
        larql::launch_quantize_q8(queries, static_cast<size_t>(p.K), nq, q8, q8s, s);
        uint4* xa = static_cast<uint4*>(larql::ensure(c, c->knn_xa, larql::q4_xa_bytes(p.K, Q)));
        float* xsp = static_cast<float*>(larql::ensure(c, c->knn_xsp, larql::q4_xsp_bytes(p.K, Q)));
        larql::launch_gate_scores_q4(p.a, p.b, static_cast<int>(n_layers), q8, q8s, xa, xsp, scores, p.F, p.K, Q, s);
    }
}

// top_k above the row length is clamped by the kernels (top_k.min(len), LV/src/index/walk.rs:569);
// any k >= 1 is taken (the output holds rows x k slots).
void check_k(size_t k, size_t rows = 1) {
    if (k < 1 || rows * k >= (size_t{1} << 31)) fail(LARQL_HIP_ERR_INVALID, "top-k: need top_k >= 1 and rows x top_k < 2^31");
}

// Top-k of rows of n scores: the selection kernels up to LARQL_HIP_TOPK_MAX, above it the
// sorted path (same order) with a context work buffer.
void topk_any(larql_hip_ctx* c, const float* S, size_t rows, size_t stride, int n, size_t k, int signed_mode,
              uint32_t* idx, float* val, hipStream_t s) {
    if (k <= static_cast<size_t>(larql::kTopkMaxK)) {
        const size_t slots = larql::topk_candidate_slots(rows, n, static_cast<int>(k));
        uint32_t* ci = nullptr;
        float* cv = nullptr;
        if (slots) {  // long rows: chunks on many CUs, then their candidates
            ci = static_cast<uint32_t*>(larql::ensure(c, c->knn_cand, 2 * slots * sizeof(uint32_t)));
            cv = reinterpret_cast<float*>(ci + slots);
        }
        larql::launch_topk(S, rows, stride, n, static_cast<int>(k), signed_mode, idx, val, s, ci, cv);
        return;
    }
    const size_t wb = larql::topk_sorted_work_bytes(rows, n);
    void* w = larql::ensure(c, c->knn_sort, wb);
    larql::launch_topk_sorted(S, rows, stride, n, k, signed_mode, idx, val, w, wb, s);
}

}  // namespace

extern "C" int larql_hip_gate_scores_dev(larql_hip_ctx* c, const uint64_t* handles, size_t n_layers,
                                         const float* queries, size_t nq, float* scores, void* stream) {
    return guarded(c, [&] {
        const KnnPlan p = plan_layers(c, handles, n_layers);
        run_scores(c, p, n_layers, queries, nq, scores, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_gate_knn_dev(larql_hip_ctx* c, const uint64_t* handles, size_t n_layers,
                                      const float* queries, size_t nq, size_t top_k, uint32_t* idx, float* scores,
                                      void* stream) {
    return guarded(c, [&] {
        const KnnPlan p = plan_layers(c, handles, n_layers);
        check_k(top_k, n_layers * nq);
        if (!idx || !scores) fail(LARQL_HIP_ERR_INVALID, "gate KNN: null outputs");
        hipStream_t s = pick_stream(c, stream);
        float* S = static_cast<float*>(larql::ensure(c, c->knn_scores, n_layers * nq * p.F * sizeof(float)));
        run_scores(c, p, n_layers, queries, nq, S, s);
        topk_any(c, S, n_layers * nq, static_cast<size_t>(p.F), p.F, top_k, 0, idx, scores, s);
    });
}

extern "C" int larql_hip_topk_dev(larql_hip_ctx* c, const float* scores, size_t rows, size_t n, size_t k,
                                  int signed_mode, uint32_t* idx, float* vals, void* stream) {
    return guarded(c, [&] {
        if (!scores || !idx || !vals) fail(LARQL_HIP_ERR_INVALID, "top-k: null pointer");
        if (n == 0 || n > 0x7FFFFFFF) fail(LARQL_HIP_ERR_INVALID, "top-k: bad row length");
        check_k(k, rows);
        topk_any(c, scores, rows, n, static_cast<int>(n), k, signed_mode ? 1 : 0, idx, vals, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_gate_knn(larql_hip_ctx* c, int format, const void* gate, size_t gate_len, size_t features,
                                  size_t hidden, const float* queries, size_t nq, size_t top_k, uint32_t* idx,
                                  float* scores) {
    return guarded(c, [&] {
        if (format != LARQL_F32 && format != LARQL_Q4_0)
            fail(LARQL_HIP_ERR_UNSUPPORTED, "gate KNN: format must be LARQL_F32 or LARQL_Q4_0");
        if (!queries || !idx || !scores || nq == 0) fail(LARQL_HIP_ERR_INVALID, "gate KNN: null pointer or nq == 0");
        const DevWeight& w = larql::cached_weight(c, format, gate, gate_len, nullptr, features, hidden);
        const uint64_t h = w.handle;
        const KnnPlan p = plan_layers(c, &h, 1);
        check_k(top_k, nq);
        const size_t qbytes = nq * hidden * sizeof(float);
        float* dq = static_cast<float*>(larql::ensure(c, c->stage_in, qbytes));
        LARQL_HIP_CHECK(hipMemcpyAsync(dq, queries, qbytes, hipMemcpyHostToDevice, c->stream));
        float* S = static_cast<float*>(larql::ensure(c, c->knn_scores, nq * p.F * sizeof(float)));
        run_scores(c, p, 1, dq, nq, S, c->stream);
        uint32_t* di = static_cast<uint32_t*>(larql::ensure(c, c->knn_idx, nq * top_k * sizeof(uint32_t)));
        float* dv = static_cast<float*>(larql::ensure(c, c->knn_val, nq * top_k * sizeof(float)));
        topk_any(c, S, nq, static_cast<size_t>(p.F), p.F, top_k, 0, di, dv, c->stream);
        LARQL_HIP_CHECK(hipMemcpyAsync(idx, di, nq * top_k * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
        LARQL_HIP_CHECK(hipMemcpyAsync(scores, dv, nq * top_k * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
    });
}

// lm-head KNN (LV/src/index/walk.rs:549-583): quantize_to_q8 of each query, the Q4_0
// matvec over the vocab, then the signed top-k, all on the device.  Work buffers: q8
// [nq][hidden], q8s [nq][hidden / 32], scores S [nq][vocab].
struct LmHeadBufs {
    int8_t* q8;
    float* q8s;
    float* S;
    uint32_t* ci = nullptr;  // top-k chunk candidates (topk_candidate_slots)
    float* cv = nullptr;
};

static void check_lm_head(const DevWeight& w, size_t nq, size_t top_k) {
    if (w.format != LARQL_Q4_0) fail(LARQL_HIP_ERR_UNSUPPORTED, "lm-head KNN: the head must be Q4_0");
    if (nq == 0) fail(LARQL_HIP_ERR_INVALID, "lm-head KNN: nq == 0");
    if (w.rows > 0x7FFFFFFF) fail(LARQL_HIP_ERR_UNSUPPORTED, "lm-head KNN: vocab too large");
    check_k(top_k, nq);
}

// Scores then the signed top-k (c: the context whose buffers the top-k uses; null: k within
// LARQL_HIP_TOPK_MAX and the chunk candidates in b.ci / b.cv).
static void launch_lm_head_knn(larql_hip_ctx* c, const DevWeight& w, const float* dq, size_t nq, size_t top_k,
                               const LmHeadBufs& b, uint32_t* di, float* dv, hipStream_t s) {
    larql::launch_quantize_q8(dq, w.cols, nq, b.q8, b.q8s, s);
    larql::launch_q4_0_matvec(w, b.q8, b.q8s, b.S, nq, s);
    if (c) topk_any(c, b.S, nq, w.rows, static_cast<int>(w.rows), top_k, 1, di, dv, s);
    else larql::launch_topk(b.S, nq, w.rows, static_cast<int>(w.rows), static_cast<int>(top_k), 1, di, dv, s, b.ci, b.cv);
}

static void run_lm_head_knn(larql_hip_ctx* c, const DevWeight& w, const float* dq, size_t nq, size_t top_k,
                            uint32_t* di, float* dv, hipStream_t s) {
    check_lm_head(w, nq, top_k);
    const size_t hidden = w.cols, nb = hidden / 32;
    LmHeadBufs b;
    b.q8 = static_cast<int8_t*>(larql::ensure(c, c->knn_q8, nq * hidden));
    b.q8s = static_cast<float*>(larql::ensure(c, c->knn_q8s, nq * nb * sizeof(float)));
    b.S = static_cast<float*>(larql::ensure(c, c->knn_scores, nq * w.rows * sizeof(float)));
    launch_lm_head_knn(c, w, dq, nq, top_k, b, di, dv, s);
}

// ── the allocation-free lm-head KNN ──────────────────────────────────────
// Its work buffers live in one fixed device array per GPU, held until the process ends.
// Host code reaches each GPU's copy only through the address hipGetSymbolAddress returns
// on that GPU (recorded once per device by noalloc_scratch_init, which every context
// creation runs with its device current): the array's name on the host is a stand-in,
// not a device address.
static __device__ __align__(256) uint8_t scratch[LARQL_HIP_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

size_t align256(size_t n) { return (n + 255) & ~size_t(255); }
}  // namespace

namespace larql {
void noalloc_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) fail(LARQL_HIP_ERR_DEVICE, "device index out of range");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[device]) return;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        fail(LARQL_HIP_ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
}
}  // namespace larql

extern "C" int larql_hip_lm_head_knn(larql_hip_ctx* c, const uint8_t* lm_head_q4, size_t len, const float* query,
                                     size_t vocab, size_t hidden, size_t top_k, uint32_t* idx, float* scores) {
    return guarded(c, [&] {
        if (!lm_head_q4 || !query || !idx || !scores) fail(LARQL_HIP_ERR_INVALID, "lm-head KNN: null pointer");
        const DevWeight& w = larql::cached_weight(c, LARQL_Q4_0, lm_head_q4, len, nullptr, vocab, hidden);
        const float* dq = stage_upload(c, c->stage_in, query, hidden);
        uint32_t* di = static_cast<uint32_t*>(larql::ensure(c, c->knn_idx, top_k * sizeof(uint32_t)));
        float* dv = static_cast<float*>(larql::ensure(c, c->knn_val, top_k * sizeof(float)));
        run_lm_head_knn(c, w, dq, 1, top_k, di, dv, c->stream);
        LARQL_HIP_CHECK(hipMemcpyAsync(idx, di, top_k * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
        LARQL_HIP_CHECK(hipMemcpyAsync(scores, dv, top_k * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
    });
}

extern "C" int larql_hip_lm_head_knn_dev(larql_hip_ctx* c, uint64_t handle, const float* queries, size_t nq,
                                         size_t top_k, uint32_t* idx, float* scores, void* stream) {
    return guarded(c, [&] {
        if (!queries || !idx || !scores) fail(LARQL_HIP_ERR_INVALID, "lm-head KNN: null pointer");
        const DevWeight& w = larql::lookup(c, handle);
        run_lm_head_knn(c, w, queries, nq, top_k, idx, scores, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_lm_head_knn_dev_noalloc(larql_hip_ctx* c, uint64_t handle, const float* queries, size_t nq,
                                                 size_t top_k, uint32_t* idx, float* scores, void* stream) {
    return guarded(c, [&] {
        if (!queries || !idx || !scores) fail(LARQL_HIP_ERR_INVALID, "lm-head KNN: null pointer");
        const DevWeight& w = larql::lookup(c, handle);
        check_lm_head(w, nq, top_k);
        if (top_k > static_cast<size_t>(larql::kTopkMaxK))
            fail(LARQL_HIP_ERR_INVALID, "lm-head KNN (no-alloc): top_k above LARQL_HIP_TOPK_MAX needs a sort buffer");
        uint8_t* base = nullptr;
        {
            std::lock_guard<std::mutex> lk(g_scratch_mu);
            base = static_cast<uint8_t*>(g_scratch_ptr[c->device]);
        }
        if (!base) fail(LARQL_HIP_ERR_STATE, "lm-head KNN (no-alloc): scratch address not set up for this device");
        const size_t hidden = w.cols, nb = hidden / 32;
        const size_t need_q8 = align256(nq * hidden), need_q8s = align256(nq * nb * sizeof(float));
        const size_t need_s = align256(nq * w.rows * sizeof(float));
        const size_t slots = larql::topk_candidate_slots(nq, static_cast<int>(w.rows), static_cast<int>(top_k));
        const size_t need_c = 2 * slots * sizeof(uint32_t);
        const size_t need = need_q8 + need_q8s + need_s + need_c;
        if (nq * w.rows * sizeof(float) / sizeof(float) / nq != w.rows || need > LARQL_HIP_NOALLOC_SCRATCH_BYTES)
            fail(LARQL_HIP_ERR_INVALID, "lm-head KNN (no-alloc): nq * (vocab * 4 + hidden * 9 / 8) plus the top-k "
                                        "candidates needs " + std::to_string(need) + " bytes; the fixed scratch "
                                        "holds " + std::to_string(LARQL_HIP_NOALLOC_SCRATCH_BYTES));
        // every byte the kernels read is written first in the same call: nothing to clear
        LmHeadBufs b;
        b.q8 = reinterpret_cast<int8_t*>(base);
        b.q8s = reinterpret_cast<float*>(base + need_q8);
        b.S = reinterpret_cast<float*>(base + need_q8 + need_q8s);
        if (slots) {
            b.ci = reinterpret_cast<uint32_t*>(base + need_q8 + need_q8s + need_s);
            b.cv = reinterpret_cast<float*>(b.ci + slots);
        }
        launch_lm_head_knn(nullptr, w, queries, nq, top_k, b, idx, scores, pick_stream(c, stream));
    });
}
