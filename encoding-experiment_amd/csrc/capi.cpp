// extern "C" entry points of liblarql_hip (declared in include/larql_hip.h).
//
// Every entry point: validate shapes on the host, lock the context, enqueue on the
// context stream (or the caller's stream for the *_dev forms) and translate any
// failure into a negative status plus a message (larql_hip_last_error).  Nothing in
// here falls back to a CPU computation: a failure is reported, and the caller decides
// (the reference callers fall back to the CPU backend on None, LV/src/index/gate.rs:684-704).
#include <atomic>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <new>

#include "larql_hip_internal.h"
#include "matvec_common.h"

using larql::DevWeight;
using larql::Error;
using larql::fail;

namespace larql {

int current_device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    LARQL_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) fail(LARQL_HIP_ERR_DEVICE, "device index out of range");
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        LARQL_HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

void* ensure(larql_hip_ctx* c, DeviceBuf& b, size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (b.n >= bytes) return b.p;
    if (b.p) {
        (void)c;
        LARQL_HIP_CHECK(hipDeviceSynchronize());  // the buffer may be in use on a caller's stream
        LARQL_HIP_CHECK(hipFree(b.p));
        b.p = nullptr;
        b.n = 0;
    }
    size_t want = bytes + bytes / 4;
    if (hipMalloc(&b.p, want) != hipSuccess) {
        b.p = nullptr;
        fail(LARQL_HIP_ERR_NOMEM, "hipMalloc of " + std::to_string(want) + " bytes failed");
    }
    b.n = want;
    return b.p;
}

const DevWeight& lookup(larql_hip_ctx* c, uint64_t handle) {
    auto it = c->weights.find(handle);
    if (it == c->weights.end()) fail(LARQL_HIP_ERR_INVALID, "unknown weight handle");
    return it->second;
}

static void check_shape(int format, size_t len, size_t rows, size_t cols, int hf) {
    if (rows == 0 || cols == 0) fail(LARQL_HIP_ERR_INVALID, "rows and cols must be nonzero");
    switch (format) {
        case LARQL_Q4_0:
        case LARQL_Q8_0:
            if (cols % 32) fail(LARQL_HIP_ERR_INVALID, "hidden must be a multiple of 32");
            break;
        case LARQL_Q4_K:
        case LARQL_Q4_KF:
        case LARQL_Q6_K:
            if (cols % 256) fail(LARQL_HIP_ERR_INVALID, "hidden must be a multiple of 256");
            break;
        case LARQL_F32:
            break;
        default: fail(LARQL_HIP_ERR_INVALID, "unknown quant format");
    }
    if (rows > 0x7FFFFFFF / 2) fail(LARQL_HIP_ERR_INVALID, "too many rows");
    const size_t need = rows * ref_row_bytes(format, cols, hf);
    if (len < need)
        fail(LARQL_HIP_ERR_INVALID, "weight buffer too small: " + std::to_string(len) + " < " +
                                        std::to_string(need) + " bytes");
}

static uint64_t register_impl(larql_hip_ctx* c, int format, const void* data, size_t len,
                              const float* q8_scales, size_t rows, size_t cols, bool on_device) {
    const int hf = format == LARQL_Q4_KF && rows && cols % 256 == 0 ? q4kf_form_checked(len, rows, cols) : kHdr148;
    check_shape(format, len, rows, cols, hf);
    if (!data) fail(LARQL_HIP_ERR_INVALID, "null weight pointer");
    if (format == LARQL_Q8_0 && !q8_scales) fail(LARQL_HIP_ERR_INVALID, "Q8_0 weights need scales");
    DevWeight w;
    w.format = format;
    w.hf = hf;
    w.rows = rows;
    w.rows_pad = pad_rows(rows);
    w.cols = cols;
    w.bytes = dev_layout_bytes(format, w.rows_pad, cols, hf);
    if (hipMalloc(&w.base, w.bytes) != hipSuccess)
        fail(LARQL_HIP_ERR_NOMEM, "hipMalloc of weight (" + std::to_string(w.bytes) + " bytes) failed");
    dev_layout_carve(w);
    if (w.rows_pad != rows) LARQL_HIP_CHECK(hipMemsetAsync(w.base, 0, w.bytes, c->stream));
    const size_t raw_bytes = rows * ref_row_bytes(format, cols, hf);
    const size_t sc_bytes = format == LARQL_Q8_0 ? rows * (cols / 32) * sizeof(float) : 0;
    try {
        const uint8_t* raw = static_cast<const uint8_t*>(data);
        const float* sc = q8_scales;
        if (!on_device) {
            uint8_t* stage = static_cast<uint8_t*>(ensure(c, c->stage_raw, raw_bytes + sc_bytes + 256));
            LARQL_HIP_CHECK(hipMemcpyAsync(stage, data, raw_bytes, hipMemcpyHostToDevice, c->stream));
            if (sc_bytes) {
                float* sdev = reinterpret_cast<float*>(stage + ((raw_bytes + 255) & ~size_t(255)));
                LARQL_HIP_CHECK(hipMemcpyAsync(sdev, q8_scales, sc_bytes, hipMemcpyHostToDevice, c->stream));
                sc = sdev;
            }
            raw = stage;
        }
        launch_repack(w, raw, sc, c->stream);
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
    } catch (...) {
        (void)hipFree(w.base);
        throw;
    }
    w.handle = c->next_handle++;
    c->weights.emplace(w.handle, w);
    return w.handle;
}

static void release(larql_hip_ctx* c, uint64_t handle);

uint64_t host_fingerprint(const void* data, size_t len) {
    const uint8_t* p = static_cast<const uint8_t*>(data);
    uint64_t h = 1469598103934665603ull ^ len;
    auto mix = [&](const uint8_t* q, size_t n) {
        for (size_t i = 0; i < n; i++) h = (h ^ q[i]) * 1099511628211ull;
    };
    if (len <= 4096) {
        mix(p, len);
    } else {
        for (size_t i = 0; i < 64; i++) mix(p + i * ((len - 64) / 63), 64);
    }
    return h;
}

const DevWeight& cached_weight(larql_hip_ctx* c, int format, const void* data, size_t len,
                               const float* q8_scales, size_t rows, size_t cols) {
    auto key = std::make_pair(data, len);
    const uint64_t fp = host_fingerprint(data, len) ^
                        (q8_scales ? host_fingerprint(q8_scales, rows * (cols / 32) * sizeof(float)) : 0);
    auto it = c->by_host.find(key);
    if (it != c->by_host.end()) {
        const DevWeight& w = lookup(c, it->second);
        if (w.format == format && w.rows == rows && w.cols == cols && w.host_fp == fp) return w;
        release(c, it->second);
    }
    uint64_t h = register_impl(c, format, data, len, q8_scales, rows, cols, false);
    auto& w = c->weights.at(h);
    w.host_ptr = data;
    w.host_len = len;
    w.host_fp = fp;
    c->by_host[key] = h;
    return w;
}

static void release(larql_hip_ctx* c, uint64_t handle) {
    auto it = c->weights.find(handle);
    if (it == c->weights.end()) fail(LARQL_HIP_ERR_INVALID, "unknown weight handle");
    LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
    if (it->second.host_ptr) c->by_host.erase(std::make_pair(it->second.host_ptr, it->second.host_len));
    (void)hipFree(it->second.base);
    c->weights.erase(it);
}

}  // namespace larql

#include "capi_util.h"

// ── lifecycle ────────────────────────────────────────────────────────────
extern "C" int larql_hip_ctx_create(int device, larql_hip_ctx** out) {
    if (!out) return LARQL_HIP_ERR_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return LARQL_HIP_ERR_DEVICE;
    if (device < 0 || device >= n) return LARQL_HIP_ERR_INVALID;
    larql_hip_ctx* c = new (std::nothrow) larql_hip_ctx();
    if (!c) return LARQL_HIP_ERR_NOMEM;
    c->device = device;
    hipDeviceProp_t prop;
    if (hipSetDevice(device) != hipSuccess || hipGetDeviceProperties(&prop, device) != hipSuccess ||
        hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return LARQL_HIP_ERR_DEVICE;
    }
    c->num_cus = prop.multiProcessorCount;
    c->device_name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
    try {
        larql::noalloc_scratch_init(device);  // with the device current (hipSetDevice above)
    } catch (const larql::Error&) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return LARQL_HIP_ERR_DEVICE;
    }
    *out = c;
    return LARQL_HIP_OK;
}

extern "C" void larql_hip_ctx_destroy(larql_hip_ctx* c) {
    if (!c) return;
    {
        std::lock_guard<std::recursive_mutex> lk(c->mu);
        (void)hipSetDevice(c->device);
        (void)hipStreamSynchronize(c->stream);
        for (auto& kv : c->weights) (void)hipFree(kv.second.base);
        c->weights.clear();
        try {
            larql_hip_decode_release(c);
        } catch (...) {
        }
        for (auto* b : {&c->stage_in, &c->stage_in2, &c->stage_out, &c->stage_raw, &c->scratch, &c->knn_scores,
                        &c->knn_q8, &c->knn_q8s, &c->knn_idx, &c->knn_val, &c->knn_handles, &c->vecmat_part,
                        &c->pair_q8, &c->pair_q8s, &c->knn_xa, &c->knn_xsp, &c->knn_xpad, &c->knn_sort, &c->knn_cand, &c->gemm_x16,
                        &c->ffn_work})
            if (b->p) (void)hipFree(b->p);
        (void)hipStreamDestroy(c->stream);
    }
    delete c;
}

extern "C" const char* larql_hip_last_error(larql_hip_ctx* c) { return c ? c->last_error.c_str() : "null context"; }

extern "C" const char* larql_hip_name(void) { return "hip (MI355X gfx950)"; }

extern "C" int larql_hip_device_info(larql_hip_ctx* c, char* buf, size_t len) {
    return guarded(c, [&] {
        if (!buf || len == 0) fail(LARQL_HIP_ERR_INVALID, "null buffer");
        size_t free_b = 0, total_b = 0;
        LARQL_HIP_CHECK(hipMemGetInfo(&free_b, &total_b));
        std::snprintf(buf, len, "HIP device %d: %s, %d CUs, %.1f GB HBM", c->device, c->device_name.c_str(),
                      c->num_cus, total_b / 1e9);
    });
}

extern "C" int larql_hip_has_q4(larql_hip_ctx* c) { return c ? 1 : 0; }
extern "C" int larql_hip_has_kv_cache(larql_hip_ctx* c) { return c ? 1 : 0; }

extern "C" int larql_hip_synchronize(larql_hip_ctx* c) {
    return guarded(c, [&] { LARQL_HIP_CHECK(hipStreamSynchronize(c->stream)); });
}

// ── registry ─────────────────────────────────────────────────────────────
extern "C" int larql_hip_register_weight(larql_hip_ctx* c, int format, const void* data, size_t len,
                                         const float* q8_scales, size_t rows, size_t cols, uint64_t* handle) {
    return guarded(c, [&] {
        if (!handle) fail(LARQL_HIP_ERR_INVALID, "null handle pointer");
        *handle = larql::register_impl(c, format, data, len, q8_scales, rows, cols, false);
    });
}

extern "C" int larql_hip_register_weight_device(larql_hip_ctx* c, int format, const void* dev_data, size_t len,
                                                const float* dev_q8_scales, size_t rows, size_t cols,
                                                uint64_t* handle) {
    return guarded(c, [&] {
        if (!handle) fail(LARQL_HIP_ERR_INVALID, "null handle pointer");
        *handle = larql::register_impl(c, format, dev_data, len, dev_q8_scales, rows, cols, true);
    });
}

extern "C" int larql_hip_release_weight(larql_hip_ctx* c, uint64_t handle) {
    return guarded(c, [&] { larql::release(c, handle); });
}

extern "C" int larql_hip_forget_host(larql_hip_ctx* c, const void* data) {
    return guarded(c, [&] {
        std::vector<uint64_t> drop;
        for (auto& kv : c->by_host)
            if (kv.first.first == data) drop.push_back(kv.second);
        for (uint64_t h : drop) larql::release(c, h);
    });
}

extern "C" int larql_hip_weight_device_bytes(larql_hip_ctx* c, uint64_t handle, size_t* bytes) {
    return guarded(c, [&] {
        if (!bytes) fail(LARQL_HIP_ERR_INVALID, "null output");
        *bytes = larql::lookup(c, handle).bytes;
    });
}

// ── host-memory trait methods ───────────────────────────────────────────
extern "C" int larql_hip_q4k_matvec(larql_hip_ctx* c, const uint8_t* q4k_data, size_t q4k_len, const float* x,
                                    float* out, size_t num_rows, size_t hidden) {
    return guarded(c, [&] {
        if (!q4k_data || !x || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const DevWeight& w = larql::cached_weight(c, LARQL_Q4_K, q4k_data, q4k_len, nullptr, num_rows, hidden);
        const float* dx = stage_upload(c, c->stage_in, x, hidden);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, num_rows * sizeof(float)));
        larql::launch_q4k_matvec(w, dx, dout, 1, nullptr, c->stream);
        download(c, out, dout, num_rows * sizeof(float));
    });
}

extern "C" int larql_hip_q4k_matmul(larql_hip_ctx* c, const uint8_t* q4k_data, size_t q4k_len, const float* x,
                                    size_t m, float* out, size_t num_rows, size_t hidden) {
    return guarded(c, [&] {
        if (!q4k_data || !x || !out || m == 0) fail(LARQL_HIP_ERR_INVALID, "null pointer or m == 0");
        const DevWeight& w = larql::cached_weight(c, LARQL_Q4_K, q4k_data, q4k_len, nullptr, num_rows, hidden);
        const float* dx = stage_upload(c, c->stage_in, x, m * hidden);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, m * num_rows * sizeof(float)));
        void* ws = m > 1 ? larql::ensure(c, c->gemm_x16, larql::q4k_gemm_ws_bytes(m, hidden)) : nullptr;
        larql::launch_q4k_matvec(w, dx, dout, m, ws, c->stream);
        download(c, out, dout, m * num_rows * sizeof(float));
    });
}

extern "C" int larql_hip_matmul(larql_hip_ctx* c, const float* a, size_t m, size_t k, const float* b, size_t n,
                                int transpose_b, float* out) {
    return guarded(c, [&] {
        if (m == 0 || n == 0) return;
        if (!out || (k > 0 && (!a || !b))) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const float* da = k ? stage_upload(c, c->stage_in, a, m * k) : nullptr;
        const float* db = k ? stage_upload(c, c->stage_in2, b, n * k) : nullptr;
        float* dc = static_cast<float*>(larql::ensure(c, c->stage_out, m * n * sizeof(float)));
        larql::launch_f32_matmul(da, db, dc, m, k, n, transpose_b != 0, c->stream);
        download(c, out, dc, m * n * sizeof(float));
    });
}

extern "C" int larql_hip_matmul_dev(larql_hip_ctx* c, const float* a, size_t m, size_t k, const float* b, size_t n,
                                    int transpose_b, float* out, void* stream) {
    return guarded(c, [&] {
        if (m == 0 || n == 0) return;
        if (!out || (k > 0 && (!a || !b))) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        larql::launch_f32_matmul(a, b, out, m, k, n, transpose_b != 0, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_q6k_matvec(larql_hip_ctx* c, const uint8_t* q6k_data, size_t q6k_len, const float* x,
                                    float* out, size_t num_rows, size_t hidden) {
    return guarded(c, [&] {
        if (!q6k_data || !x || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const DevWeight& w = larql::cached_weight(c, LARQL_Q6_K, q6k_data, q6k_len, nullptr, num_rows, hidden);
        const float* dx = stage_upload(c, c->stage_in, x, hidden);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, num_rows * sizeof(float)));
        larql::launch_q6k_matvec(w, dx, dout, 1, c->stream);
        download(c, out, dout, num_rows * sizeof(float));
    });
}

extern "C" int larql_hip_q4_matvec(larql_hip_ctx* c, const uint8_t* q4_data, size_t q4_len, const int8_t* q8_x,
                                   const float* q8_scales, float* scores, size_t num_rows, size_t hidden) {
    return guarded(c, [&] {
        if (!q4_data || !q8_x || !q8_scales || !scores) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const DevWeight& w = larql::cached_weight(c, LARQL_Q4_0, q4_data, q4_len, nullptr, num_rows, hidden);
        const int8_t* dq = stage_upload(c, c->stage_in, q8_x, hidden);
        const float* ds = stage_upload(c, c->stage_in2, q8_scales, hidden / 32);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, num_rows * sizeof(float)));
        larql::launch_q4_0_matvec(w, dq, ds, dout, 1, c->stream);
        download(c, scores, dout, num_rows * sizeof(float));
    });
}

// ── Q4_0 walk-FFN: vecmat and gate/up pair batch ────────────────────────
static void run_vecmat(larql_hip_ctx* c, const DevWeight& w, const float* act, float* out, hipStream_t s) {
    const size_t chunks = larql::q4_vecmat_chunks(w.rows, w.cols);
    float* part = static_cast<float*>(larql::ensure(c, c->vecmat_part, chunks * w.cols * sizeof(float)));
    larql::launch_q4_vecmat(w, act, out, part, chunks, s);
}

extern "C" int larql_hip_q4_vecmat(larql_hip_ctx* c, const float* activation, const uint8_t* q4_data, size_t q4_len,
                                   float* out, size_t intermediate, size_t hidden) {
    return guarded(c, [&] {
        if (!activation || !q4_data || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const DevWeight& w = larql::cached_weight(c, LARQL_Q4_0, q4_data, q4_len, nullptr, intermediate, hidden);
        const float* da = stage_upload(c, c->stage_in, activation, intermediate);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, hidden * sizeof(float)));
        run_vecmat(c, w, da, dout, c->stream);
        download(c, out, dout, hidden * sizeof(float));
    });
}

extern "C" int larql_hip_vecmat_dev(larql_hip_ctx* c, uint64_t handle, const float* activation, float* out,
                                    void* stream) {
    return guarded(c, [&] {
        if (!activation || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const DevWeight& w = larql::lookup(c, handle);
        if (w.format != LARQL_Q4_0) fail(LARQL_HIP_ERR_UNSUPPORTED, "vecmat: Q4_0 weights only");
        run_vecmat(c, w, activation, out, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_read_floor_dev(larql_hip_ctx* c, uint64_t handle, unsigned workgroups, unsigned threads,
                                       uint32_t* out, size_t out_words, void* stream) {
    return guarded(c, [&] {
        if (!out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const DevWeight& w = larql::lookup(c, handle);
        larql::launch_q4k_read_floor(w, out, out_words, workgroups, threads, c->num_cus, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_q4k_launch_shape(larql_hip_ctx* c, uint64_t handle, int* ur, int* tiles, int* pre, int* xb,
                                          int* rounds, unsigned* workgroups, unsigned* threads) {
    return guarded(c, [&] {
        const larql::Q4kShape sh = larql::q4k_mfma_shape(larql::lookup(c, handle), c->num_cus);
        if (ur) *ur = sh.ur;
        if (tiles) *tiles = sh.tiles;
        if (pre) *pre = sh.pre;
        if (xb) *xb = sh.xb;
        if (rounds) *rounds = sh.rounds;
        if (workgroups) *workgroups = sh.groups;
        if (threads) *threads = sh.threads;
    });
}

static void run_pair_batch(larql_hip_ctx* c, const DevWeight& g, const DevWeight& u, const float* x, size_t seq,
                           float* gate_out, float* up_out, hipStream_t s) {
    if (g.format != LARQL_Q4_0 || u.format != LARQL_Q4_0) fail(LARQL_HIP_ERR_UNSUPPORTED, "pair batch: Q4_0 weights");
    if (g.rows != u.rows || g.cols != u.cols) fail(LARQL_HIP_ERR_INVALID, "pair batch: gate and up shapes differ");
    if (seq == 0) return;
    const size_t hidden = g.cols;
    int8_t* q8 = static_cast<int8_t*>(larql::ensure(c, c->pair_q8, seq * hidden));
    float* q8s = static_cast<float*>(larql::ensure(c, c->pair_q8s, seq * (hidden / 32) * sizeof(float)));
    larql::launch_quantize_q8(x, hidden, seq, q8, q8s, s);
    larql::launch_q4_0_matvec_pair(g, u, q8, q8s, gate_out, up_out, seq, s);
}

extern "C" int larql_hip_q4_matvec_pair_batch(larql_hip_ctx* c, const uint8_t* gate_q4, size_t gate_len,
                                              const uint8_t* up_q4, size_t up_len, const float* x_matrix,
                                              size_t seq_len, float* gate_out, float* up_out, size_t num_rows,
                                              size_t hidden) {
    return guarded(c, [&] {
        if (!gate_q4 || !up_q4 || !x_matrix || !gate_out || !up_out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        if (seq_len == 0) return;
        // copies: the second lookup may insert into the registry
        const DevWeight g = larql::cached_weight(c, LARQL_Q4_0, gate_q4, gate_len, nullptr, num_rows, hidden);
        const DevWeight u = larql::cached_weight(c, LARQL_Q4_0, up_q4, up_len, nullptr, num_rows, hidden);
        const float* dx = stage_upload(c, c->stage_in, x_matrix, seq_len * hidden);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, 2 * seq_len * num_rows * sizeof(float)));
        run_pair_batch(c, g, u, dx, seq_len, dout, dout + seq_len * num_rows, c->stream);
        LARQL_HIP_CHECK(hipMemcpyAsync(gate_out, dout, seq_len * num_rows * sizeof(float), hipMemcpyDeviceToHost,
                                       c->stream));
        download(c, up_out, dout + seq_len * num_rows, seq_len * num_rows * sizeof(float));
    });
}

extern "C" int larql_hip_pair_batch_dev(larql_hip_ctx* c, uint64_t gate, uint64_t up, const float* x, size_t seq_len,
                                        float* gate_out, float* up_out, void* stream) {
    return guarded(c, [&] {
        if (!x || !gate_out || !up_out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const DevWeight g = larql::lookup(c, gate);
        const DevWeight u = larql::lookup(c, up);
        run_pair_batch(c, g, u, x, seq_len, gate_out, up_out, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_quantize_to_q8(larql_hip_ctx* c, const float* x, size_t n, int8_t* q8, float* scales) {
    return guarded(c, [&] {
        if (!x || !q8 || !scales) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        if (n % 32) fail(LARQL_HIP_ERR_INVALID, "length must be a multiple of 32");
        const float* dx = stage_upload(c, c->stage_in, x, n);
        uint8_t* o = static_cast<uint8_t*>(larql::ensure(c, c->stage_out, n + n / 32 * 4 + 256));
        float* os = reinterpret_cast<float*>(o + ((n + 255) & ~size_t(255)));
        larql::launch_quantize_q8(dx, n, 1, reinterpret_cast<int8_t*>(o), os, c->stream);
        LARQL_HIP_CHECK(hipMemcpyAsync(q8, o, n, hipMemcpyDeviceToHost, c->stream));
        download(c, scales, os, n / 32 * sizeof(float));
    });
}

extern "C" int larql_hip_q8_matvec(larql_hip_ctx* c, const int8_t* w_q8, size_t w_len, const float* w_scales,
                                   const int8_t* x_q8, const float* x_scales, size_t m, float* out,
                                   size_t num_rows, size_t hidden) {
    return guarded(c, [&] {
        if (!w_q8 || !w_scales || !x_q8 || !x_scales || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        if (m == 0) fail(LARQL_HIP_ERR_INVALID, "m must be >= 1");
        const DevWeight& w = larql::cached_weight(c, LARQL_Q8_0, w_q8, w_len, w_scales, num_rows, hidden);
        const int8_t* dq = stage_upload(c, c->stage_in, x_q8, m * hidden);
        const float* ds = stage_upload(c, c->stage_in2, x_scales, m * (hidden / 32));
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, m * num_rows * sizeof(float)));
        larql::launch_q8_matvec(w, dq, ds, dout, m, c->stream);
        download(c, out, dout, m * num_rows * sizeof(float));
    });
}

// ── device-resident fast path ───────────────────────────────────────────
extern "C" int larql_hip_matvec_dev(larql_hip_ctx* c, uint64_t handle, const void* x, const float* x_scales,
                                    float* out, size_t m, void* stream) {
    return guarded(c, [&] {
        const DevWeight& w = larql::lookup(c, handle);
        if (!x || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        hipStream_t s = pick_stream(c, stream);
        switch (w.format) {
            case LARQL_Q4_K: {
                void* ws = m > 1 ? larql::ensure(c, c->gemm_x16, larql::q4k_gemm_ws_bytes(m, w.cols)) : nullptr;
                larql::launch_q4k_matvec(w, static_cast<const float*>(x), out, m, ws, s);
                break;
            }
            case LARQL_Q4_KF:  // one matvec per activation row
                for (size_t i = 0; i < m; i++)
                    larql::launch_q4k_matvec(w, static_cast<const float*>(x) + i * w.cols, out + i * w.rows, 1,
                                             nullptr, s);
                break;
            case LARQL_Q6_K:
                if (m > 1) {  // the prompt pass's f32-accuracy GEMM; row exponents and K-split partials in the workspace
                    const size_t pf = larql::q4k_gemm_f32_part_floats(w, m);
                    float* part = pf ? static_cast<float*>(larql::ensure(c, c->gemm_x16, pf * sizeof(float))) : nullptr;
                    larql::launch_q4k_gemm_f32(w, static_cast<const float*>(x), out, m, part, pf, s, 0);
                } else {
                    larql::launch_q6k_matvec(w, static_cast<const float*>(x), out, m, s);
                }
                break;
            case LARQL_Q4_0:
                if (!x_scales) fail(LARQL_HIP_ERR_INVALID, "Q4_0 matvec needs Q8 activation scales");
                larql::launch_q4_0_matvec(w, static_cast<const int8_t*>(x), x_scales, out, m, s);
                break;
            case LARQL_Q8_0:
                if (!x_scales) fail(LARQL_HIP_ERR_INVALID, "Q8_0 matvec needs Q8 activation scales");
                larql::launch_q8_matvec(w, static_cast<const int8_t*>(x), x_scales, out, m, s);
                break;
            default: fail(LARQL_HIP_ERR_UNSUPPORTED, "unsupported format");
        }
    });
}

extern "C" int larql_hip_quantize_to_q8_dev(larql_hip_ctx* c, const float* x, size_t n, size_t m, int8_t* q8,
                                            float* scales, void* stream) {
    return guarded(c, [&] {
        if (!x || !q8 || !scales) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        if (n % 32) fail(LARQL_HIP_ERR_INVALID, "length must be a multiple of 32");
        larql::launch_quantize_q8(x, n, m, q8, scales, pick_stream(c, stream));
    });
}

// ── weight quantizers ───────────────────────────────────────────────────
static size_t quantized_bytes(int format, size_t n) {
    switch (format) {
        case LARQL_Q4_0:
            if (n % 32) fail(LARQL_HIP_ERR_INVALID, "length must be a multiple of 32");
            return n / 32 * 18;
        case LARQL_Q8_0:
            if (n % 32) fail(LARQL_HIP_ERR_INVALID, "length must be a multiple of 32");
            return n;
        case LARQL_Q4_K:
            if (n % 256) fail(LARQL_HIP_ERR_INVALID, "length must be a multiple of 256");
            return n / 256 * 148;
        case LARQL_Q6_K:
            if (n % 256) fail(LARQL_HIP_ERR_INVALID, "length must be a multiple of 256");
            return n / 256 * 210;
        default: fail(LARQL_HIP_ERR_UNSUPPORTED, "unsupported quant format");
    }
}

extern "C" int larql_hip_quantize_weights(larql_hip_ctx* c, int format, const float* x, size_t n, void* out,
                                          float* q8_scales) {
    return guarded(c, [&] {
        if (!x || !out || (format == LARQL_Q8_0 && !q8_scales)) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const size_t ob = quantized_bytes(format, n);
        const float* dx = stage_upload(c, c->stage_in, x, n);
        uint8_t* o = static_cast<uint8_t*>(larql::ensure(c, c->stage_out, ob + n / 32 * 4 + 512));
        float* os = reinterpret_cast<float*>(o + ((ob + 255) & ~size_t(255)));
        larql::launch_quantize_weights(format, dx, n, o, os, c->stream);
        LARQL_HIP_CHECK(hipMemcpyAsync(out, o, ob, hipMemcpyDeviceToHost, c->stream));
        if (format == LARQL_Q8_0)
            LARQL_HIP_CHECK(hipMemcpyAsync(q8_scales, os, n / 32 * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
    });
}

extern "C" int larql_hip_quantize_weights_dev(larql_hip_ctx* c, int format, const float* x, size_t n, void* out,
                                              float* q8_scales, void* stream) {
    return guarded(c, [&] {
        if (!x || !out || (format == LARQL_Q8_0 && !q8_scales)) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        (void)quantized_bytes(format, n);
        larql::launch_quantize_weights(format, x, n, out, q8_scales, pick_stream(c, stream));
    });
}
