// Decode-step entry points: KV cache (ComputeBackend::{populate_kv_layer, reset_kv_cache},
// LC/src/backend.rs:99-110), decode_token (:115-123) and the device-resident model.
//
// A model holds, per layer, four device weights: Q|K|V concatenated by rows, Wo,
// gate/up interleaved by rows (row 2n = gate n, row 2n+1 = up n, so one matvec
// epilogue sees both and writes silu(gate)*up), and Wd; plus the two norm vectors.
// The host-pointer decode_token caches the model it built, keyed by the layers'
// pointers, lengths and sampled content (the Metal backend caches its buffers by host
// pointer, LC/src/metal/buffers.rs:37-85, and re-uses them for every token).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <algorithm>
#include <string>
#include <vector>

#include "capi_util.h"
#include "decode.h"
#include "matvec_common.h"

using larql::DevWeight;
using larql::fail;

struct LayerDev {
    // Q|K|V fused by rows and gate/up interleaved by rows when each pair shares a format;
    // otherwise separate weights (mixed Q4_K / Q6_K projections, as in Q4_K_M files)
    DevWeight qkv, wo, gateup, down;
    DevWeight wq, wk, wv, gate, up;
    bool split_qkv = false, split_gu = false;
    float* input_norm = nullptr;
    float* post_attn_norm = nullptr;
    // layer variants (LC/src/pipeline.rs:76-115): post-norm layers norm the attention and
    // FFN outputs before their residual adds and the FFN input with pre_ffn_norm (null
    // vectors: the weight-free norm)
    float* pre_ffn_norm = nullptr;
    float* post_ffn_norm = nullptr;
    float norm_offset = 0.f;
    float layer_scalar = 0.f;  // 0 = disabled
    bool post_norms = false, v_norm = false;
    int act = LARQL_ACT_SILU;
    double eps = 1e-6;
    float attn_scale = 0.f;
    double rope_base = 10000.0;
    int hd = 0, nq = 0, nkv = 0, rdim = 0, window = 0;
};

struct larql_hip_model {
    std::vector<LayerDev> layers;
    size_t hidden = 0, inter = 0;
    // the largest over the layers (each layer has its own head geometry,
    // LC/src/metal/decode.rs:101-110): q and kv widths, q|k|v width, attention partial
    // floats per position split
    size_t q_dim = 0, kv_dim = 0, qkv_dim = 0, part_per_split = 0;
    bool has_head = false;
    DevWeight head;
    float* final_norm = nullptr;
    double final_eps = 1e-6;
    float final_offset = 0.f;
    size_t vocab = 0;
    std::vector<void*> allocs;
    // workspace
    float *h0 = nullptr, *h1 = nullptr, *qkv = nullptr, *attn = nullptr, *act = nullptr, *xin = nullptr;
    float* gtmp = nullptr;  // gate projection when gate and up have different formats
    float* otmp = nullptr;  // post-norm layers: attention / FFN output before its norm
    float* utmp = nullptr;  // up projection of a Q8-input FFN
    float* xn = nullptr;    // normed input of a Q8-input projection
    // Normed input handed from an EPI_RESID projection to the next norm-fused one: x * (offset
    // + w) and the producer's per-workgroup sums of x^2 (Q4_K MFMA kernels on both sides)
    float* xw = nullptr;
    double* psum = nullptr;
    int8_t* q8 = nullptr;   // Q8 activation of a Q8-input projection (quantize_to_q8)
    float* q8s = nullptr;
    float* ones = nullptr;  // weight of the weight-free norm in a fused matvec prologue
    larql::DeviceBuf part;
    larql::DeviceBuf prompt;  // batched prompt pass: activations of all positions
    // host-pointer decode_token cache key
    std::vector<uint64_t> key;
};

namespace {

void* dev_alloc(larql_hip_model* m, size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) fail(LARQL_HIP_ERR_NOMEM, "hipMalloc failed in model build");
    m->allocs.push_back(p);
    return p;
}

struct Src {
    const void* data;
    size_t len;
    size_t rows;
    const float* scales = nullptr;  // Q8_0: f32 scales [rows][cols / 32]
};

// A pointer the caller declares to be device memory: an allocation the GPU addresses
// (device, managed or pinned host memory) holding `bytes` from p.  Checked on the host
// before any copy or kernel reads it, so a host address passed by mistake is an error,
// not a GPU page fault.
void require_device_range(const void* p, size_t bytes, const char* what) {
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();
        fail(LARQL_HIP_ERR_INVALID, std::string(what) + ": not a device address (weights_on_device is set)");
    }
    if (at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeManaged && at.type != hipMemoryTypeUnified &&
        !(at.type == hipMemoryTypeHost && at.devicePointer))
        fail(LARQL_HIP_ERR_INVALID, std::string(what) + ": not a device address (weights_on_device is set)");
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) == hipSuccess && base) {
        const auto b = reinterpret_cast<uintptr_t>(base), q = reinterpret_cast<uintptr_t>(p);
        if (q < b || q - b > size || bytes > size - (q - b))
            fail(LARQL_HIP_ERR_INVALID, std::string(what) + ": device buffer shorter than its shape");
    } else {
        (void)hipGetLastError();
    }
}

// One device weight from one or more reference-layout sources: concatenated by rows
// (stride 1) or interleaved (source i -> rows i, i+n, ...).
DevWeight build_weight(larql_hip_ctx* c, larql_hip_model* m, int format, size_t cols, const std::vector<Src>& srcs,
                       bool interleave, bool on_device) {
    const bool int_fmt = format == LARQL_Q8_0 || format == LARQL_Q4_0;
    if (format != LARQL_Q4_K && format != LARQL_Q6_K && format != LARQL_Q4_KF && !int_fmt)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "decode: projections must be Q4_K, Q4_KF, Q6_K, Q8_0 or Q4_0");
    if (cols % (int_fmt ? 32 : 256))
        fail(LARQL_HIP_ERR_INVALID, "decode: projection input width must be a multiple of the block size");
    if (int_fmt && interleave) fail(LARQL_HIP_ERR_UNSUPPORTED, "decode: interleaved Q8_0 / Q4_0 weights");
    // Q4_KF: 144-byte GGUF or 160-byte pre-baked blocks, told apart by length; the sources
    // of one fused weight must agree
    const int hf = format == LARQL_Q4_KF ? larql::q4kf_form_checked(srcs[0].len, srcs[0].rows, cols) : larql::kHdr148;
    size_t rows = 0;
    for (const Src& s : srcs) {
        if (!s.data) fail(LARQL_HIP_ERR_INVALID, "decode: null weight");
        if (format == LARQL_Q4_KF && larql::q4kf_form_checked(s.len, s.rows, cols) != hf)
            fail(LARQL_HIP_ERR_INVALID, "decode: fused Q4_KF projections mix the 144- and 160-byte layouts");
        if (s.len < s.rows * larql::ref_row_bytes(format, cols, hf))
            fail(LARQL_HIP_ERR_INVALID, "decode: weight buffer shorter than its shape");
        if (format == LARQL_Q8_0 && !s.scales) fail(LARQL_HIP_ERR_INVALID, "decode: Q8_0 weight without scales");
        if (interleave && s.rows != srcs[0].rows) fail(LARQL_HIP_ERR_INVALID, "decode: gate/up shapes differ");
        rows += s.rows;
    }
    DevWeight w;
    w.format = format;
    w.hf = hf;
    w.rows = rows;
    w.rows_pad = larql::pad_rows(rows);
    w.cols = cols;
    w.bytes = larql::dev_layout_bytes(format, w.rows_pad, cols, hf);
    w.base = dev_alloc(m, w.bytes);
    larql::dev_layout_carve(w);
    LARQL_HIP_CHECK(hipMemsetAsync(w.base, 0, w.bytes, c->stream));
    size_t row0 = 0;
    for (size_t i = 0; i < srcs.size(); i++) {
        const Src& s = srcs[i];
        const size_t nbytes = s.rows * larql::ref_row_bytes(format, cols, hf);
        const size_t sbytes = format == LARQL_Q8_0 ? s.rows * (cols / 32) * sizeof(float) : 0;
        const uint8_t* raw = static_cast<const uint8_t*>(s.data);
        const float* sc = s.scales;
        if (on_device) {
            require_device_range(s.data, nbytes, "decode: weight");
            if (sbytes) require_device_range(s.scales, sbytes, "decode: Q8_0 weight scales");
        } else {
            const size_t soff = (nbytes + 255) & ~size_t(255);
            uint8_t* stage = static_cast<uint8_t*>(larql::ensure(c, c->stage_raw, soff + sbytes));
            LARQL_HIP_CHECK(hipMemcpyAsync(stage, s.data, nbytes, hipMemcpyHostToDevice, c->stream));
            if (sbytes) {
                LARQL_HIP_CHECK(hipMemcpyAsync(stage + soff, s.scales, sbytes, hipMemcpyHostToDevice, c->stream));
                sc = reinterpret_cast<const float*>(stage + soff);
            }
            raw = stage;
        }
        if (interleave) larql::launch_repack(w, raw, sc, c->stream, s.rows, i, srcs.size());
        else larql::launch_repack(w, raw, sc, c->stream, s.rows, row0, 1);
        row0 += s.rows;
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));  // the staging buffer is reused
    }
    return w;
}

float* upload_vec(larql_hip_ctx* c, larql_hip_model* m, const float* v, size_t n, bool on_device) {
    if (!v) fail(LARQL_HIP_ERR_INVALID, "decode: null norm vector");
    if (on_device) require_device_range(v, n * sizeof(float), "decode: norm vector");
    float* d = static_cast<float*>(dev_alloc(m, n * sizeof(float)));
    LARQL_HIP_CHECK(hipMemcpyAsync(d, v, n * sizeof(float), on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                   c->stream));
    return d;
}

// The HIP decode step implements RMSNorm layers with a gated FFN (SiLU or GELU-tanh), with
// or without post-norms, norm weight offsets, V-norm and a layer scalar; LayerNorm, the
// ungated FFN and biases are reported as unsupported so callers fall back
// (LI/src/layer_graph/predict.rs:397-430).  Run on every call, whether or not the layers
// match a cached model.
void check_supported(const larql_pipeline_layer& L) {
    if (L.norm_type != LARQL_NORM_RMS) fail(LARQL_HIP_ERR_UNSUPPORTED, "decode: LayerNorm layers not supported");
    if (L.ffn_type != LARQL_FFN_GATED) fail(LARQL_HIP_ERR_UNSUPPORTED, "decode: non-gated FFN not supported");
    if (L.activation != LARQL_ACT_SILU && L.activation != LARQL_ACT_GELU_TANH)
        fail(LARQL_HIP_ERR_INVALID, "decode: unknown activation");
    if (L.input_norm_bias || L.post_attn_norm_bias || L.ffn_up_bias || L.ffn_down_bias)
        fail(LARQL_HIP_ERR_UNSUPPORTED, "decode: biases not supported");
    if (!std::isfinite(L.norm_offset) || !std::isfinite(L.layer_scalar))
        fail(LARQL_HIP_ERR_INVALID, "decode: non-finite norm offset or layer scalar");
}

larql_hip_model* build_model(larql_hip_ctx* c, const larql_pipeline_layer* layers, size_t n, size_t hidden,
                             size_t inter, bool on_device) {
    if (!layers || n == 0) fail(LARQL_HIP_ERR_INVALID, "decode: no layers");
    if (hidden == 0 || inter == 0) fail(LARQL_HIP_ERR_INVALID, "decode: zero hidden/inter");
    auto* m = new larql_hip_model();
    try {
        m->hidden = hidden;
        m->inter = inter;
        for (size_t l = 0; l < n; l++) {
            const larql_pipeline_layer& L = layers[l];
            check_supported(L);
            LayerDev d;
            d.hd = static_cast<int>(L.head_dim);
            d.nq = static_cast<int>(L.num_q_heads);
            d.nkv = static_cast<int>(L.num_kv_heads);
            if (d.hd <= 0 || d.nq <= 0 || d.nkv <= 0 || d.nq % d.nkv || d.hd % 8)
                fail(LARQL_HIP_ERR_INVALID, "decode: bad head geometry");
            if (!larql::attn_supported(d.nq / d.nkv, d.hd))
                fail(LARQL_HIP_ERR_UNSUPPORTED, "decode: attention takes head_dim a multiple of 32 up to 512 and "
                                                "1..8 query heads per kv head");
            d.rdim = L.rotary_dim ? static_cast<int>(L.rotary_dim) : d.hd;
            if (d.rdim > d.hd || d.rdim % 2) fail(LARQL_HIP_ERR_INVALID, "decode: bad rotary_dim");
            d.window = static_cast<int>(L.sliding_window);
            d.eps = L.eps > 0.f ? static_cast<double>(L.eps) : 1e-6;
            d.attn_scale = L.attn_scale != 0.f ? L.attn_scale : static_cast<float>(1.0 / std::sqrt(double(d.hd)));
            d.rope_base = L.rope_base;
            const size_t qd = static_cast<size_t>(d.nq) * d.hd, kvd = static_cast<size_t>(d.nkv) * d.hd;
            m->q_dim = std::max(m->q_dim, qd);
            m->kv_dim = std::max(m->kv_dim, kvd);
            m->qkv_dim = std::max(m->qkv_dim, qd + 2 * kvd);
            m->part_per_split = std::max(m->part_per_split, larql::attn_part_floats(d.nq, 1, d.hd));
            // one fused launch needs one format (and, for Q4_KF, one byte layout)
            auto form = [&](const larql_quant_weight& q, size_t r, size_t k) {
                return q.format * 4 + (q.format == LARQL_Q4_KF ? larql::q4kf_form(q.len, r, k) : 0);
            };
            d.split_qkv = form(L.wq, qd, hidden) != form(L.wk, kvd, hidden) ||
                          form(L.wq, qd, hidden) != form(L.wv, kvd, hidden);
            if (d.split_qkv) {
                d.wq = build_weight(c, m, L.wq.format, hidden, {{L.wq.data, L.wq.len, qd, L.wq.scales}}, false,
                                    on_device);
                d.wk = build_weight(c, m, L.wk.format, hidden, {{L.wk.data, L.wk.len, kvd, L.wk.scales}}, false,
                                    on_device);
                d.wv = build_weight(c, m, L.wv.format, hidden, {{L.wv.data, L.wv.len, kvd, L.wv.scales}}, false,
                                    on_device);
            } else {
                d.qkv = build_weight(c, m, L.wq.format, hidden,
                                     {{L.wq.data, L.wq.len, qd, L.wq.scales},
                                      {L.wk.data, L.wk.len, kvd, L.wk.scales},
                                      {L.wv.data, L.wv.len, kvd, L.wv.scales}},
                                     false, on_device);
            }
            d.wo = build_weight(c, m, L.wo.format, qd, {{L.wo.data, L.wo.len, hidden, L.wo.scales}}, false, on_device);
            // the Q8-input formats have no fused gate/up epilogue: their gate and up run apart
            d.split_gu = form(L.gate, inter, hidden) != form(L.up, inter, hidden) || L.gate.format == LARQL_Q8_0 ||
                         L.gate.format == LARQL_Q4_0;
            if (d.split_gu) {
                d.gate = build_weight(c, m, L.gate.format, hidden, {{L.gate.data, L.gate.len, inter, L.gate.scales}},
                                      false, on_device);
                d.up = build_weight(c, m, L.up.format, hidden, {{L.up.data, L.up.len, inter, L.up.scales}}, false,
                                    on_device);
            } else {
                d.gateup = build_weight(c, m, L.gate.format, hidden,
                                        {{L.gate.data, L.gate.len, inter}, {L.up.data, L.up.len, inter}}, true, on_device);
            }
            d.down = build_weight(c, m, L.down.format, inter, {{L.down.data, L.down.len, hidden, L.down.scales}}, false,
                                  on_device);
            d.input_norm = upload_vec(c, m, L.input_norm, hidden, on_device);
            d.post_attn_norm = upload_vec(c, m, L.post_attn_norm, hidden, on_device);
            d.norm_offset = L.norm_offset;
            d.layer_scalar = L.layer_scalar;
            d.post_norms = L.has_post_norms != 0;
            d.v_norm = L.has_v_norm != 0;
            d.act = L.activation;
            if (d.post_norms) {
                if (L.pre_ffn_norm) d.pre_ffn_norm = upload_vec(c, m, L.pre_ffn_norm, hidden, on_device);
                if (L.post_ffn_norm) d.post_ffn_norm = upload_vec(c, m, L.post_ffn_norm, hidden, on_device);
            }
            m->layers.push_back(d);
        }
        m->h0 = static_cast<float*>(dev_alloc(m, hidden * 4));
        m->h1 = static_cast<float*>(dev_alloc(m, hidden * 4));
        m->xin = static_cast<float*>(dev_alloc(m, hidden * 4));
        m->qkv = static_cast<float*>(dev_alloc(m, m->qkv_dim * 4));
        m->attn = static_cast<float*>(dev_alloc(m, m->q_dim * 4));
        m->act = static_cast<float*>(dev_alloc(m, inter * 4));
        m->gtmp = static_cast<float*>(dev_alloc(m, inter * 4));
        m->otmp = static_cast<float*>(dev_alloc(m, hidden * 4));
        m->utmp = static_cast<float*>(dev_alloc(m, inter * 4));
        m->xn = static_cast<float*>(dev_alloc(m, hidden * 4));
        m->xw = static_cast<float*>(dev_alloc(m, hidden * 4));
        m->psum = static_cast<double*>(dev_alloc(m, (hidden / 16 + 64) * sizeof(double)));
        const size_t widest = std::max({hidden, inter, m->q_dim});
        m->q8 = static_cast<int8_t*>(dev_alloc(m, widest));
        m->q8s = static_cast<float*>(dev_alloc(m, widest / 32 * 4 + 4));
        {
            std::vector<float> one(hidden, 1.0f);
            m->ones = static_cast<float*>(dev_alloc(m, hidden * 4));
            LARQL_HIP_CHECK(hipMemcpy(m->ones, one.data(), hidden * 4, hipMemcpyHostToDevice));
        }
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
    } catch (...) {
        for (void* p : m->allocs) (void)hipFree(p);
        delete m;
        throw;
    }
    return m;
}

void destroy_model(larql_hip_ctx* c, larql_hip_model* m) {
    if (!m) return;
    (void)hipDeviceSynchronize();
    for (void* p : m->allocs) (void)hipFree(p);
    if (m->part.p) (void)hipFree(m->part.p);
    if (m->prompt.p) (void)hipFree(m->prompt.p);
    (void)c;
    delete m;
}

// ── KV cache ───────────────────────────────────────────────────────────
void kv_free_cache(larql::KVCache& kv) {
    (void)hipDeviceSynchronize();
    for (auto* p : kv.k) (void)hipFree(p);
    for (auto* p : kv.v) (void)hipFree(p);
    for (auto& r : kv.rope) (void)hipFree(r.cs);
    kv = larql::KVCache{};
}

void kv_free(larql_hip_ctx* c) { kv_free_cache(c->kv); }

// RoPE cos/sin table for (base, rdim) covering the cache capacity; built once per
// capacity (the cache only grows), on stream s, which is then synchronised so the
// table may be used from any stream afterwards.
const float2* rope_table(larql_hip_ctx* c, double base, int rdim, hipStream_t s) {
    auto& kv = c->kv;
    for (auto& r : kv.rope)
        if (r.base == base && r.rdim == rdim && r.cap >= kv.max_seq) return r.cs;
    larql::RopeTable t;
    t.base = base;
    t.rdim = rdim;
    t.cap = kv.max_seq;
    const size_t bytes = t.cap * static_cast<size_t>(rdim / 2) * sizeof(float2);
    if (hipMalloc(&t.cs, bytes ? bytes : 1) != hipSuccess) fail(LARQL_HIP_ERR_NOMEM, "RoPE table allocation failed");
    larql::launch_rope_table(t.cs, t.cap, rdim, base, s);
    LARQL_HIP_CHECK(hipStreamSynchronize(s));
    for (auto it = kv.rope.begin(); it != kv.rope.end(); ++it)
        if (it->base == base && it->rdim == rdim) {
            (void)hipFree(it->cs);
            kv.rope.erase(it);
            break;
        }
    kv.rope.push_back(t);
    return t.cs;
}

// Capacity >= need positions for every layer held (initial capacity 4096 as in the
// reference, LC/src/metal/trait_impl.rs:163; doubled on demand, so attention is not
// limited in T); growth copies the rows in use.
void kv_reserve(larql_hip_ctx* c, size_t need) {
    auto& kv = c->kv;
    if (kv.num_layers == 0 && kv.max_seq == 0) {
        kv.max_seq = need > 4096 ? (need + 7) & ~size_t(7) : 4096;  // V blocks of 8 positions
        kv.current_len = 0;
    }
    if (need <= kv.max_seq) return;
    size_t cap = kv.max_seq * 2;
    while (cap < need) cap *= 2;
    (void)hipDeviceSynchronize();
    for (size_t l = 0; l < kv.num_layers; l++) {
        const size_t row = kv.num_kv[l] * kv.head_dim[l];
        for (auto* vec : {&kv.k, &kv.v}) {
            __half* p = nullptr;
            if (hipMalloc(&p, cap * row * sizeof(__half)) != hipSuccess) fail(LARQL_HIP_ERR_NOMEM, "KV grow failed");
            // V blocks hold 8 positions: copy whole blocks (K rows up to the same bound)
            const size_t len8 = (kv.current_len + 7) & ~size_t(7);
            LARQL_HIP_CHECK(hipMemcpy(p, (*vec)[l], len8 * row * sizeof(__half), hipMemcpyDeviceToDevice));
            (void)hipFree((*vec)[l]);
            (*vec)[l] = p;
        }
    }
    kv.max_seq = cap;
}

// Layer l held with geometry [cap][num_kv][head_dim]: layers below it that are missing
// are made with the same geometry; a layer held with another geometry is made again (its
// rows dropped).  Returns whether a held layer was made again.
bool kv_layer(larql_hip_ctx* c, size_t l, size_t num_kv, size_t head_dim) {
    auto& kv = c->kv;
    const size_t row = num_kv * head_dim;
    auto make = [&](__half*& k, __half*& v) {
        if (hipMalloc(&k, kv.max_seq * row * sizeof(__half)) != hipSuccess ||
            hipMalloc(&v, kv.max_seq * row * sizeof(__half)) != hipSuccess) {
            if (k) (void)hipFree(k);
            k = v = nullptr;
            fail(LARQL_HIP_ERR_NOMEM, "KV cache allocation failed");
        }
    };
    bool remade = false;
    if (l < kv.num_layers && (kv.num_kv[l] != num_kv || kv.head_dim[l] != head_dim)) {
        (void)hipDeviceSynchronize();
        (void)hipFree(kv.k[l]);
        (void)hipFree(kv.v[l]);
        kv.k[l] = kv.v[l] = nullptr;
        make(kv.k[l], kv.v[l]);
        kv.num_kv[l] = num_kv;
        kv.head_dim[l] = head_dim;
        remade = true;
    }
    while (kv.num_layers <= l) {
        __half *k = nullptr, *v = nullptr;
        make(k, v);
        kv.k.push_back(k);
        kv.v.push_back(v);
        kv.num_kv.push_back(num_kv);
        kv.head_dim.push_back(head_dim);
        kv.num_layers++;
    }
    return remade;
}

// populate_kv_layer: layer `layer` (and any missing below it) with this geometry.
void kv_ensure_layer(larql_hip_ctx* c, size_t layer, size_t num_kv, size_t head_dim, size_t need) {
    kv_reserve(c, need);
    kv_layer(c, layer, num_kv, head_dim);
}

// A model's layers with their own geometries and room for `need` positions; when a held
// layer's geometry differs (another model), its rows are gone and the cache restarts at
// length 0.
void kv_ensure_model(larql_hip_ctx* c, const larql_hip_model* m, size_t need) {
    kv_reserve(c, need);
    bool remade = false;
    for (size_t l = 0; l < m->layers.size(); l++)
        remade |= kv_layer(c, l, static_cast<size_t>(m->layers[l].nkv), static_cast<size_t>(m->layers[l].hd));
    if (remade) c->kv.current_len = 0;
}

// Formats whose kernels take a Q8 activation (quantize_to_q8 of the f32 input): Q8_0, and
// Q4_0 except as the down projection, which takes the f32 activation
// (LC/src/metal/decode.rs:262-296, 374-404, 560-690).
bool takes_q8(const DevWeight& w, bool is_down) {
    return w.format == LARQL_Q8_0 || (w.format == LARQL_Q4_0 && !is_down);
}

// The model's Q8 activation: quantize_to_q8 of x[n], or of its norm when norm_w is given.
void quantize_input(larql_hip_model* m, const float* x, size_t n, const float* norm_w, float off, double eps,
                    hipStream_t s) {
    const float* src = x;
    if (norm_w) {
        larql::launch_rmsnorm_rows(x, norm_w, off, m->xn, 1, n, eps, s);
        src = m->xn;
    }
    larql::launch_quantize_q8(src, n, 1, m->q8, m->q8s, s);
}

// Weights whose m = 1 matvec is the Q4_K MFMA kernel (the producer / consumer epilogues).
bool q4k_mfma(const DevWeight& w) { return w.format == LARQL_Q4_K || w.format == LARQL_Q4_KF; }
// A Q4_K MFMA consumer able to take n producer partial sums.
bool takes_psum(const DevWeight& w, int n) { return q4k_mfma(w) && n <= larql::q4k_mfma_max_psum(w, 0); }

// out = W . (the model's Q8 activation), blocks accumulated in order (bit-exact int dots).
void int_proj(const DevWeight& w, larql_hip_model* m, float* out, hipStream_t s) {
    if (w.format == LARQL_Q8_0) larql::launch_q8_matvec(w, m->q8, m->q8s, out, 1, s);
    else larql::launch_q4_0_matvec(w, m->q8, m->q8s, out, 1, s);
}

// Prompt-attention options of prefill_q4 / full_pipeline_q4 (use_qk_norm, softcap); a
// decode step takes neither (zero).
struct PromptAttn {
    int qk_norm = 0;
    float softcap = 0.f;
};

// The layer launches of one decode step at T = pos + 1, x0 -> h0 (layer 0 reads its
// input from x0, which the step does not write; later layers read h0).
void enqueue_layers(larql_hip_ctx* c, larql_hip_model* m, const float* x0, int T, float* part, hipStream_t s,
                    const PromptAttn& pa = {}) {
    auto& kv = c->kv;
    // prenormed: m->xw / m->psum hold this layer's normed Q/K/V input (from the previous
    // layer's down projection), npsum partial sums
    bool prenormed = false;
    int npsum = 0;
    for (size_t l = 0; l < m->layers.size(); l++) {
        const LayerDev& L = m->layers[l];
        const float* hin = l == 0 ? x0 : m->h0;
        const size_t qd = static_cast<size_t>(L.nq) * L.hd, kvd = static_cast<size_t>(L.nkv) * L.hd;
        // Q/K/V: f32-input formats with the input norm fused into the matvec; Q8_0 from the
        // quantized normed input (one quantization shared by the three)
        bool have_q8 = false;
        auto qkv_proj = [&](const DevWeight& w, float* out) {
            if (takes_q8(w, false)) {
                if (!have_q8) quantize_input(m, hin, m->hidden, L.input_norm, L.norm_offset, L.eps, s);
                have_q8 = true;
                int_proj(w, m, out, s);
            } else {
                larql::MvArgs a;
                a.x = hin;
                a.out = out;
                a.eps = L.eps;
                if (prenormed) {
                    a.x = m->xw;
                    a.x_psum = m->psum;
                    a.x_npsum = npsum;
                } else {
                    a.norm_w = L.input_norm;
                    a.norm_offset = L.norm_offset;
                }
                larql::launch_mv(w, a, s);
            }
        };
        if (L.split_qkv) {  // three launches into the [q | k | v] buffer
            qkv_proj(L.wq, m->qkv);
            qkv_proj(L.wk, m->qkv + qd);
            qkv_proj(L.wv, m->qkv + qd + kvd);
        } else {
            qkv_proj(L.qkv, m->qkv);
        }
        if (L.v_norm) larql::launch_vnorm_rows(m->qkv + qd + kvd, 1, 0, L.nkv, L.hd, L.eps, s);

        larql::AttnArgs at{};
        at.qkv = m->qkv;
        at.kc = kv.k[l];
        at.vc = kv.v[l];
        at.out = m->attn;
        at.part = part;
        at.num_q = L.nq;
        at.num_kv = L.nkv;
        at.hd = L.hd;
        at.rdim = L.rdim;
        at.T = T;
        at.t_begin = (L.window > 0 && T > L.window) ? T - L.window : 0;
        at.scale = L.attn_scale;
        at.rope = rope_table(c, L.rope_base, L.rdim, s);
        at.qk_norm = pa.qk_norm;
        at.softcap = pa.softcap;
        larql::launch_attention(at, s);

        // h1 = h + o (Llama), or h + norm(o, post_attn_norm) for post-norm layers
        const bool o_q8 = takes_q8(L.wo, false);
        if (L.post_norms || o_q8) {
            if (o_q8) {
                quantize_input(m, m->attn, qd, nullptr, 0.f, L.eps, s);
                int_proj(L.wo, m, m->otmp, s);
            } else {
                larql::MvArgs o;
                o.x = m->attn;
                o.out = m->otmp;
                larql::launch_mv(L.wo, o, s);
            }
            if (L.post_norms)
                larql::launch_resid_norm_rows(hin, m->otmp, L.post_attn_norm, L.norm_offset, 1.0f, m->h1, 1,
                                              m->hidden, L.eps, s);
            else
                larql::launch_add_rows(hin, m->otmp, m->h1, m->hidden, s);
        }

        // FFN input norm: post_attn_norm, or pre_ffn_norm (weight-free when absent) for
        // post-norm layers
        const float* fnorm = L.post_attn_norm;
        float foff = L.norm_offset;
        if (L.post_norms) {
            fnorm = L.pre_ffn_norm ? L.pre_ffn_norm : m->ones;
            foff = L.pre_ffn_norm ? L.norm_offset : 0.0f;
        }
        const bool g_q8 = !L.split_gu ? false : takes_q8(L.gate, false), u_q8 = !L.split_gu ? false : takes_q8(L.up, false);
        // Llama O projection: h1 = h + Wo attn; it also hands the FFN its normed input when
        // both sides run the Q4_K MFMA kernel
        const int o_groups = q4k_mfma(L.wo) ? larql::q4k_mfma_groups(L.wo, 0) : 0;
        const bool ffn_prenormed = !(L.post_norms || o_q8) && q4k_mfma(L.wo) &&
                                   (L.split_gu ? !g_q8 && !u_q8 && takes_psum(L.gate, o_groups) &&
                                                     takes_psum(L.up, o_groups)
                                               : takes_psum(L.gateup, o_groups));
        if (!(L.post_norms || o_q8)) {
            larql::MvArgs o;
            o.x = m->attn;
            o.out = m->h1;
            o.epi = larql::EPI_RESID;
            o.resid = hin;
            if (ffn_prenormed) {
                o.out2 = m->xw;
                o.out2_w = fnorm;
                o.out2_off = foff;
                o.psum = m->psum;
            }
            larql::launch_mv(L.wo, o, s);
        }
        larql::MvArgs g;
        g.x = m->h1;
        g.out = m->act;
        g.act = L.act;
        g.eps = L.eps;
        if (ffn_prenormed) {
            g.x = m->xw;
            g.x_psum = m->psum;
            g.x_npsum = o_groups;
        } else {
            g.norm_w = fnorm;
            g.norm_offset = foff;
        }
        if (g_q8 || u_q8) {  // gate and up apart, then act(gate) * up
            quantize_input(m, m->h1, m->hidden, fnorm, foff, L.eps, s);
            float* outs[2] = {m->gtmp, m->utmp};
            const DevWeight* ws[2] = {&L.gate, &L.up};
            for (int i = 0; i < 2; i++) {
                if (takes_q8(*ws[i], false)) {
                    int_proj(*ws[i], m, outs[i], s);
                } else {
                    larql::MvArgs gi = g;
                    gi.out = outs[i];
                    gi.epi = larql::EPI_STORE;
                    larql::launch_mv(*ws[i], gi, s);
                }
            }
            larql::launch_gated_mul(m->gtmp, m->utmp, m->act, m->inter, L.act, s);
        } else if (L.split_gu) {  // gate, then up with act(gate) * up in its epilogue
            g.out = m->gtmp;
            larql::launch_mv(L.gate, g, s);
            g.out = m->act;
            g.epi = larql::EPI_GATED_MUL;
            g.resid = m->gtmp;
            larql::launch_mv(L.up, g, s);
        } else {
            g.epi = larql::EPI_GATED_PAIR;
            larql::launch_mv(L.gateup, g, s);
        }

        // h2 = (h1 + down) or (h1 + norm(down, post_ffn_norm)), times the layer scalar
        const float scale = L.layer_scalar != 0.0f ? L.layer_scalar : 1.0f;
        const bool d_int = L.down.format == LARQL_Q4_0 || L.down.format == LARQL_Q8_0;
        if (L.post_norms || d_int) {
            if (L.down.format == LARQL_Q4_0) {  // f32 activation (the reference's q4_f32_matvec)
                larql::launch_q4_0_f32_matvec(L.down, m->act, m->otmp, s);
            } else if (L.down.format == LARQL_Q8_0) {
                quantize_input(m, m->act, m->inter, nullptr, 0.f, L.eps, s);
                int_proj(L.down, m, m->otmp, s);
            } else {
                larql::MvArgs d;
                d.x = m->act;
                d.out = m->otmp;
                larql::launch_mv(L.down, d, s);
            }
            if (L.post_norms)
                larql::launch_resid_norm_rows(m->h1, m->otmp, L.post_ffn_norm, L.post_ffn_norm ? L.norm_offset : 0.0f,
                                              scale, m->h0, 1, m->hidden, L.eps, s);
            else
                larql::launch_add_rows(m->h1, m->otmp, m->h0, m->hidden, s, scale);
        } else {
            larql::MvArgs d;
            d.x = m->act;
            d.out = m->h0;
            d.epi = larql::EPI_RESID;
            d.resid = m->h1;
            d.out_scale = scale;
            // the next layer's normed Q/K/V input, when both sides run the Q4_K MFMA kernel
            const LayerDev* Ln = l + 1 < m->layers.size() ? &m->layers[l + 1] : nullptr;
            const int d_groups = q4k_mfma(L.down) ? larql::q4k_mfma_groups(L.down, 0) : 0;
            prenormed = Ln && q4k_mfma(L.down) &&
                        (Ln->split_qkv ? takes_psum(Ln->wq, d_groups) && takes_psum(Ln->wk, d_groups) &&
                                             takes_psum(Ln->wv, d_groups)
                                       : takes_psum(Ln->qkv, d_groups));
            if (prenormed) {
                d.out2 = m->xw;
                d.out2_w = Ln->input_norm;
                d.out2_off = Ln->norm_offset;
                d.psum = m->psum;
                npsum = d_groups;
            }
            larql::launch_mv(L.down, d, s);
            continue;
        }
        prenormed = false;
    }
}

void run_decode(larql_hip_ctx* c, larql_hip_model* m, const float* x_dev, float* hidden_out, float* logits,
                hipStream_t s, const PromptAttn& pa = {}) {
    auto& kv = c->kv;
    kv_ensure_model(c, m, kv.current_len + 1);
    const int T = static_cast<int>(kv.current_len) + 1;
    // partials for any T up to the cache capacity: the buffer grows only with the cache, so
    // a step inside the capacity allocates nothing
    const int S_cap = larql::attn_splits(static_cast<int>(kv.max_seq), 0);
    float* part = static_cast<float*>(larql::ensure(c, m->part, m->part_per_split * S_cap * sizeof(float)));
    if (m->layers.empty()) larql::launch_copy_f32(x_dev, m->h0, m->hidden, s);
    else enqueue_layers(c, m, x_dev, T, part, s, pa);
    kv.current_len = static_cast<size_t>(T);
    if (hidden_out) larql::launch_copy_f32(m->h0, hidden_out, m->hidden, s);
    if (logits) {
        if (!m->has_head) fail(LARQL_HIP_ERR_STATE, "decode: logits requested but the model has no head");
        larql::MvArgs e;
        e.x = m->h0;
        e.out = logits;
        e.norm_w = m->final_norm;
        e.norm_offset = m->final_offset;
        e.eps = m->final_eps;
        larql::launch_mv(m->head, e, s);
    }
}

uint64_t f32_bits(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return b;
}

// Cache key of a trait-call model: every field of every layer that build_model reads
// (weights and norm vectors by pointer, length and sampled content; the scalars by value).
std::vector<uint64_t> layers_key(const larql_pipeline_layer* layers, size_t n, size_t hidden, size_t inter) {
    std::vector<uint64_t> k{n, hidden, inter};
    auto vec = [&](const float* v) {
        k.push_back(reinterpret_cast<uint64_t>(v));
        k.push_back(v ? larql::host_fingerprint(v, hidden * 4) : 0);
    };
    for (size_t l = 0; l < n; l++) {
        const larql_pipeline_layer& L = layers[l];
        for (const larql_quant_weight* w : {&L.wq, &L.wk, &L.wv, &L.wo, &L.gate, &L.up, &L.down}) {
            k.push_back(reinterpret_cast<uint64_t>(w->data));
            k.push_back(w->len);
            k.push_back(static_cast<uint64_t>(w->format));
            k.push_back(w->data ? larql::host_fingerprint(w->data, w->len) : 0);
        }
        vec(L.input_norm);
        vec(L.post_attn_norm);
        vec(L.has_post_norms ? L.pre_ffn_norm : nullptr);
        vec(L.has_post_norms ? L.post_ffn_norm : nullptr);
        k.push_back((f32_bits(L.eps) << 32) | f32_bits(L.rope_base));
        k.push_back((f32_bits(L.attn_scale) << 32) | f32_bits(L.norm_offset));
        k.push_back((f32_bits(L.layer_scalar) << 32) | (static_cast<uint64_t>(L.activation & 0xFF) << 16) |
                    (static_cast<uint64_t>(L.has_post_norms != 0) << 8) | static_cast<uint64_t>(L.has_v_norm != 0));
        k.push_back((static_cast<uint64_t>(L.head_dim) << 32) | (L.num_q_heads << 16) | L.num_kv_heads);
        k.push_back((static_cast<uint64_t>(L.rotary_dim) << 32) | L.sliding_window);
    }
    return k;
}

// The trait calls' model: rebuilt when the layers' key differs from the cached one.
larql_hip_model* trait_model_for(larql_hip_ctx* c, const larql_pipeline_layer* layers, size_t n, size_t hidden,
                                 size_t inter) {
    if (!layers || n == 0) fail(LARQL_HIP_ERR_INVALID, "decode: no layers");
    for (size_t l = 0; l < n; l++) check_supported(layers[l]);
    auto key = layers_key(layers, n, hidden, inter);
    larql_hip_model*& m = c->trait_model;
    if (!m || m->key != key) {
        destroy_model(c, m);
        m = nullptr;
        m = build_model(c, layers, n, hidden, inter, false);
        m->key = key;
    }
    return m;
}

// q_dim / kv_dim of a trait call: the widest layer's, the width the reference sizes its
// per-token buffers by (LC/src/metal/decode.rs:72-76); for uniform layers, every layer's.
void check_dims(const larql_hip_model* m, size_t q_dim, size_t kv_dim, const char* what) {
    if (m->q_dim != q_dim || m->kv_dim != kv_dim)
        fail(LARQL_HIP_ERR_INVALID, std::string(what) + ": q_dim/kv_dim differ from the widest layer's");
}

}  // namespace

extern "C" int larql_hip_decode_token(larql_hip_ctx* c, const larql_pipeline_layer* layers, size_t num_layers,
                                      const float* x, size_t hidden, size_t inter, size_t q_dim, size_t kv_dim,
                                      size_t num_q_heads, size_t num_kv_heads, size_t head_dim, float rope_base,
                                      float* out) {
    return guarded(c, [&] {
        if (!layers || !x || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        // per-layer rope_base and head geometry are authoritative (FullPipelineLayer.rope_base,
        // head_dim, num_q_heads, num_kv_heads; LC/src/metal/decode.rs:101-110)
        (void)rope_base, (void)num_q_heads, (void)num_kv_heads, (void)head_dim;
        larql_hip_model* m = trait_model_for(c, layers, num_layers, hidden, inter);
        check_dims(m, q_dim, kv_dim, "decode_token");
        LARQL_HIP_CHECK(hipMemcpyAsync(m->xin, x, hidden * sizeof(float), hipMemcpyHostToDevice, c->stream));
        run_decode(c, m, m->xin, m->xin, nullptr, c->stream);
        download(c, out, m->xin, hidden * sizeof(float));
    });
}

// The batched prompt pass takes layers with gate/up fused in Q4_K and every other
// projection Q4_K or Q6_K (Q4_K and Q4_K_M files); others run position by position.
static bool prompt_batchable(const larql_hip_model* m) {
    auto ok = [](const larql::DevWeight& w) { return w.format == LARQL_Q4_K || w.format == LARQL_Q6_K; };
    for (const LayerDev& L : m->layers) {
        if (L.split_gu || L.gateup.format != LARQL_Q4_K || !ok(L.wo) || !ok(L.down)) return false;
        if (L.split_qkv ? !(ok(L.wq) && ok(L.wk) && ok(L.wv)) : !ok(L.qkv)) return false;
    }
    return true;
}

// One projection of all M positions (X rows ldx = w.cols apart) -> Y rows ldy apart: the
// f32-accuracy GEMM, Q4_K or Q6_K.
static void prompt_proj(const larql::DevWeight& w, const float* X, size_t ldx, float* Y, size_t ldy, size_t M,
                        float* spl, size_t split_n, hipStream_t s, const larql::GemmRowStats* pre = nullptr,
                        larql::GemmSplits* defer = nullptr) {
    if (ldx != w.cols) fail(LARQL_HIP_ERR_INVALID, "prompt pass: input rows do not match the weight");
    larql::launch_q4k_gemm_f32(w, X, Y, M, spl, split_n, s, ldy, pre, defer);
}

static void run_prompt(larql_hip_ctx* c, larql_hip_model* m, const float* dx, size_t M, float* dout, hipStream_t s,
                       const PromptAttn& pa = {}) {
    auto& kv = c->kv;
    kv_ensure_model(c, m, M);
    const size_t hidden = m->hidden, inter = m->inter, qmax = m->q_dim, ldmax = m->qkv_dim;
    const size_t wide = std::max({hidden, qmax, inter}), gw = std::max(hidden, 2 * inter);
    const int S = larql::attn_prompt_splits(1, static_cast<int>(M), 0);
    const size_t part_n = m->part_per_split * S * M;
    size_t split_n = 0;  // GEMM workspace: row exponents and K-split partial products
    auto need = [&](const larql::DevWeight& w) {
        split_n = std::max(split_n, larql::q4k_gemm_f32_part_floats(w, M));
    };
    for (const LayerDev& L : m->layers) {
        if (L.split_qkv) need(L.wq), need(L.wk), need(L.wv);
        else need(L.qkv);
        need(L.wo), need(L.gateup), need(L.down);
    }
    // row statistics of the normed hidden rows and of the activation rows, computed by the
    // kernels that produce those rows (two separate regions: a producer may still read
    // the previous GEMM's partial products in SPL)
    const size_t st_h = larql::gemm_row_stats_floats(M, hidden), st_a = larql::gemm_row_stats_floats(M, inter);
    const size_t n_f = 2 * M * hidden + M * wide + M * ldmax + M * qmax + M * gw + M * inter + part_n + split_n +
                       st_h + st_a + 8;
    float* base = static_cast<float*>(larql::ensure(c, m->prompt, n_f * sizeof(float)));
    float *H0 = base, *H1 = H0 + M * hidden, *XN = H1 + M * hidden, *QKV = XN + M * wide, *ATT = QKV + M * ldmax;
    float *G = ATT + M * qmax, *ACT = G + M * gw, *PART = ACT + M * inter, *SPL = PART + part_n;
    const larql::GemmRowStats xn_st = larql::gemm_row_stats_at(SPL + split_n, M, hidden);
    const larql::GemmRowStats act_st = larql::gemm_row_stats_at(SPL + split_n + st_h + 4, M, inter);
    larql::launch_copy_f32(dx, H0, M * hidden, s);
    bool xn_ready = false;  // XN holds this layer's normed input and xn_st its statistics
    for (size_t l = 0; l < m->layers.size(); l++) {
        const LayerDev& L = m->layers[l];
        // this layer's [q | k | v] rows, ld floats apart, and attention rows qd apart
        const size_t qd = static_cast<size_t>(L.nq) * L.hd, kvd = static_cast<size_t>(L.nkv) * L.hd, ld = qd + 2 * kvd;
        if (!xn_ready) {
            larql::launch_rmsnorm_rows(H0, L.input_norm, L.norm_offset, XN, M, hidden, L.eps, s);
            larql::launch_gemm_row_stats(XN, M, hidden, xn_st, s);
        }
        xn_ready = false;
        if (L.split_qkv) {  // Q, K, V into their column ranges of the [q | k | v] rows
            prompt_proj(L.wq, XN, hidden, QKV, ld, M, SPL, split_n, s, &xn_st);
            prompt_proj(L.wk, XN, hidden, QKV + qd, ld, M, SPL, split_n, s, &xn_st);
            prompt_proj(L.wv, XN, hidden, QKV + qd + kvd, ld, M, SPL, split_n, s, &xn_st);
        } else {
            prompt_proj(L.qkv, XN, hidden, QKV, ld, M, SPL, split_n, s, &xn_st);
        }
        if (L.v_norm) larql::launch_vnorm_rows(QKV + qd + kvd, M, ld, L.nkv, L.hd, L.eps, s);
        const float2* rope = rope_table(c, L.rope_base, L.rdim, s);
        larql::launch_rope_kv_rows(QKV, M, 0, qd, kvd, L.hd, L.rdim, rope, kv.k[l], kv.v[l], L.nkv, s);
        larql::AttnArgs at{};
        at.qkv = QKV;
        at.kc = kv.k[l];
        at.vc = kv.v[l];
        at.out = ATT;
        at.part = PART;
        at.num_q = L.nq;
        at.num_kv = L.nkv;
        at.hd = L.hd;
        at.rdim = L.rdim;
        at.T = 1;  // query p has T = 1 + p
        at.scale = L.attn_scale;
        at.rope = rope;
        at.batch = static_cast<int>(M);
        at.window = L.window;
        at.qkv_ld = static_cast<int>(ld);
        at.qk_norm = pa.qk_norm;
        at.softcap = pa.softcap;
        larql::launch_attention(at, s);
        const float scale = L.layer_scalar != 0.0f ? L.layer_scalar : 1.0f;
        if (L.post_norms || hidden > larql::kFusedRowMax || inter > larql::kFusedRowMax) {
            prompt_proj(L.wo, ATT, qd, G, hidden, M, SPL, split_n, s);
            larql::launch_resid_norm_rows(H0, G, L.post_attn_norm, L.norm_offset, 1.0f, H1, M, hidden, L.eps, s);
            larql::launch_rmsnorm_rows(H1, L.pre_ffn_norm, L.norm_offset, XN, M, hidden, L.eps, s);
            prompt_proj(L.gateup, XN, hidden, G, 2 * inter, M, SPL, split_n, s);
            larql::launch_gated_pair_rows(G, ACT, M * inter, L.act, s);
            prompt_proj(L.down, ACT, inter, G, hidden, M, SPL, split_n, s);
            larql::launch_resid_norm_rows(H1, G, L.post_ffn_norm, L.norm_offset, scale, H0, M, hidden, L.eps, s);
            continue;
        }
        // the split sums of wo and down, the residual adds, the next norm and the row
        // statistics of the next GEMM's input: one row kernel after each projection
        larql::GemmSplits sp{};
        prompt_proj(L.wo, ATT, qd, G, hidden, M, SPL, split_n, s, nullptr, &sp);
        larql::launch_resid_norm_stats_rows(sp.splits > 1 ? sp.part : G, M * hidden, sp.splits, H0, 1.0f, H1,
                                            L.post_attn_norm, L.norm_offset, XN, M, hidden, L.eps, xn_st, s);
        prompt_proj(L.gateup, XN, hidden, G, 2 * inter, M, SPL, split_n, s, &xn_st);
        larql::launch_gated_pair_stats_rows(G, ACT, M, inter, L.act, act_st, s);
        prompt_proj(L.down, ACT, inter, G, hidden, M, SPL, split_n, s, &act_st, &sp);
        const LayerDev* nx = l + 1 < m->layers.size() ? &m->layers[l + 1] : nullptr;
        larql::launch_resid_norm_stats_rows(sp.splits > 1 ? sp.part : G, M * hidden, sp.splits, H1, scale, H0,
                                            nx ? nx->input_norm : nullptr, nx ? nx->norm_offset : 0.0f,
                                            nx ? XN : nullptr, M, hidden, nx ? nx->eps : 0.0, xn_st, s);
        xn_ready = nx != nullptr;
    }
    larql::launch_copy_f32(H0, dout, M * hidden, s);
    kv.current_len = M;
}

extern "C" int larql_hip_prefill_q4(larql_hip_ctx* c, const larql_pipeline_layer* layers, size_t num_layers,
                                    const float* x, size_t hidden, size_t inter, size_t q_dim, size_t kv_dim,
                                    size_t seq_len, size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                                    float rope_base, int use_qk_norm, float softcap, float* out) {
    return guarded(c, [&] {
        if (!layers || !x || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        // per-layer rope_base and head geometry are authoritative (FullPipelineLayer.rope_base,
        // head_dim, num_q_heads, num_kv_heads; LC/src/metal/decode.rs:101-110)
        (void)rope_base, (void)num_q_heads, (void)num_kv_heads, (void)head_dim;
        if (seq_len == 0) return;
        larql_hip_model* m = trait_model_for(c, layers, num_layers, hidden, inter);
        check_dims(m, q_dim, kv_dim, "prefill");
        kv_ensure_model(c, m, seq_len);
        c->kv.current_len = 0;  // a new prompt at positions 0 .. seq_len - 1
        const float* dx = stage_upload(c, c->stage_in, x, seq_len * hidden);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, seq_len * hidden * sizeof(float)));
        const PromptAttn pa{use_qk_norm != 0, softcap};
        if (seq_len > 1 && prompt_batchable(m))
            run_prompt(c, m, dx, seq_len, dout, c->stream, pa);
        else
            for (size_t p = 0; p < seq_len; p++)
                run_decode(c, m, dx + p * hidden, dout + p * hidden, nullptr, c->stream, pa);
        download(c, out, dout, seq_len * hidden * sizeof(float));
    });
}

extern "C" int larql_hip_full_pipeline_q4(larql_hip_ctx* c, const larql_pipeline_layer* layers, size_t num_layers,
                                          const float* x, size_t hidden, size_t inter, size_t q_dim, size_t kv_dim,
                                          size_t seq_len, size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                                          float rope_base, int use_qk_norm, float softcap, float* out) {
    return guarded(c, [&] {
        if (!layers || !x || !out) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        // per-layer rope_base and head geometry are authoritative (FullPipelineLayer.rope_base,
        // head_dim, num_q_heads, num_kv_heads; LC/src/metal/decode.rs:101-110)
        (void)rope_base, (void)num_q_heads, (void)num_kv_heads, (void)head_dim;
        if (seq_len == 0) return;
        larql_hip_model* m = trait_model_for(c, layers, num_layers, hidden, inter);
        check_dims(m, q_dim, kv_dim, "full pipeline");
        // positions 0 .. seq_len - 1 with causal attention over each other only: run against
        // the set-aside cache, then restore the decode cache whatever happens
        std::swap(c->kv, c->kv_aside);
        struct Restore {
            larql_hip_ctx* c;
            ~Restore() { std::swap(c->kv, c->kv_aside); }
        } restore{c};
        kv_ensure_model(c, m, seq_len);
        c->kv.current_len = 0;
        const float* dx = stage_upload(c, c->stage_in, x, seq_len * hidden);
        float* dout = static_cast<float*>(larql::ensure(c, c->stage_out, seq_len * hidden * sizeof(float)));
        const PromptAttn pa{use_qk_norm != 0, softcap};
        if (seq_len > 1 && prompt_batchable(m))
            run_prompt(c, m, dx, seq_len, dout, c->stream, pa);
        else
            for (size_t p = 0; p < seq_len; p++)
                run_decode(c, m, dx + p * hidden, dout + p * hidden, nullptr, c->stream, pa);
        download(c, out, dout, seq_len * hidden * sizeof(float));
    });
}

extern "C" int larql_hip_multi_layer_q4_ffn(larql_hip_ctx* c, const larql_q4_ffn_layer* layers, size_t num_layers,
                                           const float* x, size_t inter, size_t hidden, float* out) {
    return guarded(c, [&] {
        if (!layers || !x || !out || num_layers == 0) fail(LARQL_HIP_ERR_INVALID, "null pointer or no layers");
        if (hidden % 32 || inter % 32 || hidden == 0 || inter == 0)
            fail(LARQL_HIP_ERR_INVALID, "multi-layer FFN: hidden and inter must be multiples of 32");
        // work: x ping-pong [2][hidden], gate, up, act [inter], Q8 activation
        const size_t nf = 2 * hidden + 3 * inter + hidden / 32;
        const size_t q8_off = (nf * sizeof(float) + 255) & ~size_t(255);
        uint8_t* raw = static_cast<uint8_t*>(larql::ensure(c, c->ffn_work, q8_off + hidden));
        float* base = reinterpret_cast<float*>(raw);
        float *X[2] = {base, base + hidden}, *G = base + 2 * hidden, *U = G + inter, *A = U + inter;
        float* q8s = A + inter;
        int8_t* q8 = reinterpret_cast<int8_t*>(raw + q8_off);
        LARQL_HIP_CHECK(hipMemcpyAsync(X[0], x, hidden * sizeof(float), hipMemcpyHostToDevice, c->stream));
        for (size_t l = 0; l < num_layers; l++) {
            const larql_q4_ffn_layer& L = layers[l];
            if (!L.gate || !L.up || !L.down) fail(LARQL_HIP_ERR_INVALID, "multi-layer FFN: null weight");
            const DevWeight& gw = larql::cached_weight(c, LARQL_Q4_0, L.gate, L.gate_len, nullptr, inter, hidden);
            const DevWeight& uw = larql::cached_weight(c, LARQL_Q4_0, L.up, L.up_len, nullptr, inter, hidden);
            const DevWeight& dw = larql::cached_weight(c, LARQL_Q4_0, L.down, L.down_len, nullptr, hidden, inter);
            float *xin = X[l & 1], *xout = X[(l + 1) & 1];
            larql::launch_quantize_q8(xin, hidden, 1, q8, q8s, c->stream);
            larql::launch_q4_0_matvec_pair(gw, uw, q8, q8s, G, U, 1, c->stream);
            larql::launch_gated_mul(G, U, A, inter, LARQL_ACT_SILU, c->stream);
            larql::launch_q4_0_f32_matvec(dw, A, xout, c->stream);
        }
        download(c, out, X[num_layers & 1], hidden * sizeof(float));
    });
}

extern "C" int larql_hip_populate_kv_layer(larql_hip_ctx* c, size_t layer, const float* k_data, const float* v_data,
                                           size_t seq_len, size_t num_kv_heads, size_t head_dim) {
    return guarded(c, [&] {
        if (!k_data || !v_data) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        if (num_kv_heads == 0 || head_dim == 0) fail(LARQL_HIP_ERR_INVALID, "zero kv geometry");
        kv_ensure_layer(c, layer, num_kv_heads, head_dim, seq_len);
        const size_t n = seq_len * num_kv_heads * head_dim;
        const float* dk = stage_upload(c, c->stage_in, k_data, n);
        larql::launch_f32_to_f16(dk, c->kv.k[layer], n, c->stream);
        const float* dv = stage_upload(c, c->stage_in2, v_data, n);
        larql::launch_v_to_cache(dv, true, c->kv.v[layer], seq_len, static_cast<int>(num_kv_heads),
                                 static_cast<int>(head_dim), c->stream);
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
        c->kv.current_len = seq_len;
    });
}

extern "C" int larql_hip_populate_kv_layer_f16_dev(larql_hip_ctx* c, size_t layer, const uint16_t* k_dev,
                                                   const uint16_t* v_dev, size_t seq_len, size_t num_kv_heads,
                                                   size_t head_dim) {
    return guarded(c, [&] {
        if (!k_dev || !v_dev) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        if (num_kv_heads == 0 || head_dim == 0) fail(LARQL_HIP_ERR_INVALID, "zero kv geometry");
        kv_ensure_layer(c, layer, num_kv_heads, head_dim, seq_len);
        const size_t bytes = seq_len * num_kv_heads * head_dim * sizeof(__half);
        LARQL_HIP_CHECK(hipMemcpyAsync(c->kv.k[layer], k_dev, bytes, hipMemcpyDeviceToDevice, c->stream));
        larql::launch_v_to_cache(v_dev, false, c->kv.v[layer], seq_len, static_cast<int>(num_kv_heads),
                                 static_cast<int>(head_dim), c->stream);
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
        c->kv.current_len = seq_len;
    });
}

extern "C" int larql_hip_reset_kv_cache(larql_hip_ctx* c) {
    return guarded(c, [&] { kv_free(c); });
}

extern "C" int larql_hip_kv_cache_len(larql_hip_ctx* c, size_t* len) {
    return guarded(c, [&] {
        if (!len) fail(LARQL_HIP_ERR_INVALID, "null output");
        *len = c->kv.current_len;
    });
}

extern "C" int larql_hip_kv_truncate(larql_hip_ctx* c, size_t len) {
    return guarded(c, [&] {
        if (len > c->kv.current_len) fail(LARQL_HIP_ERR_INVALID, "kv_truncate: length beyond the cache");
        c->kv.current_len = len;
    });
}

extern "C" int larql_hip_model_create(larql_hip_ctx* c, const larql_pipeline_layer* layers, size_t num_layers,
                                      size_t hidden, size_t inter, int weights_on_device, larql_hip_model** out) {
    return guarded(c, [&] {
        if (!out) fail(LARQL_HIP_ERR_INVALID, "null output");
        *out = build_model(c, layers, num_layers, hidden, inter, weights_on_device != 0);
    });
}

extern "C" int larql_hip_model_set_head(larql_hip_ctx* c, larql_hip_model* m, const larql_quant_weight* head,
                                        size_t vocab, const float* final_norm, float eps, int weights_on_device) {
    return guarded(c, [&] {
        if (!m || !head || !final_norm) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        const bool dev = weights_on_device != 0;
        m->head = build_weight(c, m, head->format, m->hidden, {{head->data, head->len, vocab}}, false, dev);
        m->final_norm = upload_vec(c, m, final_norm, m->hidden, dev);
        m->final_eps = eps > 0.f ? static_cast<double>(eps) : 1e-6;
        m->vocab = vocab;
        m->has_head = true;
        LARQL_HIP_CHECK(hipStreamSynchronize(c->stream));
    });
}

extern "C" int larql_hip_model_destroy(larql_hip_ctx* c, larql_hip_model* m) {
    return guarded(c, [&] { destroy_model(c, m); });
}

extern "C" int larql_hip_model_decode_dev(larql_hip_ctx* c, larql_hip_model* m, const float* x_dev,
                                          float* hidden_out_dev, float* logits_dev, void* stream) {
    return guarded(c, [&] {
        if (!m || !x_dev) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        run_decode(c, m, x_dev, hidden_out_dev, logits_dev, pick_stream(c, stream));
    });
}

extern "C" int larql_hip_model_prefill_dev(larql_hip_ctx* c, larql_hip_model* m, const float* x_dev, size_t seq_len,
                                           float* out_dev, void* stream) {
    return guarded(c, [&] {
        if (!m || !x_dev || !out_dev) fail(LARQL_HIP_ERR_INVALID, "null pointer");
        if (seq_len == 0) return;
        hipStream_t s = pick_stream(c, stream);
        kv_ensure_model(c, m, seq_len);
        c->kv.current_len = 0;
        if (seq_len > 1 && prompt_batchable(m))
            run_prompt(c, m, x_dev, seq_len, out_dev, s);
        else
            for (size_t p = 0; p < seq_len; p++)
                run_decode(c, m, x_dev + p * m->hidden, out_dev + p * m->hidden, nullptr, s);
    });
}

// Called by larql_hip_ctx_destroy.
void larql_hip_decode_release(larql_hip_ctx* c) {
    destroy_model(c, c->trait_model);
    c->trait_model = nullptr;
    kv_free(c);
    kv_free_cache(c->kv_aside);
}
