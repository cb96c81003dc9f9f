/*
 * larql_hip.h — C ABI of the MI355X (gfx950) backend for LARQL's quantized
 * compute path.
 *
 * This is the boundary a third `ComputeBackend` implementation binds to
 * (reference trait: larql-main/crates/larql-compute/src/backend.rs:24-164).
 * Conventions follow the reference's existing C kernel ABI
 * (larql-compute/src/cpu/ops/q4_common.rs:6-25 -> csrc/q4_dot.c:169,201):
 * plain pointers and sizes, caller-allocated outputs, no torch/HIP types in
 * the signatures.  Two additions:
 *   - a context handle (device, stream, weight registry, KV cache), and
 *   - an int status: 0 = OK, negative = error (message via
 *     larql_hip_last_error).  A nonzero status is what the Rust trait shim
 *     maps to `None`, which makes callers fall back to the CPU backend exactly
 *     as they do for an unsupported method (backend.rs:45-53, "Returns None
 *     if backend doesn't support Q4").
 *
 * Reference paths below are relative to larql-main/crates/, abbreviated
 *   LC = larql-compute, LV = larql-vindex, LI = larql-inference.
 *
 * Weight bytes are the reference's own layouts (Q4_0 18 B/32, Q4_K 148 B/256,
 * Q6_K 210 B/256, Q8_0 as i8 + separate f32 scales).  On first use a host
 * buffer is uploaded and repacked into a device layout and cached, keyed by
 * (host pointer, length) like the Metal backend's buffer cache
 * (LC/src/metal/buffers.rs:37-85); the same staleness rule applies: a caller
 * that rewrites a buffer in place must call larql_hip_forget_host first.
 *
 * Thread safety: every entry point locks the context; kernels are reentrant.
 */
#ifndef LARQL_HIP_H
#define LARQL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct larql_hip_ctx larql_hip_ctx;

#define LARQL_HIP_OK 0
#define LARQL_HIP_ERR_INVALID (-1)     /* bad argument or shape */
#define LARQL_HIP_ERR_UNSUPPORTED (-2) /* valid request this backend does not implement */
#define LARQL_HIP_ERR_DEVICE (-3)      /* HIP runtime error */
#define LARQL_HIP_ERR_NOMEM (-4)
#define LARQL_HIP_ERR_STATE (-5)       /* e.g. KV cache not initialised */

/* QuantFormat — LC/src/pipeline.rs:12-19 (same discriminant order).  LARQL_F32 is an
 * extension with no QuantFormat counterpart: plain f32 [rows][cols] (any cols), the
 * vindex's f32 gate vectors (LV/src/index/gate.rs:14-29), usable only by the gate-KNN
 * entry points.
 * LARQL_Q4_KF takes both byte layouts the reference gives that name, told apart by the
 * buffer length: exactly rows x (cols/256) x 160 bytes is the pre-baked form
 * ([8 x f16 d*sc_j][8 x f16 dmin*m_j][128 B nibbles], q4k_to_q4kf,
 * LC/src/cpu/ops/q4_common.rs:370-413; pipeline.rs:15); exactly rows x (cols/256) x 144
 * bytes is read as GGUF blocks in the layout the reference's GPU decode reads for Q4_KF
 * (llama.cpp block_q4_K: 6-bit scales and mins packed in 12 bytes, chunk c of 32 bytes
 * holding sub-block 2c in its low and 2c + 1 in its high nibbles;
 * LC/src/metal/shaders/q4kf_qkv_proj.rs:87-119).  Any other length, trailing bytes
 * included, is LARQL_HIP_ERR_INVALID (it could not be told apart). */
typedef enum {
    LARQL_Q4_0 = 0,
    LARQL_Q4_K = 1,
    LARQL_Q4_KF = 2,
    LARQL_Q6_K = 3,
    LARQL_Q8_0 = 4,
    LARQL_F32 = 5
} larql_quant_format;

/* ── lifecycle and metadata ─────────────────────────────────────────────── */

/* Backend construction; replaces MetalBackend::new() in default_backend()
 * (LC/src/lib.rs:68-78).  device = HIP device ordinal. */
int larql_hip_ctx_create(int device, larql_hip_ctx** out);
void larql_hip_ctx_destroy(larql_hip_ctx* ctx);
/* Message of the last failed call on this context ("" if none). */
const char* larql_hip_last_error(larql_hip_ctx* ctx);
/* ComputeBackend::name — LC/src/backend.rs:160 */
const char* larql_hip_name(void);
/* ComputeBackend::device_info — LC/src/backend.rs:163 */
int larql_hip_device_info(larql_hip_ctx* ctx, char* buf, size_t len);
/* ComputeBackend::has_q4 — LC/src/backend.rs:155 */
int larql_hip_has_q4(larql_hip_ctx* ctx);
/* ComputeBackend::has_kv_cache — LC/src/backend.rs:99 */
int larql_hip_has_kv_cache(larql_hip_ctx* ctx);
/* Block until all work queued on the context stream has finished. */
int larql_hip_synchronize(larql_hip_ctx* ctx);

/* ComputeBackend::matmul / matmul_transb — LC/src/backend.rs:27-31 (Metal: tiled sgemm,
 * LC/src/metal/f32_ops.rs:93-140).  f32, row-major, host pointers:
 *   transpose_b == 0: c[m][n] = a[m][k] . b[k][n]
 *   transpose_b != 0: c[m][n] = a[m][k] . b[n][k]^T
 * Each element of c is one f32 fma chain over k = 0 .. k-1 from +0 (reproducible bit for
 * bit; the reference CPU sgemm sums in its own blocked order, within f32 rounding).  Both
 * operands are uploaded on every call (no caching: callers update operands in place, as
 * the k-means centroids of LV/src/clustering/kmeans.rs:28 are).  k == 0 gives zeros;
 * m == 0 or n == 0 writes nothing.  ComputeBackend::matmul_batch (:35-43) is these calls
 * in order. */
int larql_hip_matmul(larql_hip_ctx* ctx, const float* a, size_t m, size_t k, const float* b, size_t n,
                     int transpose_b, float* c);
/* Same on device pointers, enqueued on `stream` (null: the context stream). */
int larql_hip_matmul_dev(larql_hip_ctx* ctx, const float* a, size_t m, size_t k, const float* b, size_t n,
                         int transpose_b, float* c, void* stream);

/* ── weight registry (explicit form of the Metal buffer cache) ─────────── */

/* Upload + repack a reference-layout weight from host memory.  q8_scales is
 * used only for LARQL_Q8_0 (QuantWeight.scales, LC/src/pipeline.rs:22-27). */
int larql_hip_register_weight(larql_hip_ctx* ctx, int format, const void* data, size_t len,
                              const float* q8_scales, size_t rows, size_t cols, uint64_t* handle);
/* Same, from reference-layout bytes already in device memory. */
int larql_hip_register_weight_device(larql_hip_ctx* ctx, int format, const void* dev_data, size_t len,
                                     const float* dev_q8_scales, size_t rows, size_t cols,
                                     uint64_t* handle);
int larql_hip_release_weight(larql_hip_ctx* ctx, uint64_t handle);
/* Drop cached device copies made from host pointer `data` (any length). */
int larql_hip_forget_host(larql_hip_ctx* ctx, const void* data);
/* Bytes of device memory held by one registered weight. */
int larql_hip_weight_device_bytes(larql_hip_ctx* ctx, uint64_t handle, size_t* bytes);

/* ── trait methods (host memory in, caller-allocated host memory out) ──── */
/* Weight arguments carry their byte length (the Rust slice length); a shape
 * that needs more bytes than that is rejected with LARQL_HIP_ERR_INVALID. */

/* ComputeBackend::q4_matvec — LC/src/backend.rs:49-53; CPU twin
 * q4_0_matvec_c, LC/csrc/q4_dot.c:107/169.  scores[num_rows] = Q4_0[num_rows,hidden] . Q8(x).
 * Per-block int32 dots are exact; blocks are accumulated in order as
 * acc += (float)isum_b * (f16(scale_b) * q8_scales[b]) (q4_dot.c:58-89). */
int larql_hip_q4_matvec(larql_hip_ctx* ctx, const uint8_t* q4_data, size_t q4_len, const int8_t* q8_x,
                        const float* q8_scales, float* scores, size_t num_rows, size_t hidden);

/* ComputeBackend::q4_vecmat — LC/src/backend.rs:56-60 (CPU: LC/src/cpu/ops/q4_vecmat.rs:8-18 ->
 * LC/csrc/q4_dot.c:201-232).  out[hidden] = activation[intermediate] . deq(Q4_0[intermediate, hidden]);
 * rows whose activation lies in (-1e-10, 1e-10) are skipped and each term is
 * (float)(nib - 8) * (f16(d) * act), as in the reference.  The rows are summed in chunks
 * (deterministic) rather than in one serial chain per column: results agree with the
 * reference to f32 rounding, not bit for bit. */
int larql_hip_q4_vecmat(larql_hip_ctx* ctx, const float* activation, const uint8_t* q4_data, size_t q4_len,
                        float* out, size_t intermediate, size_t hidden);

/* ComputeBackend::q4_matvec_pair_batch — LC/src/backend.rs:64-69 (Metal LC/src/metal/ops/q4_batched.rs:19-80):
 * for each of the seq_len rows x_s of x_matrix [seq_len][hidden], q = quantize_to_q8(x_s),
 * gate_out[s] = q4_matvec(gate, q), up_out[s] = q4_matvec(up, q); bit-exact with
 * larql_hip_q4_matvec.  gate_out and up_out are [seq_len][num_rows]. */
int larql_hip_q4_matvec_pair_batch(larql_hip_ctx* ctx, const uint8_t* gate_q4, size_t gate_len, const uint8_t* up_q4,
                                   size_t up_len, const float* x_matrix, size_t seq_len, float* gate_out,
                                   float* up_out, size_t num_rows, size_t hidden);

/* ComputeBackend::q4k_matvec — LC/src/backend.rs:126-130 (CPU: LC/src/cpu/ops/q4k_matvec.rs:31-90). */
int larql_hip_q4k_matvec(larql_hip_ctx* ctx, const uint8_t* q4k_data, size_t q4k_len, const float* x,
                         float* out, size_t num_rows, size_t hidden);

/* Prefill projection: out[m][num_rows] = x[m][hidden] . deq(Q4_K)^T for m tokens at once —
 * the per-position q4k_matvec loop of the Metal prefill (LC/src/metal/prefill.rs:21-110,
 * trait prefill_q4 LC/src/backend.rs:143-152) as one MFMA GEMM (fp16 operands, f32 sums).
 * m = 1 is the matvec. */
int larql_hip_q4k_matmul(larql_hip_ctx* ctx, const uint8_t* q4k_data, size_t q4k_len, const float* x, size_t m,
                         float* out, size_t num_rows, size_t hidden);

/* ComputeBackend::q6k_matvec — LC/src/backend.rs:133-137 (CPU: LC/src/cpu/ops/q6k_matvec.rs:31-90). */
int larql_hip_q6k_matvec(larql_hip_ctx* ctx, const uint8_t* q6k_data, size_t q6k_len, const float* x,
                         float* out, size_t num_rows, size_t hidden);

/* ── free functions of the reference exposed as extensions ─────────────── */

/* quantize_to_q8 — LC/src/cpu/ops/q4_common.rs:28-44 (bit-exact). n % 32 == 0. */
int larql_hip_quantize_to_q8(larql_hip_ctx* ctx, const float* x, size_t n, int8_t* q8, float* scales);

/* q8_matvec::dispatch — LC/src/cpu/ops/q8_matvec.rs:36-62, batched over m
 * activation rows: out[i*num_rows + r] = sum_b (float)isum(i,r,b) * (w_scales[r,b] * x_scales[i,b]),
 * blocks in order (bit-exact with the CPU function). */
int larql_hip_q8_matvec(larql_hip_ctx* ctx, const int8_t* w_q8, size_t w_len, const float* w_scales,
                        const int8_t* x_q8, const float* x_scales, size_t m, float* out, size_t num_rows,
                        size_t hidden);

/* Weight quantizers of the reference, on the device and byte-identical to the
 * host versions: quantize_q4_0 (LC/src/cpu/ops/q4_common.rs:50-81),
 * quantize_q4_k (:104-170), quantize_q6_k (:179-239) and quantize_weights_q8
 * (LC/src/cpu/ops/q8_matvec.rs:11-34).  x holds n floats (n % 32 == 0, or
 * n % 256 == 0 for the K formats); `out` receives the reference layout
 * (n/32*18, n/256*148, n/256*210 or n bytes); q8_scales (Q8_0 only) n/32 floats. */
int larql_hip_quantize_weights(larql_hip_ctx* ctx, int format, const float* x, size_t n, void* out,
                               float* q8_scales);

/* ── device-resident fast path (device pointers; enqueue on `stream`) ──── */

/* One matvec with a registered weight.  For LARQL_Q4_K / LARQL_Q6_K `x` is f32
 * [m][cols] and x_scales is unused (m > 1: Q4_K runs the fp16-operand prefill GEMM, Q6_K
 * the f32-accuracy GEMM of the prompt pass); for LARQL_Q4_0 / LARQL_Q8_0 `x` is int8 [m][cols] and x_scales f32
 * [m][cols/32], any m (each output row in the single-row order, bit for bit).
 * out is f32 [m][rows].
 * LARQL_Q4_KF takes f32 x too (m > 1 runs m matvecs).
 * The prefill GEMM packs x as fp16 into a workspace owned by the context; a call with a
 * larger m than any before on the context grows it (device synchronize + allocation), so
 * device calls on one context must not overlap on different streams.
 * stream: a hipStream_t, or NULL for the context stream.  Returns after enqueue. */
int larql_hip_matvec_dev(larql_hip_ctx* ctx, uint64_t handle, const void* x, const float* x_scales,
                         float* out, size_t m, void* stream);

/* Measurement aid with no counterpart in the reference: reads every device byte of a
 * registered weight once and does no arithmetic on them, so its duration is the memory
 * floor for those bytes in that launch shape.  workgroups = threads = 0 (Q4_K / Q4_KF
 * weights): the launch shape of the weight's matvec (4 * ceil(rows / 64) words of out
 * always suffice); else, for any format, `workgroups` workgroups of `threads` (64 .. 1024,
 * a multiple of 64).  out: device
 * uint32 [out_words], out_words >= the workgroup count; receives one XOR fold of the
 * bytes per workgroup. */
int larql_hip_read_floor_dev(larql_hip_ctx* ctx, uint64_t handle, unsigned workgroups, unsigned threads,
                             uint32_t* out, size_t out_words, void* stream);

/* Measurement aid with no counterpart in the reference: the launch configuration of a
 * registered Q4_K / Q4_KF weight's m = 1 matvec (q4k_mfma_kernel<ur, tiles, norm, header,
 * pre, xb>): super-blocks per wave and round (ur), 16-row tiles per workgroup, units whose
 * loads are issued with x (pre), the x-first barrier (xb, 0 or 1), rounds per wave, and
 * the grid (workgroups x threads per workgroup).  Any pointer may be NULL. */
int larql_hip_q4k_launch_shape(larql_hip_ctx* ctx, uint64_t handle, int* ur, int* tiles, int* pre, int* xb,
                               int* rounds, unsigned* workgroups, unsigned* threads);

/* q4_vecmat with a registered Q4_0 weight (rows = intermediate, cols = hidden), device
 * activation f32 [rows] and output f32 [cols].  Uses a partials buffer owned by the
 * context: device calls on one context must not overlap on different streams. */
int larql_hip_vecmat_dev(larql_hip_ctx* ctx, uint64_t handle, const float* activation, float* out, void* stream);

/* q4_matvec_pair_batch with registered Q4_0 gate and up weights of equal shape: x f32
 * [seq_len][cols] (device), gate_out / up_out f32 [seq_len][rows] (device).  Quantizes x
 * into a context-owned buffer (same overlap rule as larql_hip_vecmat_dev). */
int larql_hip_pair_batch_dev(larql_hip_ctx* ctx, uint64_t gate, uint64_t up, const float* x, size_t seq_len,
                             float* gate_out, float* up_out, void* stream);

/* quantize_to_q8 on device memory, m rows of n floats. */
int larql_hip_quantize_to_q8_dev(larql_hip_ctx* ctx, const float* x, size_t n, size_t m, int8_t* q8,
                                 float* scales, void* stream);

/* larql_hip_quantize_weights on device memory. */
int larql_hip_quantize_weights_dev(larql_hip_ctx* ctx, int format, const float* x, size_t n, void* out,
                                   float* q8_scales, void* stream);


/* ── vindex gate-KNN (vindex code, not trait methods: LV/src/index/gate.rs) ── */

/* Largest top_k of the selection kernels, and the most layers per call.  The entry points
 * that allocate take any top_k >= 1 (rows x top_k < 2^31), as the reference does: above
 * LARQL_HIP_TOPK_MAX a row is ranked by a sort (same order, more time and a work buffer);
 * the allocation-free entry point keeps the bound.  A top_k above a row's length returns
 * the whole row ranked (top_k.min(len), LV/src/index/walk.rs:569): slots past the row
 * length hold index 0xFFFFFFFF and score 0. */
#define LARQL_HIP_TOPK_MAX 512
#define LARQL_HIP_KNN_MAX_LAYERS 64

/* Gate KNN for one layer from host memory: VectorIndex::gate_knn (LV/src/index/gate.rs:108-134)
 * for each of nq queries, i.e. the per-position lists of gate_knn_batch (:500-537) before
 * their union.  format LARQL_F32: scores = gate[features, hidden] . q (gemv, :14-29);
 * format LARQL_Q4_0: gate_knn_q4 (:711-731), q quantized by quantize_to_q8 and scored by
 * q4_matvec.  Output per query: top_k (index, score) by |score| descending (top_k_from_scores,
 * :307-316), ties in index order.  idx u32 and scores f32, [nq][top_k]. */
int larql_hip_gate_knn(larql_hip_ctx* ctx, int format, const void* gate, size_t gate_len, size_t features,
                       size_t hidden, const float* queries, size_t nq, size_t top_k, uint32_t* idx,
                       float* scores);

/* Device form over several layers in one launch: handles of registered gate matrices
 * (all LARQL_F32, or all LARQL_Q4_0, with equal shapes), queries f32 [nq][hidden] in
 * device memory, idx / scores [n_layers][nq][top_k] in device memory. */
int larql_hip_gate_knn_dev(larql_hip_ctx* ctx, const uint64_t* handles, size_t n_layers, const float* queries,
                           size_t nq, size_t top_k, uint32_t* idx, float* scores, void* stream);

/* Scores only: scores f32 [n_layers][nq][features] (device). */
int larql_hip_gate_scores_dev(larql_hip_ctx* ctx, const uint64_t* handles, size_t n_layers, const float* queries,
                              size_t nq, float* scores, void* stream);

/* Top-k of each row of a device score matrix [rows][n]: signed_mode 0 orders by |score|
 * (gate.rs:307-316), 1 by the signed score (lm-head KNN, LV/src/index/walk.rs:563-580).
 * Ties in index order.  idx / vals [rows][k] (device), k >= 1. */
int larql_hip_topk_dev(larql_hip_ctx* ctx, const float* scores, size_t rows, size_t n, size_t k, int signed_mode,
                       uint32_t* idx, float* vals, void* stream);

/* lm-head KNN, the Q4 path of VectorIndex::lm_head_knn_backend (LV/src/index/walk.rs:549-583):
 * query quantized by quantize_to_q8, scores = q4_matvec(lm_head_q4 [vocab][hidden] Q4_0),
 * the top_k tokens by signed score descending (ties in index order), top_k >= 1.
 * Host-pointer form: lm_head_q4 / query / idx / scores in host memory (the head is
 * uploaded once and cached like every weight). */
int larql_hip_lm_head_knn(larql_hip_ctx* ctx, const uint8_t* lm_head_q4, size_t len, const float* query,
                          size_t vocab, size_t hidden, size_t top_k, uint32_t* idx, float* scores);
/* Device form: a registered LARQL_Q4_0 head, nq queries f32 [nq][hidden] (device),
 * idx / scores [nq][top_k] (device). */
int larql_hip_lm_head_knn_dev(larql_hip_ctx* ctx, uint64_t handle, const float* queries, size_t nq, size_t top_k,
                              uint32_t* idx, float* scores, void* stream);

/* Bytes of the fixed device array behind larql_hip_lm_head_knn_dev_noalloc (one per GPU). */
#define LARQL_HIP_NOALLOC_SCRATCH_BYTES (8u << 20)

/* larql_hip_lm_head_knn_dev without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate — code under HIP graph capture,
 * per-token serving loops, harnesses that forbid hipMalloc.  Same arguments, kernels and
 * results as larql_hip_lm_head_knn_dev; the quantized queries and the vocabulary scores
 * live in a fixed device array of LARQL_HIP_NOALLOC_SCRATCH_BYTES per GPU (8 MiB, held
 * until the process ends), with the top-k candidates of a vocabulary ranked in chunks
 * (above 14336 entries for top_k <= 64, chunks of 4096; above 12288 for larger top_k,
 * chunks of 12288), which limits a call to
 *   nq * (vocab * 4 + hidden * 9 / 8 + chunks * top_k * 8) (+ alignment) <= 8 MiB
 * (vocab 128256, top_k 5: up to 16 queries), and top_k <= LARQL_HIP_TOPK_MAX (a larger
 * top_k needs a sort buffer); larger requests return LARQL_HIP_ERR_INVALID.  Every
 * call on one GPU shares that array: calls that overlap on one GPU (different streams or
 * contexts) race. */
int larql_hip_lm_head_knn_dev_noalloc(larql_hip_ctx* ctx, uint64_t handle, const float* queries, size_t nq,
                                      size_t top_k, uint32_t* idx, float* scores, void* stream);

/* ── decode step: layers, KV cache, full-pipeline decode ───────────────── */

/* QuantWeight — LC/src/pipeline.rs:22-27.  `data`/`len` are reference-layout
 * bytes (host memory, or device memory for the *_dev model constructor);
 * `scales` only for LARQL_Q8_0. */
typedef struct {
    const void* data;
    size_t len;
    const float* scales;
    int format;
} larql_quant_weight;

/* NormType / FfnType / Activation — LC/src/pipeline.rs:31-56. */
enum { LARQL_NORM_RMS = 0, LARQL_NORM_LAYER = 1 };
enum { LARQL_FFN_GATED = 0, LARQL_FFN_STANDARD = 1 };
enum { LARQL_ACT_SILU = 0, LARQL_ACT_GELU_TANH = 1 };

/* FullPipelineLayer — LC/src/pipeline.rs:60-120, same fields in the same order.
 * Optional vectors are NULL when absent.  The HIP decode step and prompt pass implement
 * RMSNorm layers with a gated FFN and Q4_K or Q6_K projections (each its own format, as in
 * Q4_K_M files) — and Q8_0 attention / Q4_0 FFN projections (the reference decode's Q8
 * and Q4_0 paths, LC/src/metal/decode.rs:262-296, 374-404, 560-690; Q8_0 needs
 * larql_quant_weight.scales), Q4_KF in either byte layout — with the variants the
 * reference's decode reads per layer
 * (LC/src/metal/decode.rs:98-739): norm_offset (weight = offset + w), SiLU or GELU-tanh,
 * has_post_norms (h + norm(o, post_attn_norm); FFN input norm(h, pre_ffn_norm); h +
 * norm(down, post_ffn_norm); an absent pre/post-FFN weight is the weight-free norm, as the
 * CPU path has it, LI/src/forward/layer.rs:65-83), has_v_norm, layer_scalar (0 = off),
 * rotary_dim, sliding_window and attn_scale.  LayerNorm, the ungated FFN and biases are
 * reported as LARQL_HIP_ERR_UNSUPPORTED so the caller falls back (predict.rs:397-430). */
typedef struct {
    larql_quant_weight wq, wk, wv, wo;
    larql_quant_weight gate, up, down;
    const float* input_norm;
    const float* post_attn_norm;
    const float* pre_ffn_norm;
    const float* post_ffn_norm;
    const float* input_norm_bias;
    const float* post_attn_norm_bias;
    float norm_offset;
    float qk_norm_offset;
    float eps;
    int has_post_norms;
    int norm_type;
    int ffn_type;
    int activation;
    float attn_scale;
    size_t head_dim;
    size_t num_q_heads;
    size_t num_kv_heads;
    float rope_base;
    size_t rotary_dim;      /* 0 = head_dim */
    size_t sliding_window;  /* 0 = full attention */
    int has_v_norm;
    float layer_scalar;
    const float* ffn_up_bias;
    const float* ffn_down_bias;
} larql_pipeline_layer;

/* ComputeBackend::decode_token — LC/src/backend.rs:115-123.  Runs one token
 * through all layers with the KV cache (fp16 on the device, appended at the
 * current length, which then advances by one; attention is not limited in T).
 * x and out are host vectors of `hidden` floats (out = final hidden state,
 * before the final norm, as the reference returns it).  Each layer's own head_dim,
 * num_q_heads and num_kv_heads are used (layers may differ, as the reference's decode
 * reads them per layer, LC/src/metal/decode.rs:101-110): head_dim a multiple of 32 up to
 * 512, 1..8 query heads per kv head.  q_dim and kv_dim are the widest layer's (the
 * reference's buffer widths); num_q_heads, num_kv_heads, head_dim and rope_base are
 * unused, as in the reference. */
int larql_hip_decode_token(larql_hip_ctx* ctx, const larql_pipeline_layer* layers, size_t num_layers,
                           const float* x, size_t hidden, size_t inter, size_t q_dim, size_t kv_dim,
                           size_t num_q_heads, size_t num_kv_heads, size_t head_dim, float rope_base,
                           float* out);

/* ComputeBackend::prefill_q4 — LC/src/backend.rs:139-152: a prompt of seq_len tokens
 * (x: host [seq_len][hidden]) through all layers at positions 0 .. seq_len-1, the
 * post-RoPE K/V of every position stored in the cache (whose length becomes seq_len);
 * out: host [seq_len][hidden], the final hidden state of every position (before the
 * final norm).  Layers with gate|up in Q4_K and Q4_K / Q6_K elsewhere run once over all
 * positions; others run position by position through the decode-step kernels.
 * use_qk_norm != 0 scales each RoPE'd query head by 1 / sqrt(sum q^2 + 1e-6) and
 * softcap > 0 maps each scaled score s to tanh(s / softcap) * softcap (the reference's
 * fused attention, LC/src/metal/shaders/fused_attention.rs:79-88, 132-137); the cached K
 * rows are not normed, and a later decode_token applies neither. */
int larql_hip_prefill_q4(larql_hip_ctx* ctx, const larql_pipeline_layer* layers, size_t num_layers,
                         const float* x, size_t hidden, size_t inter, size_t q_dim, size_t kv_dim, size_t seq_len,
                         size_t num_q_heads, size_t num_kv_heads, size_t head_dim, float rope_base,
                         int use_qk_norm, float softcap, float* out);

/* ComputeBackend::full_pipeline_q4 — LC/src/backend.rs:71-84 (Metal LC/src/metal/trait_impl.rs:43-76 ->
 * ops/full_pipeline.rs:201-687): x [seq_len][hidden] at positions 0 .. seq_len-1 through all
 * layers with causal attention among those positions only (no KV cache: the context's decode
 * cache is left as it was); out [seq_len][hidden] (host), the last layer's hidden state of
 * every position.  The trait returns the first `hidden` floats of it (the reference calls it
 * with seq_len = 1, LI/src/layer_graph/predict.rs:406).  Layers as for decode_token, Q8_0
 * attention and Q4_0 FFN weights included; use_qk_norm and softcap as for prefill_q4. */
int larql_hip_full_pipeline_q4(larql_hip_ctx* ctx, const larql_pipeline_layer* layers, size_t num_layers,
                               const float* x, size_t hidden, size_t inter, size_t q_dim, size_t kv_dim,
                               size_t seq_len, size_t num_q_heads, size_t num_kv_heads, size_t head_dim,
                               float rope_base, int use_qk_norm, float softcap, float* out);

/* One layer of multi_layer_q4_ffn: the (gate, up, down_t) Q4_0 slices of the reference's
 * &[(&[u8], &[u8], &[u8])] with their byte lengths.  gate and up are [inter][hidden], down
 * [hidden][inter] (the interleaved_q4.bin layout, LI/src/layer_graph/predict.rs:177-191). */
typedef struct {
    const uint8_t* gate;
    size_t gate_len;
    const uint8_t* up;
    size_t up_len;
    const uint8_t* down;
    size_t down_len;
} larql_q4_ffn_layer;

/* ComputeBackend::multi_layer_q4_ffn — LC/src/backend.rs:86-96 (Metal LC/src/metal/ops/q4_batched.rs:97-212):
 * x_0 = x; per layer q = quantize_to_q8(x_l), g = q4_matvec(gate, q), u = q4_matvec(up, q)
 * (bit-exact block order), a = silu(g) * u, x_{l+1} = down . a with the f32 activation
 * (q4_f32_matvec, LC/src/metal/shaders/q4_f32_matvec.rs); out [hidden] = x_L (layers chained
 * without a residual add, as the reference chains them).  Host memory in and out; the Q4_0
 * slices are cached like every weight. */
int larql_hip_multi_layer_q4_ffn(larql_hip_ctx* ctx, const larql_q4_ffn_layer* layers, size_t num_layers,
                                 const float* x, size_t inter, size_t hidden, float* out);

/* ComputeBackend::populate_kv_layer — LC/src/backend.rs:103-107: K/V rows
 * [seq_len][num_kv_heads*head_dim] f32 (stored as fp16, RNE); sets the cache
 * length to seq_len.  The layer takes this geometry (layers below it not yet held
 * take it too); a decode whose layer geometry differs from a held layer's drops the
 * cache's rows. */
int larql_hip_populate_kv_layer(larql_hip_ctx* ctx, size_t layer, const float* k_data, const float* v_data,
                                size_t seq_len, size_t num_kv_heads, size_t head_dim);
/* ComputeBackend::reset_kv_cache — LC/src/backend.rs:110 (drops the cache). */
int larql_hip_reset_kv_cache(larql_hip_ctx* ctx);
/* Current cache length (positions held). */
int larql_hip_kv_cache_len(larql_hip_ctx* ctx, size_t* len);
/* Rewind the cache to `len` positions (len <= current length). */
int larql_hip_kv_truncate(larql_hip_ctx* ctx, size_t len);
/* populate_kv_layer from device fp16 data [seq_len][num_kv_heads*head_dim]. */
int larql_hip_populate_kv_layer_f16_dev(larql_hip_ctx* ctx, size_t layer, const uint16_t* k_dev,
                                        const uint16_t* v_dev, size_t seq_len, size_t num_kv_heads,
                                        size_t head_dim);

/* ── device-resident decoder (extension; no counterpart in the trait) ──────
 * The same decode step with the weights registered once and activations in
 * device memory, for serving loops and benchmarks.  `weights_on_device`
 * selects whether the larql_quant_weight data pointers are device addresses. */
typedef struct larql_hip_model larql_hip_model;
int larql_hip_model_create(larql_hip_ctx* ctx, const larql_pipeline_layer* layers, size_t num_layers,
                           size_t hidden, size_t inter, int weights_on_device, larql_hip_model** out);
/* Final norm + output head (LI/src/layer_graph/generate.rs:140-143): logits =
 * head . rms_norm(h, final_norm).  head: Q4_K or Q6_K [vocab][hidden]. */
int larql_hip_model_set_head(larql_hip_ctx* ctx, larql_hip_model* model, const larql_quant_weight* head,
                             size_t vocab, const float* final_norm, float eps, int weights_on_device);
int larql_hip_model_destroy(larql_hip_ctx* ctx, larql_hip_model* model);
/* One decode step on device memory: x_dev [hidden] in; hidden_out_dev [hidden]
 * (may be NULL) and logits_dev [vocab] (may be NULL; needs a head) out.  Appends
 * K/V at the current cache length and advances it.  Enqueues on `stream`. */
int larql_hip_model_decode_dev(larql_hip_ctx* ctx, larql_hip_model* model, const float* x_dev,
                               float* hidden_out_dev, float* logits_dev, void* stream);
/* A prompt on device memory (the trait's prefill_q4, LC/src/backend.rs:139-152, for a
 * registered model): x_dev [seq_len][hidden] at positions 0 .. seq_len-1 in,
 * out_dev [seq_len][hidden] (each position's last-layer hidden state) out; the KV
 * cache is reset and left at seq_len.  Enqueues on `stream`. */
int larql_hip_model_prefill_dev(larql_hip_ctx* ctx, larql_hip_model* model, const float* x_dev, size_t seq_len,
                                float* out_dev, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* LARQL_HIP_H */
