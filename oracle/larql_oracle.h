/*
 * larql_oracle.h — CPU oracle for the LARQL quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * CPU backend (larql-compute `CpuBackend`, its C kernel q4_dot.c, and the
 * larql-inference CPU numerics used by the decode step).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker.  The product library (liblarql_hip.so) never links,
 * loads or calls anything here.
 *
 * Every function cites the reference file:line it follows; paths are relative
 * to the reference repository root, abbreviated
 *   LC/ = larql-main/crates/larql-compute/
 *   LI/ = larql-main/crates/larql-inference/
 *   LV/ = larql-main/crates/larql-vindex/
 *
 * Build: gcc -O3 -mavx2 -ffp-contract=off (the reference C kernel's flags,
 * LC/build.rs:12-17, plus no mul+add contraction because Rust never fuses).
 */
#ifndef LARQL_ORACLE_H
#define LARQL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── f16 codecs ─────────────────────────────────────────────────────────── */
float    lo_f16_to_f32(uint16_t bits);          /* LC/src/cpu/ops/q4_common.rs:426-442 */
float    lo_decode_f16(uint16_t h);             /* LC/csrc/q4_dot.c:9-35              */
uint16_t lo_f32_to_f16_trunc(float v);          /* LC/src/cpu/ops/q4_common.rs:83-95  */
uint16_t lo_f32_to_f16_rne(float v);            /* IEEE-754 round-to-nearest-even (KV cache storage) */

/* ── quantizers ─────────────────────────────────────────────────────────── */
void lo_quantize_to_q8(const float* x, size_t n, int8_t* q8, float* scales);       /* q4_common.rs:28-44  */
void lo_quantize_q4_0(const float* x, size_t n, uint8_t* out);                     /* q4_common.rs:50-81  */
void lo_quantize_q4_k(const float* x, size_t n, uint8_t* out);                     /* q4_common.rs:104-170 */
void lo_quantize_q6_k(const float* x, size_t n, uint8_t* out);                     /* q4_common.rs:179-239 */
void lo_quantize_weights_q8(const float* w, size_t rows, size_t cols,
                            int8_t* q8, float* scales);                            /* q8_matvec.rs:11-34  */

/* ── matvecs ────────────────────────────────────────────────────────────── */
/* x86 scalar float order, LC/csrc/q4_dot.c:169-199 */
void lo_q4_0_matvec_x86(const uint8_t* q4, const int8_t* q8x, const float* q8s,
                        float* out, size_t rows, size_t hidden);
/* ARM/Metal int32-block order, LC/csrc/q4_dot.c:48-126 */
void lo_q4_0_matvec_blockint(const uint8_t* q4, const int8_t* q8x, const float* q8s,
                             float* out, size_t rows, size_t hidden);
/* per-block int32 dots, isum[row*blocks + b] (exact integers) */
void lo_q4_0_block_dots(const uint8_t* q4, const int8_t* q8x, int32_t* isum,
                        size_t rows, size_t hidden);
/* LC/csrc/q4_dot.c:201-232 */
void lo_q4_0_vecmat(const float* act, const uint8_t* q4, float* out,
                    size_t inter, size_t hidden);
/* LC/src/cpu/ops/q4k_matvec.rs:31-90 */
void lo_q4k_matvec(const uint8_t* q4k, const float* x, float* out, size_t rows, size_t hidden);
/* LC/src/cpu/ops/q6k_matvec.rs:31-90 */
void lo_q6k_matvec(const uint8_t* q6k, const float* x, float* out, size_t rows, size_t hidden);
/* Q4_KF in its two byte layouts (the trait's QuantFormat::Q4_KF, LC/src/pipeline.rs:15).
 * 144-byte GGUF block as the reference's GPU decode reads it (llama.cpp block_q4_K,
 * LC/src/metal/shaders/q4kf_qkv_proj.rs:87-119): [f16 d][f16 dmin][12 B: 6-bit scales and
 * mins, llama.cpp packing][128 B: chunk c of 32 bytes holds sub-block 2c in its low and
 * 2c+1 in its high nibbles].  w = d*sc_j*q - dmin*m_j, accumulated in element order. */
void lo_q4kf_gguf_matvec(const uint8_t* w, const float* x, float* out, size_t rows, size_t hidden);
/* 160-byte block with pre-baked half scales (q4k_to_q4kf, LC/src/cpu/ops/q4_common.rs:370-413):
 * [8 x f16 d*sc_j][8 x f16 dmin*m_j][128 B nibbles in the 148-byte order].  w = sc_j*q - mn_j. */
void lo_q4kf160_matvec(const uint8_t* w, const float* x, float* out, size_t rows, size_t hidden);
/* Scale and 6-bit min of sub-block j from the 12 packed bytes of a GGUF block (llama.cpp
 * get_scale_min_k4, stated in the reference at LM/src/quant/ggml.rs:252-262). */
void lo_gguf_scale_min(int j, const uint8_t* q12, uint8_t* sc, uint8_t* mn);
/* The reference's converters and GGUF quantizer (LC/src/cpu/ops/q4_common.rs): byte layouts
 * as the reference writes them.  q4k_to_gguf and quantize_q4_k_gguf pack scales and mins
 * their own way (bytes 0..7: sc | (m & 3) << 6, bytes 8..11: m >> 2 nibbles) and keep the
 * 148-byte nibble order, which the llama.cpp-layout GPU kernels do not read back. */
void lo_q4k_to_gguf(const uint8_t* q4k, size_t nblocks, uint8_t* out);        /* :321-361 */
void lo_quantize_q4_k_gguf(const float* x, size_t n, uint8_t* out);           /* :248-314 */
void lo_q4k_to_q4kf(const uint8_t* q4k, size_t nblocks, uint8_t* out);        /* :370-413 */
/* Lossless 148-byte Q4_K -> 144-byte llama.cpp layout (the 4-bit mins fit the 6-bit field):
 * test data for the GGUF path whose dequantized values equal the Q4_K block's. */
void lo_q4k_to_gguf_llamacpp(const uint8_t* q4k, size_t nblocks, uint8_t* out);

/* Q4_0 weights x f32 activation, the reference GPU's q4_f32_matvec
 * (LC/src/metal/shaders/q4_f32_matvec.rs:10-38): per block b, block_sum = sum_j
 * (lo_j - 8) x[2j] + (hi_j - 8) x[2j+1] in f32, acc += block_sum * f16(scale_b). */
void lo_q4_0_f32_matvec(const uint8_t* q4, const float* x, float* out, size_t rows, size_t hidden);

/* LC/src/cpu/ops/q8_matvec.rs:36-62 */
void lo_q8_matvec(const int8_t* wq, const float* ws, const int8_t* xq, const float* xs,
                  float* out, size_t rows, size_t hidden);
void lo_q8_block_dots(const int8_t* wq, const int8_t* xq, int32_t* isum, size_t rows, size_t hidden);

/* ── gate KNN ───────────────────────────────────────────────────────────── */
/* Top-k by |score| descending (LV/src/index/gate.rs:307-316); ties -> lower index. */
void lo_topk_abs(const float* scores, size_t n, size_t k, uint32_t* idx, float* val);
/* Top-k by signed score descending (LV/src/index/walk.rs:563-580); ties -> lower index. */
void lo_topk_signed(const float* scores, size_t n, size_t k, uint32_t* idx, float* val);
/* f32 gate scores in the canonical order shared with the HIP kernel:
 * s[f] = one sequential fmaf chain over k = 0..hidden-1 starting from +0.0f.
 * Parity unpinned for the bit patterns: the reference computes these scores in the
 * third-party matrixmultiply 0.3 sgemm (LV/src/index/gate.rs:14-29 ->
 * larql-main/crates/larql-tensor/src/sgemm.rs:41-68), whose accumulation order is not in
 * the reference tree; the value is pinned against an exact f64 dot within f32 bounds. */
void lo_gate_scores_f32(const float* gate, const float* x, float* out, size_t features, size_t hidden);

/* ── decode-step numerics (LI/src) ──────────────────────────────────────── */
void lo_rms_norm(const float* x, const float* w, float offset, double eps, float* out, size_t n); /* residual.rs:17-33 */
void lo_rope_at(float* x, size_t num_heads, size_t head_dim, size_t rotary_dim,
                double base, size_t pos);                                         /* rope.rs:22-55 */
void lo_silu_gate_up(const float* gate, const float* up, float* out, size_t n);  /* ffn/mod.rs:87-94 */
void lo_gelu_tanh_gate_up(const float* gate, const float* up, float* out, size_t n); /* ffn/mod.rs:96-103 */
/* Per-head parameter-free RMS norm, in place (LI/src/residual.rs:86-110). */
void lo_rms_norm_heads(float* x, size_t num_heads, size_t head_dim, double eps);
/* Single-query GQA over an fp16 cache laid out [t][kv_head][head_dim] (gqa.rs:29-110). */
void lo_attend_f16(const float* q, const uint16_t* kc, const uint16_t* vc, size_t T,
                   size_t num_q, size_t num_kv, size_t head_dim, float scale, float* out);
/* The same with the prompt-attention options: qk_norm != 0 L2-normalises each query head
 * (1 / sqrt(sum q^2 + 1e-6), on a copy of q), softcap > 0 caps every scaled score
 * (LC/src/metal/shaders/fused_attention.rs:79-88, 132-137). */
void lo_attend_f16_opts(const float* q, const uint16_t* kc, const uint16_t* vc, size_t T, size_t num_q,
                        size_t num_kv, size_t head_dim, float scale, int qk_norm, float softcap, float* out);
/* In place: each of num_heads heads of head_dim floats times 1 / sqrt(sum x^2 + 1e-6)
 * (fused_attention.rs:79-88: one f32 sum in element order). */
void lo_qk_norm_heads(float* x, size_t num_heads, size_t head_dim);

/* One decoder layer (Q4_K / Q6_K projections, fp16 KV cache) at position pos.
 * h is updated in place; the new K/V row is written into kc/vc at pos.
 * The fields after fmt are the layer variants of FullPipelineLayer (LC/src/pipeline.rs:76-115);
 * all zero is the Llama layer: no post-norms, SiLU, offset 0, no V-norm, no layer scalar,
 * full rotary, attention scale 1/sqrt(head_dim). */
typedef struct {
    const uint8_t *wq, *wk, *wv, *wo, *gate, *up, *down;  /* Q4_K 148-byte or Q6_K 210-byte layout */
    const float *input_norm, *post_attn_norm;
    uint16_t *k_cache, *v_cache;                             /* [max_seq][kv_heads][head_dim] fp16 */
    /* per projection (wq, wk, wv, wo, gate, up, down): 0 = Q4_K, 1 = Q6_K, 2 = Q4_KF 144-byte
     * GGUF, 3 = Q4_KF 160-byte, 4 = Q8_0 (int8 + f32 scales in *_s; its input is
     * quantize_to_q8 of the f32 input), 5 = Q4_0 (gate / up: Q8-quantized input and the block
     * matvec; down: lo_q4_0_f32_matvec of the f32 activation) — the reference GPU decode's
     * Q8 attention and Q4_0 FFN (LC/src/metal/decode.rs:262-296, 374-404, 560-690); mixed formats
     * per projection as the reference's per-layer QuantWeight allows (LC/src/pipeline.rs:22-27) */
    int fmt[7];
    const float *pre_ffn_norm, *post_ffn_norm;  /* NULL: norm without weight (LI/src/forward/layer.rs:65-68) */
    float norm_offset;                          /* weight = offset + w (LI/src/residual.rs:26-29) */
    int has_post_norms;
    int activation;                             /* 0 = SiLU, 1 = GELU-tanh (LI/src/ffn/mod.rs:87-103) */
    int has_v_norm;                             /* parameter-free RMS norm of V per head */
    float layer_scalar;                         /* 0 = disabled; else h *= layer_scalar */
    size_t rotary_dim;                          /* 0 = head_dim */
    float attn_scale;                           /* 0 = 1/sqrt(head_dim) */
    const float *wq_s, *wk_s, *wv_s, *wo_s, *gate_s, *up_s, *down_s;  /* Q8_0 weight scales */
    /* prompt-attention options of prefill_q4 / full_pipeline_q4 (LC/src/metal/shaders/
     * fused_attention.rs:79-88, 132-137): qk_norm != 0 scales each RoPE'd query head by
     * 1 / sqrt(sum q^2 + 1e-6) (K untouched); softcap > 0 maps each scaled score s to
     * tanh(s / softcap) * softcap */
    int qk_norm;
    float softcap;
    /* non-NULL: f32 K/V caches [max_seq][kv_heads][head_dim] in place of k_cache / v_cache,
     * the reference's cache element type (LC/src/metal/ops/kv_cache.rs:13-14, populate_kv_layer
     * takes f32 rows, LC/src/metal/trait_impl.rs:197-225; the CPU attention works in f32,
     * LI/src/attention/gqa.rs:29-110): the new K/V row is stored unrounded */
    float *k_cache32, *v_cache32;
} lo_layer_t;

void lo_decode_layer(const lo_layer_t* L, float* h, size_t pos,
                     size_t hidden, size_t inter, size_t num_q, size_t num_kv, size_t head_dim,
                     double rope_base, double eps);
void lo_decode_layer_window(const lo_layer_t* L, float* h, size_t pos,
                            size_t hidden, size_t inter, size_t num_q, size_t num_kv, size_t head_dim,
                            double rope_base, double eps, size_t window);
/* lo_decode_layer (window 0) with each projection's rows split over nthreads threads;
 * identical output (CPU baseline use). */
void lo_decode_layer_mt(const lo_layer_t* L, float* h, size_t pos, size_t hidden, size_t inter, size_t num_q,
                        size_t num_kv, size_t head_dim, double rope_base, double eps, int nthreads);
/* One projection (format code as lo_layer_t.fmt; q8in: Q8-quantized input for Q4_0),
 * rows split over nthreads threads; identical output to one thread. */
void lo_proj_rows_mt(int fmt, const uint8_t* w, const float* ws, int q8in, const float* x, float* out, size_t rows,
                     size_t cols, int nthreads);

/* ── deterministic inputs (splitmix64 -> Box-Muller in f64 -> f32) ─────── */
void lo_gauss_f32(uint64_t seed, float mean, float std, float* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
