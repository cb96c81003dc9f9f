/*
 * larql_oracle.c — CPU oracle for the LARQL quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY (see larql_oracle.h): a plain-C restatement of the
 * reference CPU backend, used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker.  The product never calls it.
 *
 * Reference paths: LC/ = larql-main/crates/larql-compute/,
 * LI/ = larql-main/crates/larql-inference/, LV/ = larql-main/crates/larql-vindex/.
 *
 * Numerics rules carried over from the Rust source:
 *  - f32::round is round-half-away-from-zero        -> roundf
 *  - `x.clamp(a,b) as iN` saturates, NaN -> 0       -> sat_* helpers
 *  - f32::max / f32::min ignore a NaN operand       -> fmaxf / fminf
 *  - Rust never contracts a*b+c into an FMA         -> built with -ffp-contract=off
 *
 * Parity status per function (what pins it) is recorded in the test suite;
 * lo_attend_f16's dot-product order follows no reference order (the reference
 * delegates it to ndarray), so attention agrees with the GPU to a tolerance only.
 */
#include "larql_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ── helpers ──────────────────────────────────────────────────────────── */

/* Rust `f as i32` (saturating, NaN -> 0). */
static int32_t sat_i32(float f) {
    if (isnan(f)) return 0;
    if (f >= 2147483647.0f) return 2147483647;
    if (f <= -2147483648.0f) return (-2147483647 - 1);
    return (int32_t)f;
}

/* Rust `v.clamp(lo, hi)` on f32 (NaN passes through). */
static float clampf(float v, float lo, float hi) {
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

/* Rust `f as u8` / `f as i8` after a clamp into range (NaN -> 0). */
static uint8_t f_to_u8(float f) { return isnan(f) ? 0 : (uint8_t)f; }
static int8_t  f_to_i8(float f) { return isnan(f) ? 0 : (int8_t)f; }

static uint16_t rd_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static void     wr_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)(v & 0xFF); p[1] = (uint8_t)(v >> 8); }

/* ── f16 codecs ───────────────────────────────────────────────────────── */

/* LC/src/cpu/ops/q4_common.rs:426-442 (also q4k_matvec.rs:10-25, q6k_matvec.rs:10-25). */
float lo_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u;
    int exp = (bits >> 10) & 0x1F;
    uint32_t mant = bits & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return sign ? -0.0f : 0.0f;
        float val = (float)mant / 1024.0f * ldexpf(1.0f, -14);
        return sign ? -val : val;
    }
    if (exp == 31) {
        if (mant == 0) return sign ? -INFINITY : INFINITY;
        return NAN;
    }
    float val = (1.0f + (float)mant / 1024.0f) * ldexpf(1.0f, exp - 15);
    return sign ? -val : val;
}

/* LC/csrc/q4_dot.c:9-35 — bit-level decoder used by the C kernel. */
float lo_decode_f16(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exponent = (h >> 10) & 0x1Fu;
    uint32_t mantissa = h & 0x3FFu;
    uint32_t result;
    if (exponent == 0) {
        if (mantissa == 0) {
            result = sign;
        } else {
            exponent = 1;
            while (!(mantissa & 0x400u)) { mantissa <<= 1; exponent--; }
            mantissa &= 0x3FFu;
            exponent += 127 - 15;
            result = sign | (exponent << 23) | (mantissa << 13);
        }
    } else if (exponent == 31) {
        result = sign | (255u << 23) | (mantissa << 13);
    } else {
        exponent += 127 - 15;
        result = sign | (exponent << 23) | (mantissa << 13);
    }
    float f;
    memcpy(&f, &result, 4);
    return f;
}

/* LC/src/cpu/ops/q4_common.rs:83-95 — truncating encoder, f16 subnormals flushed. */
uint16_t lo_f32_to_f16_trunc(float val) {
    uint32_t bits;
    memcpy(&bits, &val, 4);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t exp = (int32_t)((bits >> 23) & 0xFFu);
    uint32_t mant = bits & 0x7FFFFFu;
    if (exp == 0) return (uint16_t)sign;
    if (exp == 255) return (uint16_t)(sign | 0x7C00u | (mant >> 13));
    int32_t new_exp = exp - 127 + 15;
    if (new_exp >= 31) return (uint16_t)(sign | 0x7C00u);
    if (new_exp <= 0) return (uint16_t)sign;
    return (uint16_t)(sign | ((uint32_t)new_exp << 10) | (mant >> 13));
}

/* IEEE-754 binary16 round-to-nearest-even with subnormals, as the GPU's
 * v_cvt_f16_f32 does.  Used for the fp16 KV cache of the decode workload. */
uint16_t lo_f32_to_f16_rne(float val) {
    uint32_t x;
    memcpy(&x, &val, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0u));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);    /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: f16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;             /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                 /* value = m * 2^(e-150); unit = 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* ── quantizers ───────────────────────────────────────────────────────── */

static float block_amax(const float* b, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) m = fmaxf(m, fabsf(b[i]));
    return m;
}

/* LC/src/cpu/ops/q4_common.rs:28-44 */
void lo_quantize_to_q8(const float* x, size_t n, int8_t* q8, float* scales) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const float* blk = x + b * 32;
        float amax = block_amax(blk, 32);
        float scale = amax / 127.0f;
        scales[b] = scale;
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        for (int j = 0; j < 32; j++)
            q8[b * 32 + j] = f_to_i8(clampf(roundf(blk[j] * inv), -128.0f, 127.0f));
    }
}

/* LC/src/cpu/ops/q4_common.rs:50-81 (byte j: element 2j low nibble, 2j+1 high). */
void lo_quantize_q4_0(const float* x, size_t n, uint8_t* out) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; b++) {
        const float* blk = x + b * 32;
        uint8_t* o = out + b * 18;
        float amax = block_amax(blk, 32);
        float scale = amax / 7.0f;
        float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
        wr_u16(o, lo_f32_to_f16_trunc(scale));   /* inline encoder :59-71 == f32_to_f16 */
        for (int j = 0; j < 16; j++) {
            int32_t lo = sat_i32(roundf(blk[j * 2] * inv)) + 8;
            int32_t hi = sat_i32(roundf(blk[j * 2 + 1] * inv)) + 8;
            lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
            hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
            o[2 + j] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* LC/src/cpu/ops/q4_common.rs:104-170 — 148-byte Q4_K super-block:
 * [f16 d][f16 dmin][12 B scales, bytes 0..7 = 6-bit sc_j][4 B mins: min_j | min_{j+4}<<4][128 B nibbles] */
void lo_quantize_q4_k(const float* x, size_t n, uint8_t* out) {
    size_t nsb = n / 256;
    for (size_t sb = 0; sb < nsb; sb++) {
        const float* blk = x + sb * 256;
        uint8_t* o = out + sb * 148;
        float sub_min[8], sub_max[8];
        for (int j = 0; j < 8; j++) {
            float mn = INFINITY, mx = -INFINITY;
            for (int i = 0; i < 32; i++) {
                mn = fminf(mn, blk[j * 32 + i]);
                mx = fmaxf(mx, blk[j * 32 + i]);
            }
            sub_min[j] = mn;
            sub_max[j] = mx;
        }
        float gmr = 0.0f, gmin = INFINITY;
        for (int j = 0; j < 8; j++) gmr = fmaxf(gmr, sub_max[j] - sub_min[j]);
        for (int j = 0; j < 8; j++) gmin = fminf(gmin, sub_min[j]);
        float d = gmr > 0.0f ? gmr / 63.0f : 0.0f;
        float dmin = gmin < 0.0f ? -gmin / 15.0f : 0.0f;
        wr_u16(o + 0, lo_f32_to_f16_trunc(d));
        wr_u16(o + 2, lo_f32_to_f16_trunc(dmin));
        uint8_t qs[8], qm[8];
        for (int j = 0; j < 8; j++) {
            float range = sub_max[j] - sub_min[j];
            qs[j] = d > 0.0f ? f_to_u8(clampf(roundf(range / d), 0.0f, 63.0f)) : 0;
            qm[j] = dmin > 0.0f ? f_to_u8(clampf(roundf(-sub_min[j] / dmin), 0.0f, 15.0f)) : 0;
        }
        memset(o + 4, 0, 12);
        for (int j = 0; j < 8; j++) o[4 + j] = qs[j] & 0x3F;
        for (int j = 0; j < 4; j++) o[16 + j] = (uint8_t)((qm[j] & 0x0F) | ((qm[j + 4] & 0x0F) << 4));
        for (int j = 0; j < 8; j++) {
            float sc = d * (float)qs[j];
            float mn = dmin * (float)qm[j];
            float inv_sc = sc > 0.0f ? 1.0f / sc : 0.0f;
            const float* sub = blk + j * 32;
            for (int i = 0; i < 16; i++) {
                uint8_t v0 = f_to_u8(clampf(roundf((sub[i * 2] + mn) * inv_sc), 0.0f, 15.0f));
                uint8_t v1 = f_to_u8(clampf(roundf((sub[i * 2 + 1] + mn) * inv_sc), 0.0f, 15.0f));
                o[20 + j * 16 + i] = (uint8_t)(v0 | (v1 << 4));
            }
        }
    }
}

/* LC/src/cpu/ops/q4_common.rs:179-239 — 210-byte Q6_K super-block:
 * [128 B ql][64 B qh, 2 bits/elem sequential][16 x i8 scales][f16 d] */
void lo_quantize_q6_k(const float* x, size_t n, uint8_t* out) {
    size_t nsb = n / 256;
    for (size_t sb = 0; sb < nsb; sb++) {
        const float* blk = x + sb * 256;
        uint8_t* o = out + sb * 210;
        float amax = block_amax(blk, 256);
        float d = amax / 32.0f;
        int8_t sub_scales[16];
        for (int j = 0; j < 16; j++) {
            float sub_max = block_amax(blk + j * 16, 16);
            float sc = d > 0.0f ? sub_max / d : 0.0f;
            sub_scales[j] = f_to_i8(clampf(roundf(sc), -128.0f, 127.0f));
        }
        uint8_t q6[256];
        for (int j = 0; j < 16; j++) {
            float sc = d * (float)sub_scales[j];
            float inv_sc = fabsf(sc) > 1e-10f ? 1.0f / sc : 0.0f;
            for (int i = 0; i < 16; i++) {
                int idx = j * 16 + i;
                int8_t q = f_to_i8(clampf(roundf(blk[idx] * inv_sc), -32.0f, 31.0f));
                q6[idx] = (uint8_t)(q + 32);
            }
        }
        for (int i = 0; i < 128; i++) o[i] = (uint8_t)((q6[i * 2] & 0x0F) | ((q6[i * 2 + 1] & 0x0F) << 4));
        memset(o + 128, 0, 64);
        for (int i = 0; i < 256; i++) o[128 + i / 4] |= (uint8_t)(((q6[i] >> 4) & 0x03) << ((i % 4) * 2));
        for (int j = 0; j < 16; j++) o[192 + j] = (uint8_t)sub_scales[j];
        wr_u16(o + 208, lo_f32_to_f16_trunc(d));
    }
}

/* LC/src/cpu/ops/q8_matvec.rs:11-34 */
void lo_quantize_weights_q8(const float* w, size_t rows, size_t cols, int8_t* q8, float* scales) {
    size_t bpr = cols / 32;
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < bpr; b++) {
            size_t off = r * cols + b * 32;
            float amax = block_amax(w + off, 32);
            float scale = amax / 127.0f;
            float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
            scales[r * bpr + b] = scale;
            for (int j = 0; j < 32; j++)
                q8[off + j] = f_to_i8(clampf(roundf(w[off + j] * inv), -128.0f, 127.0f));
        }
}

/* ── matvecs ──────────────────────────────────────────────────────────── */

/* LC/csrc/q4_dot.c:169-199 — x86 scalar fallback, per-element float order. */
void lo_q4_0_matvec_x86(const uint8_t* q4, const int8_t* q8x, const float* q8s,
                        float* out, size_t rows, size_t hidden) {
    size_t bpr = hidden / 32, bytes = bpr * 18;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        const uint8_t* row = q4 + r * bytes;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t* blk = row + b * 18;
            float cs = lo_decode_f16(rd_u16(blk)) * q8s[b];
            const int8_t* xq = q8x + b * 32;
            for (int j = 0; j < 16; j++) {
                uint8_t byte = blk[2 + j];
                int lo_v = (byte & 0x0F) - 8;
                int hi_v = ((byte >> 4) & 0x0F) - 8;
                acc += (float)lo_v * (float)xq[j * 2] * cs;
                acc += (float)hi_v * (float)xq[j * 2 + 1] * cs;
            }
        }
        out[r] = acc;
    }
}

/* Per-block integer dot: isum_b = sum_j (nib_j - 8) * q8_j (LC/csrc/q4_dot.c:70-89). */
static int32_t q4_0_block_isum(const uint8_t* blk, const int8_t* xq) {
    int32_t s = 0;
    for (int j = 0; j < 16; j++) {
        uint8_t byte = blk[2 + j];
        s += ((byte & 0x0F) - 8) * (int32_t)xq[j * 2];
        s += (((byte >> 4) & 0x0F) - 8) * (int32_t)xq[j * 2 + 1];
    }
    return s;
}

/* LC/csrc/q4_dot.c:48-103 — ARM vdotq path (same order as the Metal q4_matvec_v4
 * kernel): acc += (float)isum_b * (f16(scale_b) * q8s_b), blocks in order. */
void lo_q4_0_matvec_blockint(const uint8_t* q4, const int8_t* q8x, const float* q8s,
                             float* out, size_t rows, size_t hidden) {
    size_t bpr = hidden / 32, bytes = bpr * 18;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        const uint8_t* row = q4 + r * bytes;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t* blk = row + b * 18;
            float cs = lo_decode_f16(rd_u16(blk)) * q8s[b];
            acc += (float)q4_0_block_isum(blk, q8x + b * 32) * cs;
        }
        out[r] = acc;
    }
}

void lo_q4_0_block_dots(const uint8_t* q4, const int8_t* q8x, int32_t* isum, size_t rows, size_t hidden) {
    size_t bpr = hidden / 32, bytes = bpr * 18;
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < bpr; b++)
            isum[r * bpr + b] = q4_0_block_isum(q4 + r * bytes + b * 18, q8x + b * 32);
}

/* LC/csrc/q4_dot.c:201-232 — scatter-accumulate, rows with |act| < 1e-10 skipped. */
void lo_q4_0_vecmat(const float* act, const uint8_t* q4, float* out, size_t inter, size_t hidden) {
    size_t bpr = hidden / 32, bytes = bpr * 18;
    for (size_t j = 0; j < hidden; j++) out[j] = 0.0f;
    for (size_t r = 0; r < inter; r++) {
        float a = act[r];
        if (a > -1e-10f && a < 1e-10f) continue;
        const uint8_t* row = q4 + r * bytes;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t* blk = row + b * 18;
            float scale = lo_decode_f16(rd_u16(blk)) * a;
            float* o = out + b * 32;
            for (int j = 0; j < 16; j++) {
                uint8_t byte = blk[2 + j];
                int lo_v = (byte & 0x0F) - 8;
                int hi_v = ((byte >> 4) & 0x0F) - 8;
                o[j * 2] += (float)lo_v * scale;
                o[j * 2 + 1] += (float)hi_v * scale;
            }
        }
    }
}

/* LC/src/cpu/ops/q4k_matvec.rs:31-90 — sequential f32: acc += (sc*q - mn) * x. */
void lo_q4k_matvec(const uint8_t* q4k, const float* x, float* out, size_t rows, size_t hidden) {
    size_t nsb = hidden / 256, bytes = nsb * 148;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = q4k + r * bytes + sb * 148;
            float d = lo_f16_to_f32(rd_u16(blk));
            float dmin = lo_f16_to_f32(rd_u16(blk + 2));
            float scales[8], mins[8];
            for (int j = 0; j < 4; j++) {
                scales[j] = (float)(blk[4 + j] & 0x3F);
                scales[j + 4] = (float)(blk[4 + j + 4] & 0x3F);
                mins[j] = (float)(blk[16 + j] & 0x0F);
                mins[j + 4] = (float)((blk[16 + j] >> 4) & 0x0F);
            }
            const uint8_t* qs = blk + 20;
            size_t xb = sb * 256;
            for (int j = 0; j < 8; j++) {
                float sc = d * scales[j];
                float mn = dmin * mins[j];
                for (int i = 0; i < 16; i++) {
                    uint8_t q = qs[j * 16 + i];
                    size_t xi = xb + j * 32 + i * 2;
                    float lo = (float)(q & 0x0F), hi = (float)((q >> 4) & 0x0F);
                    acc += (sc * lo - mn) * x[xi];
                    acc += (sc * hi - mn) * x[xi + 1];
                }
            }
        }
        out[r] = acc;
    }
}

/* LC/src/cpu/ops/q6k_matvec.rs:31-90 — val = sc * ((lo4 + 16*hi2) - 32). */
void lo_q6k_matvec(const uint8_t* q6k, const float* x, float* out, size_t rows, size_t hidden) {
    size_t nsb = hidden / 256, bytes = nsb * 210;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = q6k + r * bytes + sb * 210;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const uint8_t* scales = blk + 192;
            float d = lo_f16_to_f32(rd_u16(blk + 208));
            size_t xb = sb * 256;
            for (int j = 0; j < 16; j++) {
                float sc = d * (float)(int8_t)scales[j];
                for (int i = 0; i < 8; i++) {
                    int qi = j * 16 + i * 2;
                    uint8_t lo_byte = ql[qi / 2];
                    float lo4_0 = (float)(lo_byte & 0x0F);
                    float lo4_1 = (float)((lo_byte >> 4) & 0x0F);
                    float hi2_0 = (float)((qh[qi / 4] >> ((qi % 4) * 2)) & 0x03);
                    float hi2_1 = (float)((qh[(qi + 1) / 4] >> (((qi + 1) % 4) * 2)) & 0x03);
                    float v0 = sc * ((lo4_0 + hi2_0 * 16.0f) - 32.0f);
                    float v1 = sc * ((lo4_1 + hi2_1 * 16.0f) - 32.0f);
                    acc += v0 * x[xb + qi];
                    acc += v1 * x[xb + qi + 1];
                }
            }
        }
        out[r] = acc;
    }
}

/* ── Q4_KF: GGUF 144-byte (llama.cpp layout) and 160-byte pre-baked ─────── */

/* llama.cpp get_scale_min_k4 (the unpack of LM/src/quant/ggml.rs:252-262 and of the
 * uint16 masks of LC/src/metal/shaders/q4kf_qkv_proj.rs:93-97). */
void lo_gguf_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* Element e of a llama.cpp block: chunk c = e / 64 of 32 bytes; the first 32 elements of a
 * chunk are the low nibbles (sub-block 2c), the next 32 the high nibbles (2c + 1). */
static int gguf_nibble(const uint8_t* qs, int e) {
    int c = e / 64, l = e % 64;
    return l < 32 ? (qs[32 * c + l] & 0xF) : (qs[32 * c + l - 32] >> 4);
}

void lo_q4kf_gguf_matvec(const uint8_t* w, const float* x, float* out, size_t rows, size_t hidden) {
    size_t nsb = hidden / 256, bytes = nsb * 144;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = w + r * bytes + sb * 144;
            float d = lo_f16_to_f32(rd_u16(blk)), dmin = lo_f16_to_f32(rd_u16(blk + 2));
            for (int e = 0; e < 256; e++) {
                int j = e / 32;
                uint8_t sc, mn;
                lo_gguf_scale_min(j, blk + 4, &sc, &mn);
                float s = d * (float)sc, m = dmin * (float)mn;
                acc += (s * (float)gguf_nibble(blk + 16, e) - m) * x[sb * 256 + e];
            }
        }
        out[r] = acc;
    }
}

void lo_q4kf160_matvec(const uint8_t* w, const float* x, float* out, size_t rows, size_t hidden) {
    size_t nsb = hidden / 256, bytes = nsb * 160;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = w + r * bytes + sb * 160;
            for (int j = 0; j < 8; j++) {
                float s = lo_f16_to_f32(rd_u16(blk + 2 * j)), m = lo_f16_to_f32(rd_u16(blk + 16 + 2 * j));
                for (int i = 0; i < 16; i++) {
                    uint8_t q = blk[32 + j * 16 + i];
                    size_t xi = sb * 256 + j * 32 + i * 2;
                    acc += (s * (float)(q & 0x0F) - m) * x[xi];
                    acc += (s * (float)((q >> 4) & 0x0F) - m) * x[xi + 1];
                }
            }
        }
        out[r] = acc;
    }
}

/* The reference's 12-byte packing of 6-bit scales and mins (q4_common.rs:285-296, 343-352). */
static void ref_gguf_pack(const uint8_t* sc, const uint8_t* mn, uint8_t* p) {
    for (int j = 0; j < 4; j++) {
        p[j] = (uint8_t)((sc[j] & 0x3F) | ((mn[j] & 0x03) << 6));
        p[j + 4] = (uint8_t)((sc[j + 4] & 0x3F) | ((mn[j + 4] & 0x03) << 6));
    }
    for (int j = 0; j < 4; j++)
        p[8 + j] = (uint8_t)(((mn[2 * j] >> 2) & 0x0F) | (((mn[2 * j + 1] >> 2) & 0x0F) << 4));
}

/* LC/src/cpu/ops/q4_common.rs:321-361 */
void lo_q4k_to_gguf(const uint8_t* q4k, size_t nblocks, uint8_t* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = q4k + b * 148;
        uint8_t* o = out + b * 144;
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 4; j++) {
            sc[j] = blk[4 + j] & 0x3F;
            sc[j + 4] = blk[8 + j] & 0x3F;
            mn[j] = blk[16 + j] & 0x0F;
            mn[j + 4] = (blk[16 + j] >> 4) & 0x0F;
        }
        memcpy(o, blk, 4);
        ref_gguf_pack(sc, mn, o + 4);
        memcpy(o + 16, blk + 20, 128);
    }
}

/* LC/src/cpu/ops/q4_common.rs:248-314 (dmin = -gmin / 63 and 6-bit mins). */
void lo_quantize_q4_k_gguf(const float* x, size_t n, uint8_t* out) {
    size_t nsb = n / 256;
    for (size_t sb = 0; sb < nsb; sb++) {
        const float* blk = x + sb * 256;
        uint8_t* o = out + sb * 144;
        float sub_min[8], sub_max[8];
        for (int j = 0; j < 8; j++) {
            float mnv = INFINITY, mxv = -INFINITY;
            for (int i = 0; i < 32; i++) {
                mnv = fminf(mnv, blk[j * 32 + i]);
                mxv = fmaxf(mxv, blk[j * 32 + i]);
            }
            sub_min[j] = mnv;
            sub_max[j] = mxv;
        }
        float gmr = 0.0f, gmin = INFINITY;
        for (int j = 0; j < 8; j++) gmr = fmaxf(gmr, sub_max[j] - sub_min[j]);
        for (int j = 0; j < 8; j++) gmin = fminf(gmin, sub_min[j]);
        float d = gmr > 0.0f ? gmr / 63.0f : 0.0f;
        float dmin = gmin < 0.0f ? -gmin / 63.0f : 0.0f;
        uint8_t qs[8], qm[8];
        for (int j = 0; j < 8; j++) {
            float range = sub_max[j] - sub_min[j];
            qs[j] = d > 0.0f ? f_to_u8(clampf(roundf(range / d), 0.0f, 63.0f)) : 0;
            qm[j] = dmin > 0.0f ? f_to_u8(clampf(roundf(-sub_min[j] / dmin), 0.0f, 63.0f)) : 0;
        }
        wr_u16(o + 0, lo_f32_to_f16_trunc(d));
        wr_u16(o + 2, lo_f32_to_f16_trunc(dmin));
        ref_gguf_pack(qs, qm, o + 4);
        for (int j = 0; j < 8; j++) {
            float sc = d * (float)qs[j];
            float mn = dmin * (float)qm[j];
            float inv_sc = sc > 0.0f ? 1.0f / sc : 0.0f;
            const float* sub = blk + j * 32;
            for (int i = 0; i < 16; i++) {
                uint8_t v0 = f_to_u8(clampf(roundf((sub[i * 2] + mn) * inv_sc), 0.0f, 15.0f));
                uint8_t v1 = f_to_u8(clampf(roundf((sub[i * 2 + 1] + mn) * inv_sc), 0.0f, 15.0f));
                o[16 + j * 16 + i] = (uint8_t)(v0 | (v1 << 4));
            }
        }
    }
}

/* LC/src/cpu/ops/q4_common.rs:370-413 */
void lo_q4k_to_q4kf(const uint8_t* q4k, size_t nblocks, uint8_t* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = q4k + b * 148;
        uint8_t* o = out + b * 160;
        float d = lo_f16_to_f32(rd_u16(blk)), dmin = lo_f16_to_f32(rd_u16(blk + 2));
        for (int j = 0; j < 4; j++) {
            wr_u16(o + 2 * j, lo_f32_to_f16_trunc(d * (float)(blk[4 + j] & 0x3F)));
            wr_u16(o + 2 * (j + 4), lo_f32_to_f16_trunc(d * (float)(blk[8 + j] & 0x3F)));
            wr_u16(o + 16 + 2 * j, lo_f32_to_f16_trunc(dmin * (float)(blk[16 + j] & 0x0F)));
            wr_u16(o + 16 + 2 * (j + 4), lo_f32_to_f16_trunc(dmin * (float)((blk[16 + j] >> 4) & 0x0F)));
        }
        memcpy(o + 32, blk + 20, 128);
    }
}

/* 148 -> llama.cpp 144: scales and mins in the get_scale_min_k4 packing, nibbles moved so
 * that element 32j + l of sub-block j = 2c + h sits in nibble h of byte 32c + l. */
void lo_q4k_to_gguf_llamacpp(const uint8_t* q4k, size_t nblocks, uint8_t* out) {
    for (size_t b = 0; b < nblocks; b++) {
        const uint8_t* blk = q4k + b * 148;
        uint8_t* o = out + b * 144;
        uint8_t sc[8], mn[8];
        for (int j = 0; j < 4; j++) {
            sc[j] = blk[4 + j] & 0x3F;
            sc[j + 4] = blk[8 + j] & 0x3F;
            mn[j] = blk[16 + j] & 0x0F;
            mn[j + 4] = (blk[16 + j] >> 4) & 0x0F;
        }
        memcpy(o, blk, 4);
        uint8_t* p = o + 4;
        for (int j = 0; j < 4; j++) {
            p[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            p[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
            p[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
        }
        memset(o + 16, 0, 128);
        for (int e = 0; e < 256; e++) {
            int j = e / 32, i = e % 32;
            uint8_t byte = blk[20 + j * 16 + i / 2];
            int q = (i & 1) ? (byte >> 4) : (byte & 0xF);
            int c = j / 2, h = j % 2;
            o[16 + 32 * c + i] |= (uint8_t)(q << (4 * h));
        }
    }
}

/* LC/src/metal/shaders/q4_f32_matvec.rs:10-38 */
void lo_q4_0_f32_matvec(const uint8_t* q4, const float* x, float* out, size_t rows, size_t hidden) {
    size_t bpr = hidden / 32, bytes = bpr * 18;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            const uint8_t* blk = q4 + r * bytes + b * 18;
            float scale = lo_decode_f16(rd_u16(blk));
            const float* xb = x + b * 32;
            float block_sum = 0.0f;
            for (int j = 0; j < 16; j++) {
                uint8_t byte = blk[2 + j];
                float lo = (float)((int)(byte & 0x0F) - 8), hi = (float)((int)(byte >> 4) - 8);
                block_sum += lo * xb[j * 2] + hi * xb[j * 2 + 1];
            }
            acc += block_sum * scale;
        }
        out[r] = acc;
    }
}

/* LC/src/cpu/ops/q8_matvec.rs:36-62 */
void lo_q8_matvec(const int8_t* wq, const float* ws, const int8_t* xq, const float* xs,
                  float* out, size_t rows, size_t hidden) {
    size_t nb = hidden / 32;
    for (size_t r = 0; r < rows; r++) {
        float acc = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            float cs = ws[r * nb + b] * xs[b];
            const int8_t* w = wq + r * hidden + b * 32;
            const int8_t* v = xq + b * 32;
            int32_t isum = 0;
            for (int j = 0; j < 32; j++) isum += (int32_t)w[j] * (int32_t)v[j];
            acc += (float)isum * cs;
        }
        out[r] = acc;
    }
}

void lo_q8_block_dots(const int8_t* wq, const int8_t* xq, int32_t* isum, size_t rows, size_t hidden) {
    size_t nb = hidden / 32;
    for (size_t r = 0; r < rows; r++)
        for (size_t b = 0; b < nb; b++) {
            int32_t s = 0;
            for (int j = 0; j < 32; j++) s += (int32_t)wq[r * hidden + b * 32 + j] * (int32_t)xq[b * 32 + j];
            isum[r * nb + b] = s;
        }
}

/* ── gate KNN ─────────────────────────────────────────────────────────── */

typedef struct { float key; uint32_t idx; float val; } lo_cand_t;

static int cand_cmp(const void* a, const void* b) {
    const lo_cand_t* x = (const lo_cand_t*)a;
    const lo_cand_t* y = (const lo_cand_t*)b;
    if (x->key > y->key) return -1;
    if (x->key < y->key) return 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx ? 1 : 0);
}

static void topk_by_key(const float* s, size_t n, size_t k, int use_abs, uint32_t* idx, float* val) {
    lo_cand_t* c = (lo_cand_t*)malloc(n * sizeof(lo_cand_t));
    for (size_t i = 0; i < n; i++) {
        c[i].key = use_abs ? fabsf(s[i]) : s[i];
        c[i].idx = (uint32_t)i;
        c[i].val = s[i];
    }
    qsort(c, n, sizeof(lo_cand_t), cand_cmp);
    if (k > n) k = n;
    for (size_t i = 0; i < k; i++) { idx[i] = c[i].idx; val[i] = c[i].val; }
    free(c);
}

/* LV/src/index/gate.rs:307-316 — select_nth_unstable_by + sort_unstable_by on |score|
 * descending.  The reference leaves ties unordered; the oracle orders them by index. */
void lo_topk_abs(const float* scores, size_t n, size_t k, uint32_t* idx, float* val) {
    topk_by_key(scores, n, k, 1, idx, val);
}

/* LV/src/index/walk.rs:563-580 — same selection on the signed score (lm-head KNN). */
void lo_topk_signed(const float* scores, size_t n, size_t k, uint32_t* idx, float* val) {
    topk_by_key(scores, n, k, 0, idx, val);
}

/* f32 gate scores (LV/src/index/gate.rs:14-29 computes gate[N,h] x q[h]); the
 * reference hands the order to matrixmultiply, so the oracle fixes one: a single
 * fmaf chain over k, which the HIP kernel reproduces bit for bit. */
void lo_gate_scores_f32(const float* gate, const float* x, float* out, size_t features, size_t hidden) {
    for (size_t f = 0; f < features; f++) {
        float acc = 0.0f;
        const float* g = gate + f * hidden;
        for (size_t k = 0; k < hidden; k++) acc = fmaf(g[k], x[k], acc);
        out[f] = acc;
    }
}

/* ── decode-step numerics ─────────────────────────────────────────────── */

/* LI/src/residual.rs:17-33 — f64 sum of squares, rms cast to f32, x / rms * (offset + w). */
void lo_rms_norm(const float* x, const float* w, float offset, double eps, float* out, size_t n) {
    double sq = 0.0;
    for (size_t i = 0; i < n; i++) sq += (double)x[i] * (double)x[i];
    float rms = (float)sqrt(sq / (double)n + eps);
    for (size_t i = 0; i < n; i++) {
        float wt = w ? offset + w[i] : 1.0f;
        out[i] = x[i] / rms * wt;
    }
}

/* LI/src/attention/rope.rs:22-55 — split-half pairs (i, i+half), f64 angles. */
void lo_rope_at(float* x, size_t num_heads, size_t head_dim, size_t rotary_dim, double base, size_t pos) {
    size_t half = rotary_dim / 2;
    for (size_t h = 0; h < num_heads; h++) {
        float* v = x + h * head_dim;
        for (size_t i = 0; i < half; i++) {
            double inv_freq = 1.0 / pow(base, 2.0 * (double)i / (double)rotary_dim);
            double theta = (double)pos * inv_freq;
            float c = (float)cos(theta), s = (float)sin(theta);
            float x0 = v[i], x1 = v[half + i];
            v[i] = x0 * c - x1 * s;
            v[half + i] = x0 * s + x1 * c;
        }
    }
}

/* LI/src/ffn/mod.rs:87-94 — silu(g) * u with sigmoid = 1 / (1 + exp(-g)). */
void lo_silu_gate_up(const float* gate, const float* up, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        float g = gate[i];
        float sig = 1.0f / (1.0f + expf(-g));
        out[i] = (g * sig) * up[i];
    }
}

/* LI/src/ffn/mod.rs:96-103 — gelu_tanh(g) * u with
 * gelu_tanh(x) = 0.5 x (1 + tanh(0.7978846 (x + 0.044715 x^3))), all in f32. */
void lo_gelu_tanh_gate_up(const float* gate, const float* up, float* out, size_t n) {
    const float c = 0.7978846f;
    for (size_t i = 0; i < n; i++) {
        float x = gate[i];
        float inner = c * (x + 0.044715f * x * x * x);
        out[i] = (0.5f * x * (1.0f + tanhf(inner))) * up[i];
    }
}

/* LI/src/residual.rs:86-110 — per head: rms = sqrt(sum(f64 x^2)/hd + eps) as f32, x / rms. */
void lo_rms_norm_heads(float* x, size_t num_heads, size_t head_dim, double eps) {
    for (size_t h = 0; h < num_heads; h++) {
        float* v = x + h * head_dim;
        double sq = 0.0;
        for (size_t d = 0; d < head_dim; d++) sq += (double)v[d] * (double)v[d];
        float rms = (float)sqrt(sq / (double)head_dim + eps);
        for (size_t d = 0; d < head_dim; d++) v[d] = v[d] / rms;
    }
}

/* LI/src/attention/gqa.rs:29-110, last query row only: s = (k.q) * scale;
 * e = exp((s - max) as f64); sum in f64; p = (e as f32) * ((1/sum) as f32); out = V^T p.
 * K/V come from a cache [t][kv_head][head_dim] of fp16 (lo_attend_heads) or f32
 * (lo_attend_heads32) elements; kv_h = h / (num_q / num_kv). */
/* Query heads [h0, h1): scores, softmax in f64, then the weighted V sum with t outermost
 * (each output element still accumulates its T terms in ascending t, the same additions
 * as a t-inner loop, while V is walked row by row). */
#define LO_ATTEND_HEADS(NAME, ELEM, LOAD)                                                                    \
    static void NAME(const float* q, const ELEM* kc, const ELEM* vc, size_t T, size_t h0, size_t h1,          \
                     size_t reps, size_t kvd, size_t head_dim, float scale, float softcap, float* out) {     \
        float* sc = (float*)malloc(T * sizeof(float));                                                        \
        for (size_t h = h0; h < h1; h++) {                                                                    \
            size_t kvh = h / reps;                                                                            \
            const float* qh = q + h * head_dim;                                                               \
            for (size_t t = 0; t < T; t++) {                                                                  \
                const ELEM* kr = kc + t * kvd + kvh * head_dim;                                               \
                float dot = 0.0f;                                                                             \
                for (size_t d = 0; d < head_dim; d++) dot += LOAD(kr[d]) * qh[d];                             \
                sc[t] = dot * scale;                                                                          \
                if (softcap > 0.0f) sc[t] = tanhf(sc[t] / softcap) * softcap; /* fused_attention.rs:132-137 */\
            }                                                                                                 \
            float mx = -INFINITY;                                                                             \
            for (size_t t = 0; t < T; t++) mx = fmaxf(mx, sc[t]);                                             \
            double sum = 0.0;                                                                                 \
            for (size_t t = 0; t < T; t++) {                                                                  \
                double e = exp((double)(sc[t] - mx));                                                         \
                sc[t] = (float)e;                                                                             \
                sum += e;                                                                                     \
            }                                                                                                 \
            float inv = (float)(1.0 / sum);                                                                   \
            for (size_t t = 0; t < T; t++) sc[t] *= inv;                                                      \
            float* oh = out + h * head_dim;                                                                   \
            for (size_t d = 0; d < head_dim; d++) oh[d] = 0.0f;                                               \
            for (size_t t = 0; t < T; t++) {                                                                  \
                const ELEM* vr = vc + t * kvd + kvh * head_dim;                                               \
                for (size_t d = 0; d < head_dim; d++) oh[d] += LOAD(vr[d]) * sc[t];                           \
            }                                                                                                 \
        }                                                                                                     \
        free(sc);                                                                                             \
    }
#define LO_F32_ELEM(x) (x)
LO_ATTEND_HEADS(lo_attend_heads, uint16_t, lo_f16_to_f32)
LO_ATTEND_HEADS(lo_attend_heads32, float, LO_F32_ELEM)

void lo_attend_f16(const float* q, const uint16_t* kc, const uint16_t* vc, size_t T,
                   size_t num_q, size_t num_kv, size_t head_dim, float scale, float* out) {
    lo_attend_heads(q, kc, vc, T, 0, num_q, num_q / num_kv, num_kv * head_dim, head_dim, scale, 0.0f, out);
}

/* LC/src/metal/shaders/fused_attention.rs:79-88: s = sum of squares in element order
 * (f32), every element times rsqrt(s + 1e-6). */
void lo_qk_norm_heads(float* x, size_t num_heads, size_t head_dim) {
    for (size_t h = 0; h < num_heads; h++) {
        float* v = x + h * head_dim;
        float s = 0.0f;
        for (size_t d = 0; d < head_dim; d++) s += v[d] * v[d];
        const float r = 1.0f / sqrtf(s + 1e-6f);
        for (size_t d = 0; d < head_dim; d++) v[d] *= r;
    }
}

void lo_attend_f16_opts(const float* q, const uint16_t* kc, const uint16_t* vc, size_t T, size_t num_q,
                        size_t num_kv, size_t head_dim, float scale, int qk_norm, float softcap, float* out) {
    float* qn = (float*)malloc(num_q * head_dim * sizeof(float));
    memcpy(qn, q, num_q * head_dim * sizeof(float));
    if (qk_norm) lo_qk_norm_heads(qn, num_q, head_dim);
    lo_attend_heads(qn, kc, vc, T, 0, num_q, num_q / num_kv, num_kv * head_dim, head_dim, scale, softcap, out);
    free(qn);
}

/* A projection in its layer's format: Q4_K (0), Q6_K (1), Q4_KF 144-byte GGUF (2), Q4_KF
 * 160-byte (3), Q8_0 (4: int8 weights + f32 scales ws, input quantized by quantize_to_q8) or
 * Q4_0 (5: q8in = 1 quantizes the input and runs the block matvec, q8in = 0 the f32-input
 * matvec of the reference's down projection). */
static void lo_proj_q(int fmt, const uint8_t* w, const float* ws, int q8in, const float* x, float* out, size_t rows,
                      size_t cols) {
    if (fmt == 4 || (fmt == 5 && q8in)) {
        int8_t* q8 = (int8_t*)malloc(cols);
        float* q8s = (float*)malloc(cols / 32 * sizeof(float));
        lo_quantize_to_q8(x, cols, q8, q8s);
        if (fmt == 4) lo_q8_matvec((const int8_t*)w, ws, q8, q8s, out, rows, cols);
        else lo_q4_0_matvec_blockint(w, q8, q8s, out, rows, cols);
        free(q8);
        free(q8s);
    } else if (fmt == 5) {
        lo_q4_0_f32_matvec(w, x, out, rows, cols);
    } else if (fmt == 1) {
        lo_q6k_matvec(w, x, out, rows, cols);
    } else if (fmt == 2) {
        lo_q4kf_gguf_matvec(w, x, out, rows, cols);
    } else if (fmt == 3) {
        lo_q4kf160_matvec(w, x, out, rows, cols);
    } else {
        lo_q4k_matvec(w, x, out, rows, cols);
    }
}

/* Row-split drivers for the CPU baselines: rows of a projection go to threads in
 * contiguous slices and each slice runs the one-thread kernel, so the output equals the
 * one-thread output bit for bit (rows are independent). */
static size_t lo_fmt_row_bytes(int fmt, size_t cols) {
    switch (fmt) {
        case 1: return cols / 256 * 210;
        case 2: return cols / 256 * 144;
        case 3: return cols / 256 * 160;
        case 4: return cols;
        case 5: return cols / 32 * 18;
        default: return cols / 256 * 148;
    }
}

typedef struct {
    int fmt, q8in;
    const uint8_t* w;
    const float *ws, *x;
    float* out;
    size_t rows, cols;
} lo_proj_job;

static void* lo_proj_job_run(void* p) {
    const lo_proj_job* j = (const lo_proj_job*)p;
    if (j->rows) lo_proj_q(j->fmt, j->w, j->ws, j->q8in, j->x, j->out, j->rows, j->cols);
    return NULL;
}

static void lo_proj_n(int nt, int fmt, const uint8_t* w, const float* ws, int q8in, const float* x, float* out,
                      size_t rows, size_t cols) {
    if (nt <= 1 || rows < (size_t)nt) {
        lo_proj_q(fmt, w, ws, q8in, x, out, rows, cols);
        return;
    }
    if (nt > 256) nt = 256;
    pthread_t th[256];
    int started[256];
    lo_proj_job jb[256];
    const size_t rb = lo_fmt_row_bytes(fmt, cols);
    for (int t = 0; t < nt; t++) {
        const size_t r0 = rows * (size_t)t / (size_t)nt, r1 = rows * (size_t)(t + 1) / (size_t)nt;
        jb[t] = (lo_proj_job){fmt, q8in, w + r0 * rb, ws ? ws + r0 * (cols / 32) : NULL, x, out + r0, r1 - r0, cols};
        started[t] = pthread_create(&th[t], NULL, lo_proj_job_run, &jb[t]) == 0;
        if (!started[t]) lo_proj_job_run(&jb[t]);
    }
    for (int t = 0; t < nt; t++)
        if (started[t]) pthread_join(th[t], NULL);
}

typedef struct {
    const float* q;
    const uint16_t *kc, *vc;
    const float *kc32, *vc32;  /* non-NULL: the f32 cache */
    size_t T, h0, h1, reps, kvd, head_dim;
    float scale, softcap;
    float* out;
} lo_attend_job;

static void* lo_attend_job_run(void* p) {
    const lo_attend_job* j = (const lo_attend_job*)p;
    if (j->h1 <= j->h0) return NULL;
    if (j->kc32)
        lo_attend_heads32(j->q, j->kc32, j->vc32, j->T, j->h0, j->h1, j->reps, j->kvd, j->head_dim, j->scale,
                          j->softcap, j->out);
    else
        lo_attend_heads(j->q, j->kc, j->vc, j->T, j->h0, j->h1, j->reps, j->kvd, j->head_dim, j->scale, j->softcap,
                        j->out);
    return NULL;
}

/* Attention with the query heads split over nt threads (each head is independent); kc32 /
 * vc32 non-NULL: the f32 cache instead of kc / vc. */
static void lo_attend_n(int nt, const float* q, const uint16_t* kc, const uint16_t* vc, const float* kc32,
                        const float* vc32, size_t T, size_t num_q, size_t num_kv, size_t head_dim, float scale,
                        float softcap, float* out) {
    if (nt <= 1) {
        lo_attend_job j = {q, kc, vc, kc32, vc32, T, 0, num_q, num_q / num_kv, num_kv * head_dim, head_dim, scale,
                           softcap, out};
        lo_attend_job_run(&j);
        return;
    }
    if (nt > 256) nt = 256;
    pthread_t th[256];
    int started[256];
    lo_attend_job jb[256];
    for (int t = 0; t < nt; t++) {
        jb[t] = (lo_attend_job){q, kc, vc, kc32, vc32, T, num_q * (size_t)t / (size_t)nt,
                                num_q * (size_t)(t + 1) / (size_t)nt, num_q / num_kv, num_kv * head_dim, head_dim,
                                scale, softcap, out};
        started[t] = pthread_create(&th[t], NULL, lo_attend_job_run, &jb[t]) == 0;
        if (!started[t]) lo_attend_job_run(&jb[t]);
    }
    for (int t = 0; t < nt; t++)
        if (started[t]) pthread_join(th[t], NULL);
}

void lo_proj_rows_mt(int fmt, const uint8_t* w, const float* ws, int q8in, const float* x, float* out, size_t rows,
                     size_t cols, int nthreads) {
    lo_proj_n(nthreads, fmt, w, ws, q8in, x, out, rows, cols);
}

/* One decoder layer (LI/src/attention/block.rs:52-157, LI/src/forward/layer.rs:50-94; per-op
 * order of the reference GPU decode LC/src/metal/decode.rs:144-739):
 *   xn = norm(h, input_norm); q, k, v = projections; [V-norm]; RoPE(q, k) at pos;
 *   K/V appended at pos (LC/src/metal/ops/kv_cache.rs:73-105) as fp16 (RNE), or unrounded
 *   into the f32 cache (k_cache32); attention;
 *   o = Wo att;
 *   Llama:       h1 = h + o;                          f = norm(h1, post_attn_norm)
 *   post-norms:  h1 = h + norm(o, post_attn_norm);    f = norm(h1, pre_ffn_norm)
 *   a = act(gate f) * (up f); dn = Wd a;
 *   Llama:       h2 = h1 + dn;   post-norms: h2 = h1 + norm(dn, post_ffn_norm)
 *   layer_scalar != 0: h2 *= layer_scalar.
 * norm(x, w) = x / rms * (norm_offset + w) (LI/src/residual.rs:17-33); an absent
 * pre/post-FFN weight is the weight-free norm (LI/src/forward/layer.rs:65-68, 80-83). */
void lo_decode_layer(const lo_layer_t* L, float* h, size_t pos,
                     size_t hidden, size_t inter, size_t num_q, size_t num_kv, size_t head_dim,
                     double rope_base, double eps) {
    lo_decode_layer_window(L, h, pos, hidden, inter, num_q, num_kv, head_dim, rope_base, eps, 0);
}

/* Same, attending over the last `window` positions only when window > 0 and T = pos + 1
 * exceeds it: t_start = T - window (LC/src/metal/shaders/kv_attention.rs:35). */
static void lo_decode_layer_impl(const lo_layer_t* L, float* h, size_t pos, size_t hidden, size_t inter,
                                 size_t num_q, size_t num_kv, size_t head_dim, double rope_base, double eps,
                                 size_t window, int nt);

void lo_decode_layer_window(const lo_layer_t* L, float* h, size_t pos,
                            size_t hidden, size_t inter, size_t num_q, size_t num_kv, size_t head_dim,
                            double rope_base, double eps, size_t window) {
    lo_decode_layer_impl(L, h, pos, hidden, inter, num_q, num_kv, head_dim, rope_base, eps, window, 1);
}

/* The same layer with each projection's rows split over nthreads threads (identical
 * output; the CPU baseline's all-core decode). */
void lo_decode_layer_mt(const lo_layer_t* L, float* h, size_t pos, size_t hidden, size_t inter, size_t num_q,
                        size_t num_kv, size_t head_dim, double rope_base, double eps, int nthreads) {
    lo_decode_layer_impl(L, h, pos, hidden, inter, num_q, num_kv, head_dim, rope_base, eps, 0, nthreads);
}

static void lo_decode_layer_impl(const lo_layer_t* L, float* h, size_t pos, size_t hidden, size_t inter,
                                 size_t num_q, size_t num_kv, size_t head_dim, double rope_base, double eps,
                                 size_t window, int nt) {
    size_t qd = num_q * head_dim, kvd = num_kv * head_dim;
    const size_t rdim = L->rotary_dim ? L->rotary_dim : head_dim;
    const float off = L->norm_offset;
    float* xn = (float*)malloc(hidden * sizeof(float));
    float* q = (float*)malloc(qd * sizeof(float));
    float* k = (float*)malloc(kvd * sizeof(float));
    float* v = (float*)malloc(kvd * sizeof(float));
    float* att = (float*)malloc(qd * sizeof(float));
    float* o = (float*)malloc(hidden * sizeof(float));
    float* g = (float*)malloc(inter * sizeof(float));
    float* u = (float*)malloc(inter * sizeof(float));
    float* a = (float*)malloc(inter * sizeof(float));

    lo_rms_norm(h, L->input_norm, off, eps, xn, hidden);
    lo_proj_n(nt, L->fmt[0], L->wq, L->wq_s, 1, xn, q, qd, hidden);
    lo_proj_n(nt, L->fmt[1], L->wk, L->wk_s, 1, xn, k, kvd, hidden);
    lo_proj_n(nt, L->fmt[2], L->wv, L->wv_s, 1, xn, v, kvd, hidden);
    if (L->has_v_norm) lo_rms_norm_heads(v, num_kv, head_dim, eps);
    lo_rope_at(q, num_q, head_dim, rdim, rope_base, pos);
    lo_rope_at(k, num_kv, head_dim, rdim, rope_base, pos);
    if (L->qk_norm) lo_qk_norm_heads(q, num_q, head_dim);  /* after RoPE, Q only: the cache keeps K */
    const int f32kv = L->k_cache32 != NULL;
    for (size_t i = 0; i < kvd; i++) {
        if (f32kv) {
            L->k_cache32[pos * kvd + i] = k[i];
            L->v_cache32[pos * kvd + i] = v[i];
        } else {
            L->k_cache[pos * kvd + i] = lo_f32_to_f16_rne(k[i]);
            L->v_cache[pos * kvd + i] = lo_f32_to_f16_rne(v[i]);
        }
    }
    float scale = L->attn_scale != 0.0f ? L->attn_scale : (float)(1.0 / sqrt((double)head_dim));
    const size_t T = pos + 1, t0 = (window > 0 && T > window) ? T - window : 0;
    if (f32kv)
        lo_attend_n(nt, q, NULL, NULL, L->k_cache32 + t0 * kvd, L->v_cache32 + t0 * kvd, T - t0, num_q, num_kv,
                    head_dim, scale, L->softcap, att);
    else
        lo_attend_n(nt, q, L->k_cache + t0 * kvd, L->v_cache + t0 * kvd, NULL, NULL, T - t0, num_q, num_kv, head_dim,
                    scale, L->softcap, att);
    lo_proj_n(nt, L->fmt[3], L->wo, L->wo_s, 1, att, o, hidden, qd);
    if (L->has_post_norms) {
        lo_rms_norm(o, L->post_attn_norm, off, eps, xn, hidden);
        for (size_t i = 0; i < hidden; i++) h[i] = h[i] + xn[i];
        lo_rms_norm(h, L->pre_ffn_norm, off, eps, xn, hidden);
    } else {
        for (size_t i = 0; i < hidden; i++) h[i] = h[i] + o[i];
        lo_rms_norm(h, L->post_attn_norm, off, eps, xn, hidden);
    }
    lo_proj_n(nt, L->fmt[4], L->gate, L->gate_s, 1, xn, g, inter, hidden);
    lo_proj_n(nt, L->fmt[5], L->up, L->up_s, 1, xn, u, inter, hidden);
    if (L->activation == 1) lo_gelu_tanh_gate_up(g, u, a, inter);
    else lo_silu_gate_up(g, u, a, inter);
    lo_proj_n(nt, L->fmt[6], L->down, L->down_s, 0, a, o, hidden, inter);
    if (L->has_post_norms) {
        lo_rms_norm(o, L->post_ffn_norm, off, eps, xn, hidden);
        for (size_t i = 0; i < hidden; i++) h[i] = h[i] + xn[i];
    } else {
        for (size_t i = 0; i < hidden; i++) h[i] = h[i] + o[i];
    }
    if (L->layer_scalar != 0.0f)
        for (size_t i = 0; i < hidden; i++) h[i] = h[i] * L->layer_scalar;

    free(xn); free(q); free(k); free(v); free(att); free(o); free(g); free(u); free(a);
}

/* ── deterministic inputs ─────────────────────────────────────────────── */

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Gaussian samples: splitmix64 -> two uniforms in (0,1] -> Box-Muller in f64 -> f32. */
void lo_gauss_f32(uint64_t seed, float mean, float std, float* out, size_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = (double)((splitmix64(&s) >> 11) + 1) * 0x1.0p-53;
        double u2 = (double)((splitmix64(&s) >> 11) + 1) * 0x1.0p-53;
        double r = sqrt(-2.0 * log(u1));
        double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
        out[i] = (float)((double)mean + (double)std * z0);
        if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)std * z1);
    }
}
