"""Pins the CPU oracle (oracle/larql_oracle.c) before it is trusted as the checker.

What pins each oracle function (reference paths relative to larql-main/crates/):

  f16 decode (lo_f16_to_f32, lo_decode_f16)   all 65536 codes vs numpy's IEEE float16
                                              + ggml.rs:388-473 known answers; the two
                                              reference decoders agree bit for bit.
  f16 encode, truncating                      known answers (ggml.rs scales), monotone,
                                              round-toward-zero bracket vs numpy f16 grid.
  f16 encode, RNE (KV cache)                  bit-exact vs numpy astype(float16) (IEEE RNE).
  quantize_to_q8                              q4_common.rs:535-541 zero input; half-away
                                              rounding known answers; |q*s - x| <= s/2.
  quantize_q4_0                               q4_common.rs:545-569 sizes / zero block;
                                              per-element error <= scale/2 on ramps (pins
                                              the 2j/2j+1 nibble order and the f32 scale).
  q4_0 matvec / vecmat (x86 order)            BIT-EXACT vs the reference's own q4_dot.c
                                              compiled from its sources (oracle/_ref) and vs
                                              the committed golden outputs of that build.
  q4_0 matvec (int-block order)               exact integer block dots vs numpy int64 brute
                                              force; ggml.rs:388-418 element known answers.
  quantize_q4_k                               two hand-derived 148-byte super-blocks as literal
                                              bytes: d = gmr/63 and dmin = -gmin/15 with the
                                              truncating f16 (a case where nearest differs), the
                                              min nibble of sub-block j >= 4 in the high half,
                                              .5 ties of sc_j, m_j and q rounding half away.
  q4k_matvec                                  test_metal_shaders.rs:1301-1331 hand block
                                              (closed form); one-hot probes of hand-built
                                              blocks (closed form per element).
  quantize_q6_k                               a hand-derived 210-byte super-block as literal
                                              bytes (sub-scale .5 tie, qh bit placement, d =
                                              amax/32) and a truncating-f16 d case.
  q6k_matvec                                  test_metal_shaders.rs:1334-1361 hand block;
                                              one-hot probes of hand-built qh/ql/scale bytes.
  quantize_weights_q8 / q8_matvec             exact integer block dots vs numpy; the
                                              q8_matvec.rs:290-316 cosine > 0.999 check.
  top-k (abs / signed)                        test_vindex.rs:134-160 known answers; vs
                                              numpy stable argsort on random scores.
  gate_scores_f32 (canonical fma chain)       vs math.fsum-exact f64 dot within f32 bounds.
  rms_norm / silu / gelu / attention          closed forms: attention over T=1 returns V
                                              (LC/src/cpu/ops/attention.rs:66-75), equal keys
                                              give the mean of V; rms of output = 1;
                                              gelu_tanh vs f64 tanh; per-head norm by hand.
  rope_at                                     pos 0 = identity; pairs 1 and half-1 against
                                              theta = pos * base^(-2i/rdim) (full and partial
                                              rotary; pass-through past rdim).
  decode_layer                                a float64 restatement from dequantized weights
                                              (Llama layer; post-norm / offset / GELU / V-norm /
                                              scalar layer) within 1e-5, while each planted
                                              mistake (swapped norms, silu(up)*gate, dropped
                                              residual, RoPE on V, wrong RoPE exponent, wrong
                                              kv-head map) moves it by > 1e-2; zero weights
                                              leave h unchanged.
"""
import json
import math
import os

import numpy as np
import pytest

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def known():
    with open(os.path.join(GOLD, "known_answers.json")) as f:
        return json.load(f)


# ── f16 ───────────────────────────────────────────────────────────────────
def test_f16_decode_all_codes_match_ieee():
    codes = np.arange(65536, dtype=np.uint32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(c)) for c in codes], dtype=np.float32)
    got2 = np.array([oracle.decode_f16(int(c)) for c in codes], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and np.array_equal(np.isnan(got2), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.array_equal(got2[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_known_answers():
    for code, val in known()["f16"]["pairs"]:
        assert oracle.f16_to_f32(code) == np.float32(val)
        assert oracle.decode_f16(code) == np.float32(val)


def test_f16_trunc_encoder():
    assert oracle.f32_to_f16_trunc(1.0) == 0x3C00
    assert oracle.f32_to_f16_trunc(2.0) == 0x4000
    assert oracle.f32_to_f16_trunc(0.5) == 0x3800
    assert oracle.f32_to_f16_trunc(0.0) == 0 and oracle.f32_to_f16_trunc(-0.0) == 0x8000
    assert oracle.f32_to_f16_trunc(1e6) == 0x7C00            # overflow -> inf
    assert oracle.f32_to_f16_trunc(1e-6) == 0                 # f16 subnormal range flushed
    rng = np.random.default_rng(0)
    xs = np.exp(rng.uniform(np.log(6.2e-5), np.log(60000.0), 4000)).astype(np.float32)
    for x in xs:
        h = oracle.f32_to_f16_trunc(float(x))
        v = np.float32(np.uint16(h).view(np.float16))
        nxt = np.float32(np.nextafter(np.float16(v), np.float16(np.inf)))
        assert v <= x < nxt, (x, v, nxt)                      # round toward zero onto the f16 grid


def test_f16_rne_encoder_matches_numpy():
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 5, 20000).astype(np.float32),
        np.array([65519.0, 65520.0, 65504.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 6.1e-5, -0.0, 0.0], np.float32),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_rne(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ── Q8 activation quantizer ───────────────────────────────────────────────
def test_q8_zero_input():
    q, s = oracle.quantize_to_q8(np.zeros(known()["q8_zero_input"]["n"], np.float32))
    assert np.all(q == 0) and s[0] == 0.0


def test_q8_rounding_half_away_and_bound():
    x = np.zeros(32, np.float32)
    x[0] = 127.0      # scale = 1.0 exactly
    x[1], x[2], x[3], x[4] = 2.5, -2.5, 0.5, -126.5
    q, s = oracle.quantize_to_q8(x)
    assert s[0] == 1.0
    assert list(q[:5]) == [127, 3, -3, 1, -127]              # round half away from zero
    rng = np.random.default_rng(2)
    x = rng.standard_normal(4096).astype(np.float32)
    q, s = oracle.quantize_to_q8(x)
    err = np.abs(q.astype(np.float32) * np.repeat(s, 32) - x)
    assert np.all(err <= np.repeat(s, 32) * 0.5000001 + 1e-12)


# ── Q4_0 ──────────────────────────────────────────────────────────────────
def test_q4_0_sizes_and_zero_block():
    k = known()
    for n, nbytes in k["q4_0_sizes"]["cases"]:
        assert oracle.quantize_q4_0(np.ones(n, np.float32)).size == nbytes
    q = oracle.quantize_q4_0(np.zeros(32, np.float32))
    assert list(q[:2]) == k["q4_0_zero_input"]["scale_bytes"]
    assert np.all(q[2:] == k["q4_0_zero_input"]["nibble_byte"])
    with pytest.raises(ValueError, match="multiple of 32"):
        oracle.quantize_q4_0(np.ones(33, np.float32))


def _deq_q4_0(q4, n):
    blocks = q4.reshape(-1, 18)
    sc = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    nib = blocks[:, 2:]
    vals = np.empty((blocks.shape[0], 32), np.float32)
    vals[:, 0::2] = (nib & 15).astype(np.float32) - 8
    vals[:, 1::2] = (nib >> 4).astype(np.float32) - 8
    return (vals * sc[:, None]).reshape(-1)[:n]


def test_q4_0_roundtrip_error_bound():
    x = ((np.arange(32) - 16) * 0.5).astype(np.float32)            # q4_common.rs:571-595 ramp
    q = oracle.quantize_q4_0(x)
    d = _deq_q4_0(q, 32)
    scale = np.float32(np.uint16(int(q[0]) | (int(q[1]) << 8)).view(np.float16))
    assert np.max(np.abs(d - x)) <= scale * 0.5 + 1e-3               # reference bound is < 2.0
    rng = np.random.default_rng(3)
    x = rng.standard_normal(32 * 64).astype(np.float32)
    d = _deq_q4_0(oracle.quantize_q4_0(x), x.size)
    amax = np.abs(x.reshape(-1, 32)).max(1)
    assert np.all(np.abs(d - x).reshape(-1, 32).max(1) <= amax / 7 * 0.5 * 1.002 + 1e-6)


def _onehot_q8(k, n):
    q8 = np.zeros(n, np.int8)
    q8[k] = 1
    return q8, np.ones(n // 32, np.float32)


def test_q4_0_element_known_answers():
    k = known()
    blk = np.array(k["q4_0_basic"]["block"], np.uint8)
    for e, want in k["q4_0_basic"]["expect"].items():
        q8, s8 = _onehot_q8(int(e), 32)
        assert oracle.q4_0_matvec_blockint(blk, q8, s8, 1, 32)[0] == want
        assert oracle.q4_0_matvec_x86(blk, q8, s8, 1, 32)[0] == want
    blk = np.array(k["q4_0_zero_scale"]["block"], np.uint8)
    q8 = np.full(32, 5, np.int8)
    assert oracle.q4_0_matvec_x86(blk, q8, np.ones(1, np.float32), 1, 32)[0] == 0.0
    blks = np.array(k["q4_0_two_blocks"]["blocks"], np.uint8)
    for e, want in k["q4_0_two_blocks"]["expect"].items():
        q8, s8 = _onehot_q8(int(e), 64)
        assert oracle.q4_0_matvec_blockint(blks, q8, s8, 1, 64)[0] == want


def test_q4_0_against_reference_golden():
    g = np.load(os.path.join(GOLD, "q4_0_ref.npz"))
    for tag in ("small", "mid"):
        rows, hidden = int(g[f"{tag}_rows"]), int(g[f"{tag}_hidden"])
        out = oracle.q4_0_matvec_x86(g[f"{tag}_q4"], g[f"{tag}_q8"], g[f"{tag}_q8s"], rows, hidden)
        assert np.array_equal(out.view(np.uint32), g[f"{tag}_matvec_out"].view(np.uint32))
        # the recorded inputs are what the oracle's quantizers produce from the recorded x
        q8, s8 = oracle.quantize_to_q8(g[f"{tag}_x"])
        assert np.array_equal(q8, g[f"{tag}_q8"]) and np.array_equal(s8, g[f"{tag}_q8s"])
    q4 = oracle.quantize_q4_0(g["small_w"])
    assert np.array_equal(q4, g["small_q4"])
    out = oracle.q4_0_vecmat(g["vecmat_act"], g["vecmat_q4"], int(g["vecmat_inter"]), int(g["vecmat_hidden"]))
    assert np.array_equal(out.view(np.uint32), g["vecmat_out"].view(np.uint32))


def test_q4_0_against_compiled_reference_random():
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(4)
    for rows, hidden in ((33, 256), (128, 2560)):
        q4 = rng.integers(0, 256, rows * hidden // 32 * 18, dtype=np.uint8)
        q4.reshape(-1, 18)[:, 1] &= 0x3B                           # keep scales finite and modest
        q8 = rng.integers(-128, 128, hidden, dtype=np.int8)
        s8 = rng.uniform(0, 0.05, hidden // 32).astype(np.float32)
        a = oracle.q4_0_matvec_x86(q4, q8, s8, rows, hidden)
        b = oracle.ref_q4_0_matvec(q4, q8, s8, rows, hidden)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        act = rng.standard_normal(rows).astype(np.float32)
        act[::5] = 0.0
        a = oracle.q4_0_vecmat(act, q4, rows, hidden)
        b = oracle.ref_q4_0_vecmat(act, q4, rows, hidden)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4_0_block_dots_exact_and_blockint_close():
    rng = np.random.default_rng(5)
    rows, hidden = 40, 512
    q4 = oracle.quantize_q4_0(rng.standard_normal(rows * hidden).astype(np.float32))
    q8, s8 = oracle.quantize_to_q8(rng.standard_normal(hidden).astype(np.float32))
    isum = oracle.q4_0_block_dots(q4, q8, rows, hidden)
    blocks = q4.reshape(rows, hidden // 32, 18)[:, :, 2:]
    w = np.empty((rows, hidden // 32, 32), np.int64)
    w[:, :, 0::2] = (blocks & 15).astype(np.int64) - 8
    w[:, :, 1::2] = (blocks >> 4).astype(np.int64) - 8
    ref = (w * q8.astype(np.int64).reshape(1, -1, 32)).sum(-1)
    assert np.array_equal(isum, ref)
    deq = _deq_q4_0(q4, rows * hidden).reshape(rows, hidden).astype(np.float64)
    xd = q8.astype(np.float64) * np.repeat(s8, 32)
    ref_f = deq @ xd
    out = oracle.q4_0_matvec_blockint(q4, q8, s8, rows, hidden)
    assert np.max(np.abs(out - ref_f)) / np.max(np.abs(ref_f)) < 1e-5


# ── Q4_K ──────────────────────────────────────────────────────────────────
def _q4k_block(d=1.0, dmin=0.0, sc=(0,) * 8, mins=(0,) * 8, nib=None):
    b = np.zeros(148, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    for j in range(8):
        b[4 + j] = sc[j]
    for j in range(4):
        b[16 + j] = (mins[j] & 15) | ((mins[j + 4] & 15) << 4)
    if nib is not None:
        b[20:] = nib
    return b


def test_q4k_hand_block_closed_form():
    ka = known()["q4k_hand_block"]
    rows, hidden = 64, 256
    blk = _q4k_block(d=1.0, sc=(ka["scale0"],) + (0,) * 7, nib=np.full(128, ka["nibble_byte"], np.uint8))
    assert list(blk[:2]) == ka["d_bytes"]
    data = np.tile(blk, rows)
    x = np.sin(np.arange(hidden, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    out = oracle.q4k_matvec(data, x, rows, hidden)
    expect = np.float32(0.0)
    for v in x[:32]:
        expect = np.float32(expect + np.float32(1.0) * v)          # (sc*1 - 0) * x, sequential
    assert np.all(out == expect)


def test_q4k_onehot_probes_closed_form():
    # d = 0.5, dmin = 0.25, sc_j = j+1, min_j = 2j+1 (4-bit), nibble byte 20+16j+i = (i | (15-i)<<4)
    sc = tuple(j + 1 for j in range(8))
    mins = tuple(2 * j + 1 for j in range(8))
    nib = np.array([(i % 16) | ((15 - i % 16) << 4) for i in range(128)], np.uint8)
    blk = _q4k_block(d=0.5, dmin=0.25, sc=sc, mins=mins, nib=nib)
    for e in (0, 1, 2, 31, 32, 33, 100, 129, 254, 255):
        j, w = divmod(e, 32)
        i, hi = divmod(w, 2)
        q = (15 - i) if hi else i
        want = 0.5 * sc[j] * q - 0.25 * mins[j]
        x = np.zeros(256, np.float32)
        x[e] = 1.0
        assert oracle.q4k_matvec(blk, x, 1, 256)[0] == np.float32(want), e


def test_q4k_quantizer_layout_and_error():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(256 * 8) * 0.02).astype(np.float32)
    q = oracle.quantize_q4_k(x)
    assert q.size == 8 * 148
    b = q.reshape(8, 148)
    assert np.all(b[:, 12:16] == 0)                          # only bytes 0..7 of the scale area used
    assert np.all(b[:, 4:12] <= 63)
    # dequantize through the matvec with one-hot x: matches the per-element closed form
    for sb in range(2):
        blk = b[sb]
        d = np.float32(blk[0:2].copy().view(np.float16)[0])
        dmin = np.float32(blk[2:4].copy().view(np.float16)[0])
        for e in (0, 77, 200, 255):
            j = e // 32
            byte = blk[20 + j * 16 + (e % 32) // 2]
            qv = (byte >> 4) if e % 2 else (byte & 15)
            m = (blk[16 + j] & 15) if j < 4 else (blk[16 + j - 4] >> 4)
            want = np.float32(np.float32(d * np.float32(blk[4 + j])) * np.float32(qv)) - np.float32(dmin * np.float32(m))
            xx = np.zeros(256, np.float32)
            xx[e] = 1.0
            assert oracle.q4k_matvec(blk, xx, 1, 256)[0] == want
            # the reconstruction stays within one quantization step of the input
            step = float(d) * int(blk[4 + j]) + float(dmin) * 16
            assert abs(float(want) - float(x[sb * 256 + e])) <= step + 1e-6


# ── Q6_K ──────────────────────────────────────────────────────────────────
def test_q6k_hand_block_closed_form():
    ka = known()["q6k_hand_block"]
    rows, hidden = 64, 256
    blk = np.zeros(210, np.uint8)
    blk[208:210] = ka["d_bytes"]
    blk[192] = ka["scale0"]
    blk[:128] = ka["ql_byte"]
    data = np.tile(blk, rows)
    x = np.sin(np.arange(hidden, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    out = oracle.q6k_matvec(data, x, rows, hidden)
    expect = np.float32(0.0)
    for v in x[:16]:
        expect = np.float32(expect + np.float32(-29.0) * v)
    # sub-blocks 1..15 have sc = 0 and contribute exact zeros
    assert np.all(out == expect)


def test_q6k_onehot_probes_closed_form():
    blk = np.zeros(210, np.uint8)
    blk[:128] = (np.arange(128) * 37 % 256).astype(np.uint8)     # arbitrary low nibbles
    blk[128:192] = (np.arange(64) * 91 % 256).astype(np.uint8)  # arbitrary 2-bit pairs
    blk[192:208] = np.array([(-1) ** j * (j + 1) for j in range(16)], np.int8).view(np.uint8)
    blk[208:210] = np.array([0.125], np.float16).view(np.uint8)
    for e in (0, 1, 2, 3, 4, 15, 16, 17, 100, 127, 128, 200, 255):
        lo4 = (blk[e // 2] >> (4 * (e % 2))) & 15
        hi2 = (blk[128 + e // 4] >> (2 * (e % 4))) & 3
        sc = np.int8(blk[192 + e // 16].view(np.int8))
        want = np.float32(np.float32(0.125) * np.float32(sc)) * np.float32((lo4 + 16.0 * hi2) - 32.0)
        x = np.zeros(256, np.float32)
        x[e] = 1.0
        assert oracle.q6k_matvec(blk, x, 1, 256)[0] == want, e


def test_q6k_quantizer_layout_and_error():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(256 * 4) * 0.02).astype(np.float32)
    q = oracle.quantize_q6_k(x).reshape(4, 210)
    for sb in range(4):
        d = float(q[sb, 208:210].copy().view(np.float16)[0])
        amax = np.abs(x[sb * 256:(sb + 1) * 256]).max()
        assert abs(d - amax / 32) <= amax / 32 * 2 ** -10         # truncated f16 of amax/32
        for e in (0, 5, 130, 255):
            xx = np.zeros(256, np.float32)
            xx[e] = 1.0
            v = oracle.q6k_matvec(q[sb], xx, 1, 256)[0]
            sc = int(np.int8(q[sb, 192 + e // 16].view(np.int8)))
            assert abs(v - x[sb * 256 + e]) <= d * sc * 0.5 + d + 1e-7


# ── Q8 weights ───────────────────────────────────────────────────────────
def test_q8_matvec_exact_dots_and_cosine():
    rows, hidden = 32, 256                                      # q8_matvec.rs:290-316
    w = np.cos(np.arange(rows * hidden, dtype=np.float32) * np.float32(0.001)).astype(np.float32)
    x = np.sin(np.arange(hidden, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    wq, ws = oracle.quantize_weights_q8(w, rows, hidden)
    xq, xs = oracle.quantize_to_q8(x)
    isum = oracle.q8_block_dots(wq, xq, rows, hidden)
    ref = (wq.astype(np.int64).reshape(rows, -1, 32) * xq.astype(np.int64).reshape(1, -1, 32)).sum(-1)
    assert np.array_equal(isum, ref)
    out = oracle.q8_matvec(wq, ws, xq, xs, rows, hidden)
    f = w.reshape(rows, hidden).astype(np.float64) @ x.astype(np.float64)
    cos = np.dot(out, f) / (np.linalg.norm(out) * np.linalg.norm(f))
    assert cos > 0.999


# ── top-k ────────────────────────────────────────────────────────────────
def test_topk_known_answers():
    ka = known()["gate_knn_orthogonal"]
    gate0 = np.array(ka["gate0"], np.float32)
    for case in ka["cases"]:
        s = oracle.gate_scores_f32(gate0, np.array(case["query"], np.float32), 3, 4)
        idx, val = oracle.topk_abs(s, case["k"])
        if "idx" in case:
            assert list(idx) == case["idx"] and np.allclose(val, case["score"])
        else:
            assert list(idx[: len(case["idx_prefix"])]) == case["idx_prefix"]
    gate1 = np.array(ka["gate1"], np.float32)
    s = oracle.gate_scores_f32(gate1, np.array([0, 0, 1, 0], np.float32), 3, 4)
    idx, val = oracle.topk_abs(s, 1)
    assert idx[0] == 2 and val[0] == -1.0                      # |score| ranking keeps the sign


def test_topk_vs_numpy_stable_argsort():
    rng = np.random.default_rng(8)
    for n, k in ((10240, 32), (100, 100), (50, 7)):
        s = rng.standard_normal(n).astype(np.float32)
        s[::13] = s[1]                                          # force ties
        idx, val = oracle.topk_abs(s, k)
        ref = np.argsort(-np.abs(s), kind="stable")[:k]
        assert np.array_equal(idx, ref)
        idx, val = oracle.topk_signed(s, k)
        ref = np.argsort(-s, kind="stable")[:k]
        assert np.array_equal(idx, ref)


def test_gate_scores_canonical_chain():
    rng = np.random.default_rng(9)
    f, h = 16, 2560
    g = rng.standard_normal((f, h)).astype(np.float32)
    x = rng.standard_normal(h).astype(np.float32)
    s = oracle.gate_scores_f32(g, x, f, h)
    exact = np.array([math.fsum((g[i].astype(np.float64) * x.astype(np.float64)).tolist()) for i in range(f)])
    bound = h * 2.0 ** -24 * (np.abs(g).astype(np.float64) @ np.abs(x).astype(np.float64))
    assert np.all(np.abs(s - exact) <= bound)
    # a single fma chain from +0.0 in k order
    acc = np.float32(0.0)
    for k in range(h):
        acc = np.float32(np.float64(g[3, k]) * np.float64(x[k]) + np.float64(acc))  # fma == exact product then one rounding
    assert s[3] == acc


# ── decode numerics ──────────────────────────────────────────────────────
def test_rms_norm_properties():
    rng = np.random.default_rng(10)
    x = rng.standard_normal(4096).astype(np.float32) * 3
    y = oracle.rms_norm(x, np.ones(4096, np.float32))
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1.0) < 1e-5
    rms = np.float32(np.sqrt(np.sum(x.astype(np.float64) ** 2) / 4096 + 1e-6))
    assert np.array_equal(y, (x / rms) * np.float32(1.0))


def test_rope_closed_forms():
    rng = np.random.default_rng(11)
    x = rng.standard_normal(4 * 128).astype(np.float32)
    assert np.array_equal(oracle.rope_at(x, 4, 128, 500000.0, 0), x)        # pos 0 = identity
    y = oracle.rope_at(x, 4, 128, 500000.0, 2048)
    xv, yv = x.reshape(4, 2, 64), y.reshape(4, 2, 64)
    assert np.allclose(np.hypot(xv[:, 0], xv[:, 1]), np.hypot(yv[:, 0], yv[:, 1]), rtol=1e-5)
    # pair 0 has inv_freq = 1: rotation by exactly `pos` radians
    c, s = np.float32(math.cos(7.0)), np.float32(math.sin(7.0))
    y = oracle.rope_at(x, 4, 128, 500000.0, 7)
    assert y[0] == x[0] * c - x[64] * s and y[64] == x[0] * s + x[64] * c


def test_attention_closed_forms():
    rng = np.random.default_rng(12)
    nq, nkv, hd = 8, 2, 16
    q = rng.standard_normal(nq * hd).astype(np.float32)
    kc = rng.standard_normal(nkv * hd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(nkv * hd).astype(np.float16).view(np.uint16)
    out = oracle.attend_f16(q, kc, vc, 1, nq, nkv, hd, 0.25)
    v = vc.view(np.float16).astype(np.float32).reshape(nkv, hd)
    for h in range(nq):
        assert np.array_equal(out[h * hd:(h + 1) * hd], v[h // (nq // nkv)])   # T=1 returns V
    T = 5
    krow = rng.standard_normal(nkv * hd).astype(np.float16)
    kc = np.tile(krow, T).view(np.uint16)                                     # equal keys
    vs = rng.standard_normal(T * nkv * hd).astype(np.float16)
    out = oracle.attend_f16(q, kc, vs.view(np.uint16), T, nq, nkv, hd, 0.25)
    mean = vs.astype(np.float64).reshape(T, nkv, hd).mean(0)
    for h in range(nq):
        assert np.allclose(out[h * hd:(h + 1) * hd], mean[h // 4], rtol=1e-5, atol=1e-6)


def test_attention_window_closed_forms():
    """Sliding window (LC/src/metal/shaders/kv_attention.rs:35): a window of one position
    returns that position's V; a window covering the whole cache changes nothing; the
    window is the attention over the trailing slice of the cache."""
    rng = np.random.default_rng(13)
    nq, nkv, hd, T = 6, 2, 32, 9
    q = rng.standard_normal(nq * hd).astype(np.float32)
    kc = rng.standard_normal(T * nkv * hd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(T * nkv * hd).astype(np.float16).view(np.uint16)
    out = oracle.attend_f16(q, kc, vc, T, nq, nkv, hd, 0.2, t_start=T - 1)
    v_last = vc.view(np.float16).astype(np.float32).reshape(T, nkv, hd)[T - 1]
    for h in range(nq):
        assert np.array_equal(out[h * hd:(h + 1) * hd], v_last[h // 3])
    full = oracle.attend_f16(q, kc, vc, T, nq, nkv, hd, 0.2)
    assert np.array_equal(oracle.attend_f16(q, kc, vc, T, nq, nkv, hd, 0.2, t_start=0), full)
    # softmax over the window only: recompute in f64 from the raw rows
    t0 = 4
    k = kc.view(np.float16).astype(np.float64).reshape(T, nkv, hd)
    v = vc.view(np.float16).astype(np.float64).reshape(T, nkv, hd)
    win = oracle.attend_f16(q, kc, vc, T, nq, nkv, hd, 0.2, t_start=t0)
    for h in range(nq):
        s = k[t0:, h // 3] @ q[h * hd:(h + 1) * hd].astype(np.float64) * 0.2
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ v[t0:, h // 3]
        assert np.allclose(win[h * hd:(h + 1) * hd], ref, rtol=1e-5, atol=1e-6)


def test_attention_qk_norm_softcap_closed_forms():
    """Prompt-attention options (LC/src/metal/shaders/fused_attention.rs:79-88, 132-137) on two
    positions, where the softmax is the logistic function of the score difference: q = (3, 4,
    0, ..) has L2 norm 5; K rows 0 and (5, 0, ..), V rows 0 and e0, scale 0.5, so out[0] =
    1 / (1 + exp(-s1)) with s1 = 0.5 * 5 * q0 and, with QK-norm, q0 = 3 / sqrt(25 + 1e-6);
    with softcap c, s1 -> c * tanh(s1 / c).  The RMS norm in place of the L2 norm, the cap
    applied before the scale, or the cap without its factor c each miss by > 1e-2."""
    hd = 32
    q = np.zeros(hd, np.float32)
    q[:2] = (3.0, 4.0)
    kc = np.zeros(2 * hd, np.float16)
    kc[hd] = 5.0
    vc = np.zeros(2 * hd, np.float16)
    vc[hd] = 1.0
    kc, vc = kc.view(np.uint16), vc.view(np.uint16)
    logistic = lambda s: 1.0 / (1.0 + math.exp(-s))
    qn0 = 3.0 / math.sqrt(25.0 + 1e-6)
    cases = {(False, 0.0): 0.5 * 5 * 3.0, (True, 0.0): 0.5 * 5 * qn0,
             (False, 2.0): 2.0 * math.tanh(0.5 * 5 * 3.0 / 2.0), (True, 2.0): 2.0 * math.tanh(0.5 * 5 * qn0 / 2.0),
             (True, -1.0): 0.5 * 5 * qn0}                          # a cap <= 0 is off
    for (qk, cap), s1 in cases.items():
        out = oracle.attend_f16(q, kc, vc, 2, 1, 1, hd, 0.5, qk_norm=qk, softcap=cap)
        assert abs(out[0] - logistic(s1)) <= 1e-6, (qk, cap, out[0], logistic(s1))
        assert not np.any(out[1:])
    got = oracle.attend_f16(q, kc, vc, 2, 1, 1, hd, 0.5, qk_norm=True, softcap=2.0)[0]
    rms0 = 3.0 / math.sqrt(25.0 / hd + 1e-6)
    for wrong in (2.0 * math.tanh(0.5 * 5 * rms0 / 2.0),           # RMS, not L2
                  0.5 * 2.0 * math.tanh(5 * qn0 / 2.0),            # cap before the scale
                  math.tanh(0.5 * 5 * qn0 / 2.0)):                 # cap without its factor
        assert abs(got - logistic(wrong)) > 1e-2
    # the QK-norm helper: unit heads, each head on its own
    x = np.random.default_rng(5).standard_normal(3 * hd).astype(np.float32)
    x[hd:2 * hd] *= 100.0
    y = oracle.qk_norm_heads(x, 3, hd).reshape(3, hd)
    assert np.allclose(np.linalg.norm(y.astype(np.float64), axis=1), 1.0, atol=1e-6)
    assert np.allclose(y * np.linalg.norm(x.reshape(3, hd).astype(np.float64), axis=1, keepdims=True),
                       x.reshape(3, hd), rtol=1e-5, atol=1e-6)


def test_silu_closed_form():
    g = np.array([0.0, 1.0, -2.0, 10.0], np.float32)
    u = np.array([3.0, 2.0, 1.0, 0.5], np.float32)
    out = oracle.silu_gate_up(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert out[0] == 0.0 and np.allclose(out, ref, rtol=1e-6)


def test_decode_layer_zero_weights_is_identity():
    hidden, inter, nq, nkv, hd = 256, 512, 2, 1, 128
    z = lambda r, c: np.zeros(r * c // 256 * 148, np.uint8)  # noqa: E731  d = 0 -> every matvec is 0
    layer = dict(wq=z(nq * hd, hidden), wk=z(nkv * hd, hidden), wv=z(nkv * hd, hidden), wo=z(hidden, nq * hd),
                 gate=z(inter, hidden), up=z(inter, hidden), down=z(hidden, inter),
                 input_norm=np.ones(hidden, np.float32), post_attn_norm=np.ones(hidden, np.float32),
                 k_cache=np.zeros(4 * nkv * hd, np.uint16), v_cache=np.zeros(4 * nkv * hd, np.uint16))
    h = oracle.gauss(13, hidden)
    out = oracle.decode_layer(layer, h, 2, hidden, inter, nq, nkv, hd, 500000.0)
    assert np.array_equal(out, h)


# ── pins written from the reference's rules by hand ──────────────────────
# Q4_K known-answer super-blocks (LC/src/cpu/ops/q4_common.rs:104-170), bytes derived by
# hand.  Block A, every value exact in binary: sub-block ranges 15.75, 1, 0, 0.625, 4,
# 1.5, 6.25, 5 and mins -7.5, -1, 0, 0.25, -3, -3.5, -1.25, -2 give
#   d = 15.75 / 63 = 0.25 (f16 0x3400), dmin = 7.5 / 15 = 0.5 (f16 0x3800),
#   sc_j = round(range_j / d) = 63, 4, 0, 3 (2.5 rounds half away), 16, 6, 25, 20,
#   m_j = round(-min_j / dmin) = 15, 2, 0, 0 (-0.5 -> -1 -> clamp 0), 6, 7, 3 (2.5), 4,
#   min bytes m_j | m_{j+4} << 4 = 0x6F, 0x72, 0x30, 0x40,
#   nibbles q = round((x + dmin m_j) / (d sc_j)): sub-block 1 has d sc = dmin m = 1, so
#   x = -0.5 -> 0.5 -> 1 (half away), x = -0.75 -> 0.25 -> 0; sub-block 4 (d sc = 4,
#   dmin m = 3) x = -1 -> 0.5 -> 1.
_Q4K_A_SPEC = {0: ([-7.5, 8.25], 0.0), 1: ([-1.0, 0.0, -0.5, -0.25, -0.75], -1.0), 2: ([], 0.0),
               3: ([0.25, 0.875], 0.5), 4: ([-3.0, 1.0, -1.0], 0.0), 5: ([-3.5, -2.0], -3.0),
               6: ([-1.25, 5.0], 0.0), 7: ([-2.0, 3.0], 0.0)}
_Q4K_A_BYTES = bytes([0x00, 0x34, 0x00, 0x38, 63, 4, 0, 3, 16, 6, 25, 20, 0, 0, 0, 0, 0x6F, 0x72, 0x30, 0x40]
                     + [0x10] + [0] * 15 + [0x10, 0x11] + [0] * 14 + [0] * 16 + [0x10] + [0x11] * 15
                     + [0x10] + [0x11] * 15 + [0x10] + [0] * 15 + [0x10] + [0] * 15 + [0x10] + [0] * 15)
# Block B, values at N(0, 0.02) scale where the truncating f16 encoder matters:
#   gmr = fl(0.03 + 0.1) = 0.13, d = fl(0.13 / 63) = 0.002063492 -> f16 truncated 0x1839
#   (round-to-nearest would give 0x183A); gmin = -0.1, dmin = fl(0.1 / 15) = 0.006666667
#   -> 0x1ED3 (nearest: 0x1ED4); -min/dmin = 10.5 and 13.5 for sub-blocks 2 and 5 round
#   half away to 11 and 14.
_Q4K_B_SPEC = {0: ([-0.1, 0.03], 0.01), 1: ([0.02, -0.04, 0.05], 0.0), 2: ([-0.07, 0.06], -0.03),
               3: ([0.011, 0.012], 0.0115), 4: ([-0.02, -0.005], -0.01), 5: ([-0.09, 0.0], -0.045),
               6: ([0.0, 0.08], 0.04), 7: ([-0.033, 0.066], 0.022)}
_Q4K_B_BYTES = bytes.fromhex(
    "3918d31e3f2c3f00072c27300000000" "03fe60b50" + "10" + "11" * 15 + "0101" + "00" * 14 + "10" + "00" * 15
    + "00" * 16 + "10" + "11" * 15 + "10" + "11" * 15 + "10" + "00" * 15 + "10" + "11" * 15)


def _spec_block(spec, sub=32):
    x = np.zeros(8 * sub, np.float32)
    for j, (vals, fill) in spec.items():
        x[sub * j:sub * (j + 1)] = np.float32(fill)
        for i, v in enumerate(vals):
            x[sub * j + i] = np.float32(v)
    return x


def test_q4k_quantizer_known_answer_bytes():
    assert len(_Q4K_A_BYTES) == 148 and len(_Q4K_B_BYTES) == 148
    assert oracle.quantize_q4_k(_spec_block(_Q4K_A_SPEC)).tobytes() == _Q4K_A_BYTES
    assert oracle.quantize_q4_k(_spec_block(_Q4K_B_SPEC)).tobytes() == _Q4K_B_BYTES
    both = np.concatenate([_spec_block(_Q4K_A_SPEC), _spec_block(_Q4K_B_SPEC)])
    assert oracle.quantize_q4_k(both).tobytes() == _Q4K_A_BYTES + _Q4K_B_BYTES


# Q6_K known-answer super-block (q4_common.rs:179-239), by hand: amax = 4 so d = 4/32 =
# 0.125 (f16 0x3000); sub-block maxima 4, 0.3125, 0, 1, 0 x 11, 2 give sc_j = 32, 3 (2.5
# rounds half away), 0, 8, ..., 16; q = round(x / (d sc_j)) + 32: x = 4 -> 33, -4 -> 31,
# +-0.3125 (d sc = 0.375) -> 33 / 31, 0.15625 -> 32, -1 -> 31, 0.5 (d sc = 1) -> 33 (half
# away), 2 -> 33.  33 = 0b10_0001 (lo4 1, hi2 2), 31 = 0b01_1111 (lo4 15, hi2 1), 32 (lo4 0,
# hi2 2); hi2 of element i sits in byte 128 + i/4 at bits 2(i%4), so a byte of four 32s
# is 0xAA, elements (32, 31, 32, 32) give 0xA6 and (31, 32, 32, 32) 0xA9.
_Q6K_X = {0: 4.0, 1: -4.0, 16: 0.3125, 17: -0.3125, 18: 0.15625, 48: -1.0, 53: 0.5, 255: 2.0}


def _q6k_expected():
    ql = [0] * 128
    ql[0], ql[8], ql[24], ql[26], ql[127] = 0xF1, 0xF1, 0x0F, 0x10, 0x10
    qh = [0xAA] * 64
    qh[0], qh[4], qh[12] = 0xA6, 0xA6, 0xA9
    sc = [32, 3, 0, 8] + [0] * 11 + [16]
    return bytes(ql + qh + sc + [0x00, 0x30])


def test_q6k_quantizer_known_answer_bytes():
    x = np.zeros(256, np.float32)
    for i, v in _Q6K_X.items():
        x[i] = v
    assert oracle.quantize_q6_k(x).tobytes() == _q6k_expected()
    # truncating f16 of d: amax 0.3 -> d = fl(0.3 / 32) = 0.009375 -> 0x20CC (nearest 0x20CD);
    # sub-block maxima 0.3 -> sc = 32, 0.1 -> fl(0.1 / d) = 10.666667 -> 11, 0.05 -> 5.33 -> 5
    x = np.zeros(256, np.float32)
    x[0], x[16], x[40] = np.float32(0.3), np.float32(-0.1), np.float32(0.05)
    q = oracle.quantize_q6_k(x)
    assert list(q[208:210]) == [0xCC, 0x20]
    assert list(q[192:195].view(np.int8)) == [32, 11, 5]


def test_rope_pairs_beyond_zero_closed_form():
    """theta_i = pos * base^(-2i/rdim) for pairs i = 1 and i = half-1 (LI/src/attention/rope.rs:33-51):
    a wrong exponent (i/rdim, 2i/head_dim with partial rotary) fails here; pair 0 cannot tell."""
    rng = np.random.default_rng(21)
    for hd, rdim, pos, base in ((128, 128, 2048, 500000.0), (64, 32, 37, 10000.0), (96, 96, 5, 1e6)):
        x = rng.standard_normal(3 * hd).astype(np.float32)
        y = oracle.rope_at(x, 3, hd, base, pos, rotary_dim=rdim)
        half = rdim // 2
        for h in range(3):
            for i in (1, half - 1):
                theta = pos * math.pow(base, -2.0 * i / rdim)
                c, s = np.float32(math.cos(theta)), np.float32(math.sin(theta))
                x0, x1 = x[h * hd + i], x[h * hd + half + i]
                assert y[h * hd + i] == x0 * c - x1 * s, (hd, rdim, i)
                assert y[h * hd + half + i] == x0 * s + x1 * c, (hd, rdim, i)
            # dimensions past the rotary part pass through unchanged
            assert np.array_equal(y[h * hd + rdim:(h + 1) * hd], x[h * hd + rdim:(h + 1) * hd])


def test_gelu_tanh_closed_form():
    g = np.array([0.0, 1.0, -2.0, 3.0, -0.5], np.float32)
    u = np.array([3.0, 2.0, 1.0, 0.5, -4.0], np.float32)
    out = oracle.gelu_tanh_gate_up(g, u)
    gd = g.astype(np.float64)
    ref = 0.5 * gd * (1 + np.tanh(math.sqrt(2 / math.pi) * (gd + 0.044715 * gd ** 3))) * u
    assert out[0] == 0.0 and np.allclose(out, ref, rtol=2e-6)
    assert abs(out[1] - 0.8411920 * 2) < 1e-5                  # gelu_tanh(1) = 0.841192


def test_rms_norm_heads_closed_form():
    x = np.array([3.0, 4.0, 0.0, 0.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    y = oracle.rms_norm_heads(x, 2, 4, eps=0.0)
    assert np.allclose(y[:4], np.array([3, 4, 0, 0]) / 2.5) and np.allclose(y[4:], 1.0)


# ── decode layer against a float64 restatement ──────────────────────────
def _f16(b):
    return float(np.uint16(b).view(np.float16))


def _deq_q4k(q, rows, cols):
    blk = q.reshape(rows * cols // 256, 148)
    out = np.empty((blk.shape[0], 256), np.float64)
    for n, b in enumerate(blk):
        d, dmin = _f16(int(b[0]) | int(b[1]) << 8), _f16(int(b[2]) | int(b[3]) << 8)
        for j in range(8):
            sc, m = int(b[4 + j]) & 63, (int(b[16 + j % 4]) >> (4 * (j // 4))) & 15
            nib = b[20 + 16 * j:36 + 16 * j]
            qv = np.empty(32, np.float64)
            qv[0::2], qv[1::2] = nib & 15, nib >> 4
            out[n, 32 * j:32 * j + 32] = d * sc * qv - dmin * m
    return out.reshape(rows, cols)


def _deq_q6k(q, rows, cols):
    blk = q.reshape(rows * cols // 256, 210)
    out = np.empty((blk.shape[0], 256), np.float64)
    e = np.arange(256)
    for n, b in enumerate(blk):
        lo4 = (b[e // 2] >> (4 * (e % 2))) & 15
        hi2 = (b[128 + e // 4] >> (2 * (e % 4))) & 3
        sc = b[192 + e // 16].view(np.int8).astype(np.float64)
        out[n] = _f16(int(b[208]) | int(b[209]) << 8) * sc * (lo4 + 16.0 * hi2 - 32.0)
    return out.reshape(rows, cols)


def test_deq_helpers_match_oracle_matvecs():
    rng = np.random.default_rng(22)
    w = (rng.standard_normal(16 * 512) * 0.05).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    for quant, deq, mv in ((oracle.quantize_q4_k, _deq_q4k, oracle.q4k_matvec),
                           (oracle.quantize_q6_k, _deq_q6k, oracle.q6k_matvec)):
        q = quant(w)
        ref = deq(q, 16, 512) @ x.astype(np.float64)
        assert np.allclose(mv(q, x, 16, 512), ref, rtol=1e-5, atol=1e-6)


def _ref_layer64(P, h, kc, vc, pos, dims, mut=()):
    """One layer in float64 from dequantized weights, written from the reference formulas:
    RMSNorm LI/src/residual.rs:17-33 (x / sqrt(mean x^2 + eps) * (offset + w)); RoPE
    LI/src/attention/rope.rs:22-55 (split-half pairs, theta = pos base^(-2i/rdim)); GQA
    LI/src/attention/gqa.rs:29-110 (kv head h / reps, softmax of scaled dots); SiLU / GELU
    gate x up LI/src/ffn/mod.rs:87-103; residual and post-norm order
    LI/src/attention/block.rs:139-150 and LI/src/forward/layer.rs:54-94; V-norm
    LI/src/residual.rs:86-110; layer scalar LI/src/forward/layer.rs:98-108.
    `mut` plants one mistake, to show the comparison would catch it."""
    hidden, inter, nq, nkv, hd = dims
    eps, off = 1e-6, P.get("norm_offset", 0.0)
    rdim = P.get("rotary_dim", 0) or hd

    def norm(x, w):
        r = np.sqrt(np.sum(x * x) / x.size + eps)
        return x / r * ((off + w) if w is not None else 1.0)

    W = P["deq"]
    q8in = P.get("q8_input", ())

    def proj(name, x):
        """W x; projections whose format takes a Q8 input see quantize_to_q8(x) (f32)."""
        if name in q8in:
            q, s8 = oracle.quantize_to_q8(x.astype(np.float32))
            x = q.astype(np.float64) * np.repeat(s8.astype(np.float64), 32)
        return W[name] @ x

    h = h.astype(np.float64)
    nin, npost = P["input_norm"], P["post_attn_norm"]
    if "swap_norms" in mut:
        nin, npost = npost, nin
    xn = norm(h, nin)
    q, k, v = proj("wq", xn), proj("wk", xn), proj("wv", xn)
    if P.get("has_v_norm"):
        v = v.reshape(nkv, hd)
        v = (v / np.sqrt((v * v).mean(1, keepdims=True) + eps)).reshape(-1)
    half = rdim // 2
    th = pos * np.power(P["rope_base"], -2.0 * np.arange(half) / rdim)
    if "rope_exp" in mut:
        th = pos * np.power(P["rope_base"], -1.0 * np.arange(half) / rdim)
    c, s = np.cos(th), np.sin(th)

    def rope(t, n):
        t = t.reshape(n, hd).copy()
        a, b = t[:, :half].copy(), t[:, half:2 * half].copy()
        t[:, :half], t[:, half:2 * half] = a * c - b * s, a * s + b * c
        return t.reshape(-1)

    q, k = rope(q, nq), rope(k, nkv)
    if P.get("qk_norm"):           # per query head, after RoPE; RMS under the planted "qk_rms"
        qh = q.reshape(nq, hd)
        ss = (qh * qh).sum(1, keepdims=True) / (hd if "qk_rms" in mut else 1)
        q = (qh / np.sqrt(ss + 1e-6)).reshape(-1)
        if "qk_norm_k" in mut:
            kh = k.reshape(nkv, hd)
            k = (kh / np.sqrt((kh * kh).sum(1, keepdims=True) + 1e-6)).reshape(-1)
    if "rope_v" in mut:
        v = rope(v, nkv)
    kvd = nkv * hd
    if kc.dtype == np.float32:   # the reference's f32 cache (kv_cache.rs:13-14): the new row unrounded
        K = kc.astype(np.float64).reshape(-1, kvd)[:pos + 1].copy()
        V = vc.astype(np.float64).reshape(-1, kvd)[:pos + 1].copy()
        K[pos], V[pos] = k.astype(np.float32), v.astype(np.float32)
        if "kv_fp16" in mut:     # planted: the new row rounded as an fp16 cache rounds it
            K[pos], V[pos] = k.astype(np.float16), v.astype(np.float16)
    else:
        K = kc.view(np.float16).astype(np.float64).reshape(-1, kvd)[:pos + 1].copy()
        V = vc.view(np.float16).astype(np.float64).reshape(-1, kvd)[:pos + 1].copy()
        K[pos] = k.astype(np.float16)                              # fp16 cache row, RNE
        V[pos] = v.astype(np.float16)
    scale = P.get("attn_scale", 0.0) or 1.0 / math.sqrt(hd)
    att = np.empty(nq * hd)
    for qh in range(nq):
        kvh = qh % nkv if "kv_map" in mut else qh // (nq // nkv)
        sc = K[:, kvh * hd:(kvh + 1) * hd] @ q[qh * hd:(qh + 1) * hd] * scale
        cap = P.get("softcap", 0.0)
        if cap > 0:
            sc = (np.tanh(sc / scale / cap) * cap * scale) if "cap_pre_scale" in mut else np.tanh(sc / cap) * cap
        p = np.exp(sc - sc.max())
        att[qh * hd:(qh + 1) * hd] = (p / p.sum()) @ V[:, kvh * hd:(kvh + 1) * hd]
    o = proj("wo", att)
    if P.get("has_post_norms"):
        h1 = h + norm(o, npost)
        f = norm(h1, P.get("pre_ffn_norm"))
    else:
        h1 = (o if "drop_residual" in mut else h + o)
        f = norm(h1, npost)
    g, u = proj("gate", f), proj("up", f)
    if "gate_up_swap" in mut:
        g, u = u, g
    if P.get("activation") == "gelu_tanh":
        a = 0.5 * g * (1 + np.tanh(math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3))) * u
    else:
        a = g / (1 + np.exp(-g)) * u
    dn = proj("down", a)
    h2 = h1 + (norm(dn, P.get("post_ffn_norm")) if P.get("has_post_norms") else dn)
    if P.get("layer_scalar", 0.0) != 0.0:
        h2 = h2 * P["layer_scalar"]
    return h2


def _tiny_layer(seed, dims, formats, std=0.08, **variant):
    hidden, inter, nq, nkv, hd = dims
    rng = np.random.default_rng(seed)
    shapes = dict(wq=(nq * hd, hidden), wk=(nkv * hd, hidden), wv=(nkv * hd, hidden), wo=(hidden, nq * hd),
                  gate=(inter, hidden), up=(inter, hidden), down=(hidden, inter))
    P = dict(deq={}, formats=formats, rope_base=10000.0, **variant)
    P["q8_input"] = tuple(n for n, f in formats.items() if f == "q8_0" or (f == "q4_0" and n != "down"))
    for name, (r, c) in shapes.items():
        w = (rng.standard_normal(r * c) * std).astype(np.float32)
        if formats.get(name) == "q6_k":
            P[name] = oracle.quantize_q6_k(w)
            P["deq"][name] = _deq_q6k(P[name], r, c)
        elif formats.get(name) == "q8_0":
            P[name], P[name + "_s"] = oracle.quantize_weights_q8(w, r, c)
            P["deq"][name] = (P[name].astype(np.float64).reshape(r, -1, 32) *
                              P[name + "_s"].astype(np.float64).reshape(r, -1, 1)).reshape(r, c)
        elif formats.get(name) == "q4_0":
            P[name] = oracle.quantize_q4_0(w)
            P["deq"][name] = _deq_q4_0(P[name], r * c).astype(np.float64).reshape(r, c)
        else:
            P[name] = oracle.quantize_q4_k(w)
            P["deq"][name] = _deq_q4k(P[name], r, c)
    P["input_norm"] = (1.0 + 0.5 * rng.standard_normal(hidden)).astype(np.float32)
    P["post_attn_norm"] = (0.3 + 0.2 * rng.standard_normal(hidden)).astype(np.float32)
    if variant.get("has_post_norms"):
        P["pre_ffn_norm"] = (0.7 + 0.3 * rng.standard_normal(hidden)).astype(np.float32)
        P["post_ffn_norm"] = (1.2 + 0.3 * rng.standard_normal(hidden)).astype(np.float32)
    return P


def _run_layer_case(P, dims, pos, seed, f32_kv=False):
    hidden, inter, nq, nkv, hd = dims
    rng = np.random.default_rng(seed)
    kvd = nkv * hd
    kc = rng.standard_normal((pos + 2) * kvd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((pos + 2) * kvd).astype(np.float16).view(np.uint16)
    if f32_kv:   # f32 cache rows that no fp16 holds exactly
        kc = rng.standard_normal((pos + 2) * kvd).astype(np.float32)
        vc = rng.standard_normal((pos + 2) * kvd).astype(np.float32)
    h = rng.standard_normal(hidden).astype(np.float32)
    layer = {k: v for k, v in P.items() if k not in ("deq", "rope_base", "q8_input")}
    layer["k_cache"], layer["v_cache"] = kc.copy(), vc.copy()
    got = oracle.decode_layer(layer, h, pos, hidden, inter, nq, nkv, hd, P["rope_base"])
    return got, (lambda mut=(): _ref_layer64(P, h, kc, vc, pos, dims, mut))


def _rel(a, b):
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_decode_layer_llama_matches_float64_composition():
    """lo_decode_layer (Llama: pre-norm, SiLU, no post-norms) against the float64
    restatement within 1e-5; each planted mistake moves the output by more than 1e-2."""
    dims = (256, 512, 4, 2, 64)
    P = _tiny_layer(31, dims, {"wv": "q6_k", "down": "q6_k"})
    got, ref = _run_layer_case(P, dims, pos=5, seed=32)
    assert _rel(got, ref()) <= 1e-5
    for mut in ("swap_norms", "gate_up_swap", "drop_residual", "rope_v", "rope_exp", "kv_map"):
        assert _rel(got, ref((mut,))) > 1e-2, mut


def test_decode_layer_f32_kv_matches_float64_composition():
    """The f32-cache mode (the reference's cache, LC/src/metal/ops/kv_cache.rs:13-14; CPU
    attention in f32, LI/src/attention/gqa.rs:29-110): cached rows read as f32 and the new
    row stored unrounded.  Within 3e-6 of the float64 restatement (measured <= 1e-6);
    rounding the new row to fp16 (what an fp16 cache does) moves it by more than 5e-5
    (measured >= 2.2e-4), and the Llama mistakes still move it by more than 1e-2."""
    dims = (256, 512, 4, 2, 64)
    P = _tiny_layer(35, dims, {"wv": "q6_k"})
    for pos in (0, 1, 3):
        got, ref = _run_layer_case(P, dims, pos=pos, seed=36 + pos, f32_kv=True)
        e, e16 = _rel(got, ref()), _rel(got, ref(("kv_fp16",)))
        print(f"f32 kv pos={pos}: vs float64 {e:.2e}, vs fp16-rounded new row {e16:.2e}")
        assert e <= 3e-6
        assert e16 > 5e-5
    for mut in ("swap_norms", "gate_up_swap", "drop_residual", "rope_v", "kv_map"):
        assert _rel(got, ref((mut,))) > 1e-2, mut


def test_decode_layer_variants_match_float64_composition():
    """Post-norms with pre/post-FFN weights, norm offset 1, GELU-tanh, V-norm, a layer scalar,
    partial rotary and an explicit attention scale (a Gemma-style layer,
    LC/src/pipeline.rs:76-115), then the same with the pre/post-FFN weights absent."""
    dims = (256, 512, 4, 2, 64)
    var = dict(has_post_norms=True, norm_offset=1.0, activation="gelu_tanh", has_v_norm=True,
               layer_scalar=0.75, rotary_dim=32, attn_scale=0.2)
    P = _tiny_layer(33, dims, {"wq": "q6_k"}, **var)
    got, ref = _run_layer_case(P, dims, pos=3, seed=34)
    assert _rel(got, ref()) <= 1e-5
    for mut in ("swap_norms", "gate_up_swap", "rope_exp", "kv_map"):
        assert _rel(got, ref((mut,))) > 1e-2, mut
    # the same layer under SiLU, offset 0, no V-norm, no scalar is far away
    for k, v in (("activation", "silu"), ("norm_offset", 0.0), ("has_v_norm", False), ("layer_scalar", 0.0)):
        Q = dict(P, **{k: v})
        assert _rel(got, _ref_layer64(Q, *_inputs_of(P, dims, 3, 34))) > 1e-2, k
    P2 = dict(P, pre_ffn_norm=None, post_ffn_norm=None)
    got2, ref2 = _run_layer_case(P2, dims, pos=3, seed=34)
    assert _rel(got2, ref2()) <= 1e-5 and _rel(got2, got) > 1e-2


def test_decode_layer_qk_norm_softcap_match_float64_composition():
    """The prompt-attention options in the oracle layer (QK-norm of the RoPE'd query heads,
    the score cap) against the float64 restatement within 1e-5; planted mistakes (K normed
    too, the RMS norm for the L2 norm, the cap before the scale) each move it by > 1e-2, and
    each option alone is far from the layer without it."""
    dims = (256, 512, 4, 2, 64)
    P = _tiny_layer(35, dims, {}, std=0.3, qk_norm=True, softcap=1.0, attn_scale=0.5)
    got, ref = _run_layer_case(P, dims, pos=6, seed=36)
    assert _rel(got, ref()) <= 1e-5
    for mut in ("qk_norm_k", "qk_rms", "cap_pre_scale"):
        assert _rel(got, ref((mut,))) > 1e-2, mut
    for k, v in (("qk_norm", False), ("softcap", 0.0)):
        Q = dict(P, **{k: v})
        got_q, ref_q = _run_layer_case(Q, dims, pos=6, seed=36)
        assert _rel(got_q, ref_q()) <= 1e-5 and _rel(got_q, got) > 1e-2, k


def _inputs_of(P, dims, pos, seed):
    hidden, inter, nq, nkv, hd = dims
    rng = np.random.default_rng(seed)
    kvd = nkv * hd
    kc = rng.standard_normal((pos + 2) * kvd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((pos + 2) * kvd).astype(np.float16).view(np.uint16)
    h = rng.standard_normal(hidden).astype(np.float32)
    return h, kc, vc, pos, dims


# ── Q4_KF: GGUF 144-byte (llama.cpp layout) and 160-byte pre-baked ─────────
# Scales sc = 1, 2, 3, 4, 33, 47, 50, 63 and mins m = 5, 6, 7, 8, 17, 31, 42, 60 packed by
# hand in the llama.cpp layout: byte j (j < 4) = sc_j | (sc_{j+4} >> 4) << 6, byte 4 + j =
# m_j | (m_{j+4} >> 4) << 6, byte 8 + j = (sc_{j+4} & 15) | (m_{j+4} & 15) << 4.
_GGUF_SC = (1, 2, 3, 4, 33, 47, 50, 63)
_GGUF_M = (5, 6, 7, 8, 17, 31, 42, 60)
_GGUF_Q12 = bytes([0x81, 0x82, 0xC3, 0xC4, 0x45, 0x46, 0x87, 0xC8, 0x11, 0xFF, 0xA2, 0xCF])


def test_gguf_scale_min_known_answer():
    q12 = np.frombuffer(_GGUF_Q12, np.uint8)
    for j in range(8):
        assert oracle.gguf_scale_min(j, q12) == (_GGUF_SC[j], _GGUF_M[j]), j


def test_q4kf_gguf_onehot_probes_closed_form():
    """Element e of a llama.cpp block: chunk c = e // 64 of 32 bytes, low nibbles first
    (sub-block 2c), then high nibbles (2c + 1); w = d sc_j q - dmin m_j."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0.5], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.25], np.float16).view(np.uint8)
    blk[4:16] = np.frombuffer(_GGUF_Q12, np.uint8)
    blk[16:] = (np.arange(128) * 37 % 256).astype(np.uint8)
    for e in (0, 1, 31, 32, 33, 63, 64, 95, 96, 130, 191, 192, 224, 255):
        c, l = divmod(e, 64)
        q = (blk[16 + 32 * c + l] & 15) if l < 32 else (blk[16 + 32 * c + l - 32] >> 4)
        j = e // 32
        want = np.float32(np.float32(0.5) * np.float32(_GGUF_SC[j])) * np.float32(q) - \
            np.float32(np.float32(0.25) * np.float32(_GGUF_M[j]))
        x = np.zeros(256, np.float32)
        x[e] = 1.0
        assert oracle.q4kf_gguf_matvec(blk, x, 1, 256)[0] == want, e


def test_q4k_to_llamacpp_gguf_is_lossless():
    """The 148 -> llama.cpp-144 converter (test data for the GGUF path) keeps every
    dequantized value: the GGUF matvec of converted bytes equals the Q4_K matvec bit for
    bit (same element order), also on fuzzed bytes with the unused scale bits set."""
    rng = np.random.default_rng(40)
    rows, cols = 24, 1024
    q = oracle.quantize_q4_k((rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    fz = rng.integers(0, 256, q.size, dtype=np.uint8)
    fz.reshape(-1, 148)[:, 1] &= 0x3B                              # finite, modest d
    fz.reshape(-1, 148)[:, 3] &= 0x3B                              # and dmin
    x = rng.standard_normal(cols).astype(np.float32)
    for blocks in (q, fz):
        a = oracle.q4k_matvec(blocks, x, rows, cols)
        b = oracle.q4kf_gguf_matvec(oracle.q4k_to_gguf_llamacpp(blocks), x, rows, cols)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4kf160_known_answer_and_onehot():
    """q4k_to_q4kf (q4_common.rs:370-413) of the hand block A above: d sc_j = 0.25 x (63, 4,
    0, 3, 16, 6, 25, 20) and dmin m_j = 0.5 x (15, 2, 0, 0, 6, 7, 3, 4), all exact in f16;
    the 128 nibble bytes copied."""
    q4k = np.frombuffer(_Q4K_A_BYTES, np.uint8)
    kf = oracle.q4k_to_q4kf(q4k)
    sc = np.array([15.75, 1.0, 0.0, 0.75, 4.0, 1.5, 6.25, 5.0], np.float16)
    mn = np.array([7.5, 1.0, 0.0, 0.0, 3.0, 3.5, 1.5, 2.0], np.float16)
    assert kf[:16].tobytes() == sc.tobytes() and kf[16:32].tobytes() == mn.tobytes()
    assert kf[32:].tobytes() == _Q4K_A_BYTES[20:]
    for e in (0, 1, 33, 34, 130, 255):
        j, w = divmod(e, 32)
        byte = kf[32 + 16 * j + w // 2]
        q = (byte >> 4) if w % 2 else (byte & 15)
        x = np.zeros(256, np.float32)
        x[e] = 1.0
        assert oracle.q4kf160_matvec(kf, x, 1, 256)[0] == np.float32(sc[j]) * np.float32(q) - np.float32(mn[j])


def test_reference_gguf_packing_known_answers():
    """The reference's own GGUF writers (q4_common.rs:248-361) pack 6-bit mins as byte j =
    sc_j | (m_j & 3) << 6 and byte 8 + j = (m_2j >> 2) | (m_2j+1 >> 2) << 4, and keep the
    148-byte nibble order.  Block A (sc 63, 4, 0, 3, 16, 6, 25, 20; m 15, 2, 0, 0, 6, 7, 3, 4)
    through q4k_to_gguf: FF 84 00 03 90 C6 D9 14 03 00 11 10.  quantize_q4_k_gguf of block A's
    input: dmin = fl(7.5 / 63) = 0.11904762 -> f16 0x2F9E (truncated), m_j = round(-min_j /
    dmin) = 63, 8 (8.4), 0, 0 (-2.1), 25 (25.2), 29 (29.4), 11 (10.5 half away), 17 (16.8).
    Read back with the llama.cpp unpack these bytes give other scales and mins (the
    reference's GPU kernels and its writers disagree); this build reads Q4_KF as the GPU
    kernels do."""
    g = oracle.q4k_to_gguf(np.frombuffer(_Q4K_A_BYTES, np.uint8))
    assert g[:4].tobytes() == _Q4K_A_BYTES[:4]
    assert g[4:16].tobytes() == bytes([0xFF, 0x84, 0x00, 0x03, 0x90, 0xC6, 0xD9, 0x14, 0x03, 0x00, 0x11, 0x10])
    assert g[16:].tobytes() == _Q4K_A_BYTES[20:]
    assert oracle.gguf_scale_min(4, g[4:16]) != (16, 6)
    q = oracle.quantize_q4_k_gguf(_spec_block(_Q4K_A_SPEC))
    assert q[:16].tobytes() == bytes([0x00, 0x34, 0x9E, 0x2F, 0xFF, 0x04, 0x00, 0x03, 0x50, 0x46, 0xD9, 0x54,
                                      0x2F, 0x00, 0x76, 0x42])
    # nibbles q = round((x + dmin m_j) / (d sc_j)): sub-block 1 (d sc = 1, dmin m = 0.952):
    # x = 0 -> 1, -0.5 -> 0.45 -> 0, -0.25 -> 0.70 -> 1; sub-block 4 (d sc = 4, dmin m = 2.976):
    # x = 1 -> 0.99 -> 1, -1 -> 0.49 -> 0, fill 0 -> 0.74 -> 1
    assert list(q[32:36]) == [0x10, 0x10, 0x00, 0x00]
    assert list(q[80:84]) == [0x10, 0x10, 0x11, 0x11]


def test_decode_layer_q8_attention_q4_0_ffn_matches_float64_composition():
    """Q8_0 attention projections and a Q4_0 FFN (the reference GPU decode's Q8 / Q4_0 paths,
    LC/src/metal/decode.rs:262-296, 374-404, 560-690): the projections that take a Q8 input
    see quantize_to_q8 of their f32 input, the Q4_0 down projection the f32 activation.  The
    float64 restatement quantizes the same f32 inputs; 1e-5 as above."""
    dims = (256, 512, 4, 2, 64)
    fm = {"wq": "q8_0", "wk": "q8_0", "wv": "q8_0", "wo": "q8_0", "gate": "q4_0", "up": "q4_0", "down": "q4_0"}
    P = _tiny_layer(35, dims, fm)
    got, ref = _run_layer_case(P, dims, pos=4, seed=36)
    print(f"q8/q4_0 layer rel {_rel(got, ref()):.2e}")
    assert _rel(got, ref()) <= 1e-5
    for mut in ("swap_norms", "gate_up_swap", "drop_residual", "kv_map"):
        assert _rel(got, ref((mut,))) > 1e-2, mut


def test_threaded_drivers_equal_one_thread():
    """The row-split drivers of the CPU baselines (lo_proj_rows_mt, lo_decode_layer_mt) run
    the one-thread kernels on contiguous row slices: identical output for every format,
    thread counts that do and do not divide the rows, and more threads than rows."""
    dims = (256, 512, 4, 2, 64)
    fm = {"wq": "q8_0", "wk": "q6_k", "wv": "q4_k", "wo": "q4_0", "gate": "q4_0", "up": "q4_k", "down": "q4_0"}
    P = _tiny_layer(41, dims, fm)
    hidden, inter, nq, nkv, hd = dims
    rng = np.random.default_rng(42)
    x = rng.standard_normal(hidden).astype(np.float32)
    for name, rows in (("wq", nq * hd), ("wk", nkv * hd), ("wv", nkv * hd), ("gate", inter), ("up", inter)):
        f = fm[name]
        q8in = f == "q4_0"
        one = oracle.proj_rows_mt(f, P[name], x, rows, hidden, 1, P.get(name + "_s"), q8in)
        for t in (3, 7, rows + 5):
            got = oracle.proj_rows_mt(f, P[name], x, rows, hidden, t, P.get(name + "_s"), q8in)
            assert np.array_equal(one.view(np.uint32), got.view(np.uint32)), (name, t)
    kvd = nkv * hd
    pos = 9
    kc = rng.standard_normal((pos + 2) * kvd).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal((pos + 2) * kvd).astype(np.float16).view(np.uint16)
    h = rng.standard_normal(hidden).astype(np.float32)
    layer = {k: v for k, v in P.items() if k not in ("deq", "rope_base", "q8_input")}
    outs = []
    for t in (1, 5):
        layer["k_cache"], layer["v_cache"] = kc.copy(), vc.copy()
        outs.append((oracle.decode_layer(layer, h, pos, *dims, 10000.0, threads=t),
                     layer["k_cache"].copy(), layer["v_cache"].copy()))
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a.view(np.uint32) if a.dtype == np.float32 else a,
                              b.view(np.uint32) if b.dtype == np.float32 else b)


def test_q4_0_f32_matvec_closed_form():
    """q4_f32_matvec (LC/src/metal/shaders/q4_f32_matvec.rs:10-38): one-hot probes give
    (nib - 8) * f16(scale) per element (element 2j the low, 2j + 1 the high nibble of byte j),
    and random inputs agree with a float64 dequantized dot within f32 rounding."""
    blk = np.zeros(2 * 18, np.uint8)
    blk[0:2] = np.array([0.75], np.float16).view(np.uint8)
    blk[18:20] = np.array([-2.5], np.float16).view(np.uint8)
    blk[2:18] = (np.arange(16) * 29 % 256).astype(np.uint8)
    blk[20:36] = (np.arange(16) * 53 % 256).astype(np.uint8)
    for e in (0, 1, 2, 31, 32, 33, 50, 63):
        b, w = divmod(e, 32)
        byte = blk[18 * b + 2 + w // 2]
        nib = (byte >> 4) if w % 2 else (byte & 15)
        x = np.zeros(64, np.float32)
        x[e] = 1.0
        assert oracle.q4_0_f32_matvec(blk, x, 1, 64)[0] == np.float32(int(nib) - 8) * np.float32((0.75, -2.5)[b])
    rng = np.random.default_rng(37)
    rows, cols = 20, 1024
    q4 = oracle.quantize_q4_0(rng.standard_normal(rows * cols).astype(np.float32))
    x = rng.standard_normal(cols).astype(np.float32)
    ref = _deq_q4_0(q4, rows * cols).astype(np.float64).reshape(rows, cols) @ x.astype(np.float64)
    assert np.allclose(oracle.q4_0_f32_matvec(q4, x, rows, cols), ref, rtol=1e-5, atol=1e-5)
