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
  quantize_q4_k / q4k_matvec                  test_metal_shaders.rs:1301-1331 hand block
                                              (closed form); one-hot probes of hand-built
                                              blocks (closed form per element); dequant
                                              error bound of the quantizer.
  quantize_q6_k / q6k_matvec                  test_metal_shaders.rs:1334-1361 hand block;
                                              one-hot probes of hand-built qh/ql/scale bytes.
  quantize_weights_q8 / q8_matvec             exact integer block dots vs numpy; the
                                              q8_matvec.rs:290-316 cosine > 0.999 check.
  top-k (abs / signed)                        test_vindex.rs:134-160 known answers; vs
                                              numpy stable argsort on random scores.
  gate_scores_f32 (canonical fma chain)       vs math.fsum-exact f64 dot within f32 bounds.
  rms_norm / rope / silu / attention          closed forms: rope(pos=0) = identity, pair
                                              norm preserved; attention over T=1 returns V
                                              (LC/src/cpu/ops/attention.rs:66-75), equal keys
                                              give the mean of V; rms of output = 1.
  decode_layer                                composition of the above; all-zero weights
                                              leave h unchanged (residual identity).
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
