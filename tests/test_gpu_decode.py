"""GPU parity of the decode step (ComputeBackend::decode_token, populate_kv_layer,
reset_kv_cache; larql-compute/src/backend.rs:99-123) against the CPU oracle's
Llama layer (oracle.decode_layer: LI/src/attention/{rope,gqa}.rs, LI/src/residual.rs,
LI/src/ffn/mod.rs composed in the reference GPU decode's op order).

Bar: max|gpu - cpu| / max|cpu| <= 1e-3 on the hidden state / logits (floating-point
outputs), and the greedy next token (argmax of the logits) identical.
The KV cache is fp16 on both sides (new rows rounded to nearest even).
"""
import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def q4k(rows, cols, seed, std=0.02):
    return oracle.quantize_q4_k(oracle.gauss(seed, rows * cols, 0.0, std))


def q6k(rows, cols, seed, std=0.02):
    return oracle.quantize_q6_k(oracle.gauss(seed, rows * cols, 0.0, std))


def q4kf(rows, cols, seed, std=0.02):
    """Q4_KF, 144-byte GGUF (llama.cpp layout): Q4_K converted losslessly, then bits 4..5 of
    every 6-bit min set at random so mins above 15 occur."""
    g = oracle.q4k_to_gguf_llamacpp(q4k(rows, cols, seed, std)).reshape(-1, 144)
    rng = np.random.default_rng(seed)
    g[:, 8:12] |= ((rng.integers(0, 4, (g.shape[0], 4)) << 4) | (rng.integers(0, 4, (g.shape[0], 4)) << 6)).astype(np.uint8)
    return g.reshape(-1)


def q4kf160(rows, cols, seed, std=0.02):
    """Q4_KF, 160-byte pre-baked half scales (the reference's q4k_to_q4kf)."""
    return oracle.q4k_to_q4kf(q4k(rows, cols, seed, std))


def q4_0(rows, cols, seed, std=0.02):
    return oracle.quantize_q4_0(oracle.gauss(seed, rows * cols, 0.0, std))


MAKERS = {"q4_k": q4k, "q6_k": q6k, "q4_kf": q4kf, "q4_kf160": q4kf160, "q4_0": q4_0}
HIP_FORMAT = {"q6_k": larql_hip.Q6_K, "q4_kf": larql_hip.Q4_KF, "q4_kf160": larql_hip.Q4_KF, "q8_0": larql_hip.Q8_0,
              "q4_0": larql_hip.Q4_0}


class SmallModel:
    """formats: projection name -> "q6_k" / "q4_kf" / "q4_kf160" (default Q4_K).  variant: layer
    variants of FullPipelineLayer (larql-compute/src/pipeline.rs:76-115) in the oracle's
    keys: norm_offset, has_post_norms (with pre/post-FFN norm weights unless
    ffn_norm_weights=False), activation ("silu" | "gelu_tanh"), has_v_norm, layer_scalar,
    rotary_dim."""

    def __init__(self, n_layers, hidden, inter, nq, nkv, hd, cap, seed=0, formats=None, variant=None):
        self.n, self.hidden, self.inter, self.nq, self.nkv, self.hd = n_layers, hidden, inter, nq, nkv, hd
        self.formats = dict(formats or {})
        self.variant = dict(variant or {})
        ffn_w = self.variant.pop("ffn_norm_weights", True)
        self.layers = []
        qd, kvd = nq * hd, nkv * hd
        shapes = dict(wq=(qd, hidden), wk=(kvd, hidden), wv=(kvd, hidden), wo=(hidden, qd), gate=(inter, hidden),
                      up=(inter, hidden), down=(hidden, inter))
        for l in range(n_layers):
            s = seed + 100 * l
            L = {}
            for i, (name, (r, c)) in enumerate(shapes.items()):
                if self.formats.get(name) == "q8_0":   # int8 weights + f32 scales (QuantWeight.scales)
                    L[name], L[name + "_s"] = oracle.quantize_weights_q8(oracle.gauss(s + 1 + i, r * c, 0.0, 0.02), r, c)
                else:
                    L[name] = MAKERS[self.formats.get(name, "q4_k")](r, c, s + 1 + i)
            L.update(input_norm=(1.0 + 0.1 * oracle.gauss(s + 8, hidden)).astype(np.float32),
                     post_attn_norm=(1.0 + 0.1 * oracle.gauss(s + 9, hidden)).astype(np.float32),
                     k_cache=np.zeros(cap * kvd, np.uint16), v_cache=np.zeros(cap * kvd, np.uint16),
                     formats=self.formats, **self.variant)
            if self.variant.get("has_post_norms") and ffn_w:
                L.update(pre_ffn_norm=(0.8 + 0.2 * oracle.gauss(s + 10, hidden)).astype(np.float32),
                         post_ffn_norm=(0.5 + 0.2 * oracle.gauss(s + 11, hidden)).astype(np.float32))
            self.layers.append(L)

    def hip_layers(self, rope_base, window=0):
        fm = {k: HIP_FORMAT[v] for k, v in self.formats.items() if v in HIP_FORMAT}
        v = self.variant
        act = larql_hip.ACT_GELU_TANH if v.get("activation") == "gelu_tanh" else larql_hip.ACT_SILU
        return [larql_hip.make_layer(L["wq"], L["wk"], L["wv"], L["wo"], L["gate"], L["up"], L["down"],
                                     L["input_norm"], L["post_attn_norm"], head_dim=self.hd,
                                     num_q_heads=self.nq, num_kv_heads=self.nkv, rope_base=rope_base,
                                     sliding_window=window, formats=fm, norm_offset=v.get("norm_offset", 0.0),
                                     has_post_norms=v.get("has_post_norms", False),
                                     pre_ffn_norm=L.get("pre_ffn_norm"), post_ffn_norm=L.get("post_ffn_norm"),
                                     activation=act, has_v_norm=v.get("has_v_norm", False),
                                     layer_scalar=v.get("layer_scalar", 0.0), rotary_dim=v.get("rotary_dim", 0),
                                     scales={n: L[n + "_s"] for n in self.formats if n + "_s" in L})
                for L in self.layers]


def run_sequence(hip, T0, n_tokens, n_layers=2, hidden=512, inter=1024, nq=8, nkv=2, hd=64, rope=500000.0,
                 window=0, formats=None, variant=None):
    print(f"[decode] layers={n_layers} hidden={hidden} nq={nq} nkv={nkv} hd={hd} T0={T0} tokens={n_tokens} "
          f"window={window} formats={formats} variant={variant}", flush=True)
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=T0 + n_tokens + 1, seed=T0, formats=formats,
                   variant=variant)
    kvd = nkv * hd
    hip.reset_kv_cache()
    for l, L in enumerate(m.layers):
        k = oracle.gauss(5000 + l, T0 * kvd)
        v = oracle.gauss(6000 + l, T0 * kvd)
        hip.populate_kv_layer(l, k, v, T0, nkv, hd)
        L["k_cache"][: T0 * kvd] = k.astype(np.float16).view(np.uint16)
        L["v_cache"][: T0 * kvd] = v.astype(np.float16).view(np.uint16)
    assert hip.kv_cache_len() == T0
    layers = m.hip_layers(rope, window)
    errs = []
    for i in range(n_tokens):
        x = oracle.gauss(7000 + i, hidden)
        got = hip.decode_token(layers, x, hidden, inter, nq * hd, kvd, nq, nkv, hd, rope)
        ref = x.copy()
        for L in m.layers:
            ref = oracle.decode_layer(L, ref, T0 + i, hidden, inter, nq, nkv, hd, rope, window=window)
        e = rel_err(got, ref)
        errs.append(e)
        print(f"  token {i} pos {T0 + i}: rel_err={e:.3e}", flush=True)
        assert e <= REL_TOL, (i, e)
    assert hip.kv_cache_len() == T0 + n_tokens
    return errs


def test_decode_fp16_cache_drift_against_f32_cache(hip):
    """The reference keeps K/V in f32 (LC/src/metal/ops/kv_cache.rs:13-14; populate_kv_layer
    takes f32 rows, LC/src/metal/trait_impl.rs:197-225; the CPU attention is f32,
    LI/src/attention/gqa.rs:29-110); this backend stores them in fp16.  After a 512-position
    cache populated from f32 rows, 64 tokens are decoded through 4 layers: every step's
    hidden state stays within 1e-3 of the oracle run with f32 caches (populated and new
    rows unrounded), so the fp16 cache's drift is inside the bar over a generation.  The
    same steps against the oracle's fp16 cache measure the kernels alone."""
    n_layers, hidden, inter, nq, nkv, hd, T0, n = 4, 512, 1024, 8, 2, 64, 512, 64
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=T0 + n + 1, seed=77)
    m16 = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=T0 + n + 1, seed=77)
    kvd = nkv * hd
    hip.reset_kv_cache()
    for l, (L, L16) in enumerate(zip(m.layers, m16.layers)):
        k, v = oracle.gauss(5100 + l, T0 * kvd), oracle.gauss(5200 + l, T0 * kvd)
        hip.populate_kv_layer(l, k, v, T0, nkv, hd)
        L["k_cache"] = np.zeros((T0 + n + 1) * kvd, np.float32)
        L["v_cache"] = np.zeros((T0 + n + 1) * kvd, np.float32)
        L["k_cache"][: T0 * kvd], L["v_cache"][: T0 * kvd] = k, v
        L16["k_cache"][: T0 * kvd] = k.astype(np.float16).view(np.uint16)
        L16["v_cache"][: T0 * kvd] = v.astype(np.float16).view(np.uint16)
    layers = m.hip_layers(500000.0)
    drift, kern = [], []
    for i in range(n):
        x = oracle.gauss(7100 + i, hidden)
        got = hip.decode_token(layers, x, hidden, inter, nq * hd, kvd, nq, nkv, hd, 500000.0)
        ref, ref16 = x.copy(), x.copy()
        for L, L16 in zip(m.layers, m16.layers):
            ref = oracle.decode_layer(L, ref, T0 + i, hidden, inter, nq, nkv, hd, 500000.0)
            ref16 = oracle.decode_layer(L16, ref16, T0 + i, hidden, inter, nq, nkv, hd, 500000.0)
        drift.append(rel_err(got, ref))
        kern.append(rel_err(got, ref16))
    print(f"[kv drift] {n} tokens after {T0}: vs f32 cache max {max(drift):.3e} (last {drift[-1]:.3e}); "
          f"vs fp16 cache max {max(kern):.3e}", flush=True)
    assert max(kern) <= REL_TOL
    assert max(drift) <= REL_TOL


def test_decode_short_cache(hip):
    run_sequence(hip, T0=5, n_tokens=3)


def test_decode_multi_split_cache(hip):
    # T crosses many 64-position attention splits and the 1024 cap of the reference kernel
    run_sequence(hip, T0=2047, n_tokens=2)


def test_decode_empty_cache(hip):
    # first token: T = 1, attention returns V of the new position
    run_sequence(hip, T0=0, n_tokens=2, n_layers=1)


def test_decode_gqa_ratio_and_rope_base(hip):
    run_sequence(hip, T0=100, n_tokens=2, n_layers=1, nq=16, nkv=2, hd=128, hidden=1024, inter=512, rope=10000.0)


def test_decode_sliding_window(hip):
    # windows whose first position is not a multiple of 8 (the attention chunks start at
    # the window start rounded down to 8 and mask the positions before it), one that
    # covers a whole 64-position chunk, and one longer than the cache (no effect)
    run_sequence(hip, T0=100, n_tokens=2, n_layers=1, window=41)
    run_sequence(hip, T0=150, n_tokens=2, n_layers=1, window=70)
    run_sequence(hip, T0=20, n_tokens=2, n_layers=1, window=64)


@pytest.mark.parametrize("nq,nkv,hd,T0", [(24, 8, 96, 70), (2, 2, 256, 130), (16, 2, 32, 65), (8, 1, 160, 9),
                                          (4, 1, 512, 70), (8, 2, 384, 9), (4, 4, 448, 130)])
def test_decode_head_geometries(hip, nq, nkv, hd, T0):
    # hd a multiple of 32 up to 512 (beyond 256 the new K/V row takes two elements per
    # thread), 1..8 query heads per kv head (q_dim a multiple of 256 for the Q4_K output
    # projection)
    run_sequence(hip, T0=T0, n_tokens=2, n_layers=1, nq=nq, nkv=nkv, hd=hd, hidden=512, inter=512)


# per-layer head geometry: a head_dim-512 layer with one kv head between 128- and 64-wide
# ones (Gemma-4's global layers, LC/src/pipeline.rs:100-101)
MIXED_GEOMS = [(8, 4, 128), (4, 1, 512), (8, 2, 64)]


def _mixed_layers(hidden, inter, cap, seed, formats=None):
    parts = [SmallModel(1, hidden, inter, nq, nkv, hd, cap=cap, seed=seed + 10 * i, formats=formats)
             for i, (nq, nkv, hd) in enumerate(MIXED_GEOMS)]
    return parts, [p.hip_layers(10000.0)[0] for p in parts]


def _mixed_oracle(parts, x, pos, hidden, inter):
    h = x.copy()
    for (nq, nkv, hd), p in zip(MIXED_GEOMS, parts):
        h = oracle.decode_layer(p.layers[0], h, pos, hidden, inter, nq, nkv, hd, 10000.0)
    return h


@pytest.mark.parametrize("formats", [None, {"wv": "q6_k", "down": "q6_k"}])
def test_per_layer_head_geometry(hip, formats):
    """Layers with their own head geometry (the reference decode reads it per layer,
    LC/src/metal/decode.rs:101-110): caches populated at each layer's width, decode_token
    steps, then prefill_q4 and full_pipeline_q4 of a prompt from position 0, every result
    against the oracle's layers at their own geometry.  q_dim / kv_dim are the widest
    layer's; any other width is an error."""
    hidden, inter, T0, n_tok, seq = 512, 1024, 37, 3, 6
    parts, layers = _mixed_layers(hidden, inter, cap=T0 + n_tok + seq + 2, seed=300, formats=formats)
    qmax = max(nq * hd for nq, _, hd in MIXED_GEOMS)
    kvmax = max(nkv * hd for _, nkv, hd in MIXED_GEOMS)
    print(f"[per-layer geometry] {MIXED_GEOMS} formats={formats} q_dim={qmax} kv_dim={kvmax}", flush=True)
    hip.reset_kv_cache()
    for l, ((nq, nkv, hd), p) in enumerate(zip(MIXED_GEOMS, parts)):
        kvd = nkv * hd
        k, v = oracle.gauss(400 + l, T0 * kvd), oracle.gauss(410 + l, T0 * kvd)
        hip.populate_kv_layer(l, k, v, T0, nkv, hd)
        p.layers[0]["k_cache"][: T0 * kvd] = k.astype(np.float16).view(np.uint16)
        p.layers[0]["v_cache"][: T0 * kvd] = v.astype(np.float16).view(np.uint16)
    for i in range(n_tok):
        x = oracle.gauss(500 + i, hidden)
        got = hip.decode_token(layers, x, hidden, inter, qmax, kvmax, 8, 2, 64, 10000.0)
        e = rel_err(got, _mixed_oracle(parts, x, T0 + i, hidden, inter))
        print(f"  decode pos {T0 + i}: rel_err={e:.3e}", flush=True)
        assert e <= REL_TOL, (i, e)
    assert hip.kv_cache_len() == T0 + n_tok
    be = larql_hip.HipBackend(0, strict=False)
    try:
        assert be.decode_token(layers, oracle.gauss(1, hidden), hidden, inter, qmax // 2, kvmax, 8, 2, 64,
                               10000.0) is None
        assert "widest layer" in be.last_error()
    finally:
        be.close()
    xs = np.stack([oracle.gauss(600 + q, hidden) for q in range(seq)])
    ref = [_mixed_oracle(parts, xs[q], q, hidden, inter) for q in range(seq)]
    for entry in ("prefill", "full_pipeline"):
        hip.reset_kv_cache()
        fn = hip.prefill_q4 if entry == "prefill" else hip.full_pipeline_q4
        got = fn(layers, xs, hidden, inter, qmax, kvmax, seq, 8, 2, 64, 10000.0)
        e = max(rel_err(got[q], ref[q]) for q in range(seq))
        print(f"  {entry} seq={seq}: worst rel_err={e:.3e}", flush=True)
        assert e <= REL_TOL, (entry, e)
    assert hip.kv_cache_len() == 0   # full_pipeline left the (reset) decode cache alone


@pytest.mark.parametrize("formats", [{"wv": "q6_k", "down": "q6_k"}, {"wq": "q6_k", "up": "q6_k"},
                                     {"gate": "q6_k", "wo": "q6_k"}])
def test_decode_mixed_projection_formats(hip, formats):
    # Q4_K_M-style layers: some projections Q6_K (split Q|K|V launches, gate then up with
    # silu(gate) * up in the up epilogue)
    run_sequence(hip, T0=40, n_tokens=2, n_layers=2, formats=formats)


@pytest.mark.parametrize("formats", [
    {"gate": "q4_kf", "up": "q4_kf", "down": "q4_kf"},               # Q4_K attention, GGUF FFN
    {n: "q4_kf" for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")},
    {n: "q4_kf160" for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")},
    {"wq": "q4_kf", "wk": "q4_kf160", "wv": "q6_k", "gate": "q4_kf160", "up": "q4_kf"},
])
def test_decode_q4kf_layers(hip, formats):
    """Q4_KF projections in both byte layouts (144-byte GGUF as the reference's GPU decode
    reads it, 160-byte pre-baked), fused where a group shares format and layout, split
    otherwise; decode against the oracle layer."""
    run_sequence(hip, T0=30, n_tokens=2, n_layers=2, formats=formats)


@pytest.mark.parametrize("formats,variant", [
    ({n: "q8_0" for n in ("wq", "wk", "wv", "wo")} | {n: "q4_0" for n in ("gate", "up", "down")}, None),
    ({"wq": "q8_0", "wv": "q8_0", "down": "q4_0"}, None),                     # mixed with Q4_K
    ({n: "q8_0" for n in ("wq", "wk", "wv", "wo")} | {n: "q4_0" for n in ("gate", "up", "down")},
     dict(has_post_norms=True, norm_offset=1.0, activation="gelu_tanh", layer_scalar=0.5)),
])
def test_decode_q8_attention_q4_0_ffn(hip, formats, variant):
    """Q8_0 attention projections and Q4_0 FFN projections (the reference GPU decode's Q8 and
    Q4_0 paths: the normed input quantized by quantize_to_q8, bit-exact block dots; the Q4_0
    down projection on the f32 activation), alone, mixed with Q4_K, and in a post-norm layer."""
    run_sequence(hip, T0=21, n_tokens=2, n_layers=2, formats=formats, variant=variant)


def _oracle_positions(m, x, hidden, inter, nq, nkv, hd, rope):
    out = []
    for p in range(x.shape[0]):
        h = x[p].copy()
        for L in m.layers:
            h = oracle.decode_layer(L, h, p, hidden, inter, nq, nkv, hd, rope)
        out.append(h)
    return np.stack(out)


@pytest.mark.parametrize("seq,formats", [(1, None), (6, None),
                                         (4, {n: "q8_0" for n in ("wq", "wk", "wv", "wo")} |
                                          {n: "q4_0" for n in ("gate", "up", "down")})])
def test_full_pipeline_q4_matches_oracle_and_keeps_cache(hip, seq, formats):
    """full_pipeline_q4 (backend.rs:71-84): positions 0..seq-1 with causal attention among
    themselves only; every position's hidden state against the oracle, and the decode cache
    (9 populated positions) neither read nor changed: the next decode_token continues it."""
    n_layers, hidden, inter, nq, nkv, hd, T0 = 2, 512, 1024, 8, 2, 64, 9
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=T0 + seq + 2, seed=61, formats=formats)
    layers = m.hip_layers(10000.0)
    kvd = nkv * hd
    hip.reset_kv_cache()
    for l in range(n_layers):
        k, v = oracle.gauss(960 + l, T0 * kvd), oracle.gauss(970 + l, T0 * kvd)
        hip.populate_kv_layer(l, k, v, T0, nkv, hd)
    x = np.stack([oracle.gauss(990 + p, hidden) for p in range(seq)])
    got = hip.full_pipeline_q4(layers, x, hidden, inter, nq * hd, kvd, seq, nq, nkv, hd, 10000.0)
    ref = _oracle_positions(m, x, hidden, inter, nq, nkv, hd, 10000.0)
    e = max(rel_err(got[p], ref[p]) for p in range(seq))
    print(f"[full pipeline] seq={seq} formats={formats}: worst rel_err={e:.3e}", flush=True)
    assert e <= REL_TOL
    assert hip.kv_cache_len() == T0
    for l, L in enumerate(m.layers):   # the oracle's caches: the populated rows again
        L["k_cache"][:] = 0
        L["v_cache"][:] = 0
        L["k_cache"][: T0 * kvd] = oracle.gauss(960 + l, T0 * kvd).astype(np.float16).view(np.uint16)
        L["v_cache"][: T0 * kvd] = oracle.gauss(970 + l, T0 * kvd).astype(np.float16).view(np.uint16)
    nxt = oracle.gauss(999, hidden)
    got = hip.decode_token(layers, nxt, hidden, inter, nq * hd, kvd, nq, nkv, hd, 10000.0)
    ref = nxt.copy()
    for L in m.layers:
        ref = oracle.decode_layer(L, ref, T0, hidden, inter, nq, nkv, hd, 10000.0)
    assert rel_err(got, ref) <= REL_TOL


@pytest.mark.parametrize("n_layers,inter,hidden", [(3, 1024, 512), (2, 10240, 2560)])
def test_multi_layer_q4_ffn_matches_oracle(hip, n_layers, inter, hidden):
    """multi_layer_q4_ffn (backend.rs:86-96; Metal ops/q4_batched.rs:97-212): per layer
    quantize_to_q8, Q4_0 gate and up (block-integer order), silu(gate) * up, Q4_0 down on the
    f32 activation; layers chained output to input."""
    layers_q4, x = [], oracle.gauss(1200, hidden)
    for l in range(n_layers):
        layers_q4.append((q4_0(inter, hidden, 1210 + l, 0.05), q4_0(inter, hidden, 1220 + l, 0.05),
                          q4_0(hidden, inter, 1230 + l, 0.05)))
    got = hip.multi_layer_q4_ffn(layers_q4, x, inter, hidden)
    ref = x.copy()
    for g, u, d in layers_q4:
        q8, q8s = oracle.quantize_to_q8(ref)
        gs = oracle.q4_0_matvec_blockint(g, q8, q8s, inter, hidden)
        us = oracle.q4_0_matvec_blockint(u, q8, q8s, inter, hidden)
        ref = oracle.q4_0_f32_matvec(d, oracle.silu_gate_up(gs, us), hidden, inter)
    e = rel_err(got, ref)
    print(f"[multi-layer q4 ffn] {n_layers} x [{inter}x{hidden}]: rel_err={e:.3e}", flush=True)
    assert e <= REL_TOL


def test_prefill_q4_q4kf_layers(hip):
    """A prompt through Q4_KF layers (run position by position through the decode kernels)."""
    n_layers, hidden, inter, nq, nkv, hd, seq = 2, 512, 1024, 8, 2, 64, 7
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=19,
                   formats={"gate": "q4_kf", "up": "q4_kf", "down": "q4_kf", "wo": "q4_kf160"})
    layers = m.hip_layers(10000.0)
    x = np.stack([oracle.gauss(880 + p, hidden) for p in range(seq)])
    hip.reset_kv_cache()
    got = hip.prefill_q4(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)
    worst = 0.0
    for p in range(seq):
        ref = x[p].copy()
        for L in m.layers:
            ref = oracle.decode_layer(L, ref, p, hidden, inter, nq, nkv, hd, 10000.0)
        worst = max(worst, rel_err(got[p], ref))
    print(f"[prefill q4kf] worst rel_err={worst:.3e}", flush=True)
    assert worst <= REL_TOL


VARIANTS = [
    dict(norm_offset=1.0),                                                    # Gemma 2/3 norm weights
    dict(activation="gelu_tanh"),
    dict(has_post_norms=True, norm_offset=1.0, activation="gelu_tanh"),       # Gemma-3-style layer
    dict(has_post_norms=True, ffn_norm_weights=False),                        # weight-free pre/post-FFN norms
    dict(has_v_norm=True, layer_scalar=0.5, rotary_dim=32),                   # Gemma-4-style V-norm, scalar
]


@pytest.mark.parametrize("variant", VARIANTS)
def test_decode_layer_variants(hip, variant):
    """FullPipelineLayer variants (larql-compute/src/pipeline.rs:76-115) on the decode step
    against the oracle layer of the same variant: norm offset, GELU-tanh, post-norms with
    and without pre/post-FFN weights, V-norm, layer scalar, partial rotary."""
    run_sequence(hip, T0=40, n_tokens=2, n_layers=2, variant=variant)


@pytest.mark.parametrize("variant", VARIANTS[1:3] + VARIANTS[4:])
def test_decode_layer_variants_mixed_formats(hip, variant):
    # separate gate and up launches carry the activation in the up epilogue
    run_sequence(hip, T0=12, n_tokens=2, n_layers=1, formats={"gate": "q6_k", "wv": "q6_k"}, variant=variant)


@pytest.mark.parametrize("variant", VARIANTS)
def test_prefill_q4_layer_variants(hip, variant):
    """The batched prompt pass with each layer variant: every position within the bar."""
    n_layers, hidden, inter, nq, nkv, hd, seq = 2, 512, 1024, 8, 2, 64, 12
    print(f"[prefill variant] {variant}", flush=True)
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=91, variant=variant)
    layers = m.hip_layers(10000.0)
    x = np.stack([oracle.gauss(850 + p, hidden) for p in range(seq)])
    hip.reset_kv_cache()
    got = hip.prefill_q4(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)
    worst = 0.0
    for p in range(seq):
        ref = x[p].copy()
        for L in m.layers:
            ref = oracle.decode_layer(L, ref, p, hidden, inter, nq, nkv, hd, 10000.0)
        worst = max(worst, rel_err(got[p], ref))
    print(f"  worst position rel_err={worst:.3e}", flush=True)
    assert worst <= REL_TOL


@pytest.mark.parametrize("seq,formats,window", [(6, {"wv": "q6_k"}, 0), (20, {"wo": "q6_k", "down": "q6_k"}, 0),
                                                 (6, {"up": "q6_k"}, 0), (6, None, 0), (70, None, 0),
                                                 (70, None, 37)])
def test_prefill_q4_matches_oracle_and_decode(hip, seq, formats, window):
    """prefill_q4 (backend.rs:139-152): a prompt from position 0; every position's hidden
    state against the oracle layers, the cache left at seq positions, and the next
    decode_token against decoding the prompt token by token.  Layers with gate/up fused
    in Q4_K take the batched pass (Q4_K and Q6_K GEMMs with f32 operands, prompt-mode
    attention: within the 1e-3 bar); split gate/up runs position
    by position (bit-identical to token-by-token decode)."""
    n_layers, hidden, inter, nq, nkv, hd = 2, 512, 1024, 8, 2, 64
    print(f"[prefill] seq={seq} formats={formats} window={window}", flush=True)
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=77, formats=formats)
    layers = m.hip_layers(10000.0, window)
    x = np.stack([oracle.gauss(8000 + p, hidden) for p in range(seq)])
    hip.reset_kv_cache()
    got = hip.prefill_q4(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)
    assert got is not None and hip.kv_cache_len() == seq
    worst = 0.0
    for p in range(seq):
        ref = x[p].copy()
        for L in m.layers:
            ref = oracle.decode_layer(L, ref, p, hidden, inter, nq, nkv, hd, 10000.0, window=window)
        e = rel_err(got[p], ref)
        worst = max(worst, e)
        assert e <= REL_TOL, (p, e)
    print(f"  worst position rel_err={worst:.3e}", flush=True)
    nxt = oracle.gauss(9000, hidden)
    after_prefill = hip.decode_token(layers, nxt, hidden, inter, nq * hd, nkv * hd, nq, nkv, hd, 10000.0)
    hip.reset_kv_cache()
    for p in range(seq):
        hip.decode_token(layers, x[p], hidden, inter, nq * hd, nkv * hd, nq, nkv, hd, 10000.0)
    stepwise = hip.decode_token(layers, nxt, hidden, inter, nq * hd, nkv * hd, nq, nkv, hd, 10000.0)
    if formats and ("gate" in formats or "up" in formats):
        assert np.array_equal(after_prefill, stepwise)
    else:
        e = rel_err(after_prefill, stepwise.astype(np.float64))
        print(f"  next token after batched prefill vs stepwise: rel_err={e:.3e}", flush=True)
        assert e <= REL_TOL


PROMPT_OPTS = [(True, 0.0), (False, 1.5), (True, 1.5)]


@pytest.mark.parametrize("entry", ["prefill", "full_pipeline"])
@pytest.mark.parametrize("formats", [None, {"up": "q6_k"}])
@pytest.mark.parametrize("qk_norm,softcap", PROMPT_OPTS)
def test_prompt_attention_options(hip, entry, formats, qk_norm, softcap):
    """use_qk_norm and softcap of prefill_q4 / full_pipeline_q4 (LC/src/metal/shaders/
    fused_attention.rs:79-88, 132-137; LC/src/metal/trait_impl.rs:43-76, 150-192): every
    position against the oracle layers with the same options, on the batched pass (Q4_K
    layers) and position by position (split gate/up).  After prefill_q4 the next
    decode_token (no options) continues from the cache, whose K rows are not normed."""
    n_layers, hidden, inter, nq, nkv, hd, seq = 2, 512, 1024, 8, 2, 64, 10
    print(f"[prompt options] {entry} formats={formats} qk_norm={qk_norm} softcap={softcap}", flush=True)
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=83, formats=formats,
                   variant=dict(attn_scale=0.25))
    for L in m.layers:
        L.update(qk_norm=qk_norm, softcap=softcap, attn_scale=0.25)
    layers = m.hip_layers(10000.0)
    for hl in layers:
        hl.attn_scale = 0.25
    x = np.stack([oracle.gauss(870 + p, hidden) for p in range(seq)])
    hip.reset_kv_cache()
    call = hip.prefill_q4 if entry == "prefill" else hip.full_pipeline_q4
    got = call(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0, use_qk_norm=qk_norm,
               softcap=softcap)
    worst = 0.0
    for p in range(seq):
        ref = x[p].copy()
        for L in m.layers:
            ref = oracle.decode_layer(L, ref, p, hidden, inter, nq, nkv, hd, 10000.0)
        e = rel_err(got[p], ref)
        worst = max(worst, e)
        assert e <= REL_TOL, (p, e)
    print(f"  worst position rel_err={worst:.3e}", flush=True)
    if entry == "prefill":
        assert hip.kv_cache_len() == seq
        nxt = oracle.gauss(879, hidden)
        got = hip.decode_token(layers, nxt, hidden, inter, nq * hd, nkv * hd, nq, nkv, hd, 10000.0)
        ref = nxt.copy()
        for L in m.layers:
            ref = oracle.decode_layer(dict(L, qk_norm=False, softcap=0.0), ref, seq, hidden, inter, nq, nkv, hd,
                                      10000.0)
        assert rel_err(got, ref) <= REL_TOL


def _double_rows_q4k(w, r0, r1, cols):
    """Q4_K rows r0..r1-1 times exactly 2: the f16 d and dmin of each of their 148-byte
    super-blocks doubled (every dequantized weight is d * sc * q - dmin * m)."""
    b = w.reshape(-1, cols // 256, 148).copy()
    hdr = b[r0:r1, :, 0:4].copy().view(np.float16)
    b[r0:r1, :, 0:4] = (hdr * np.float16(2)).view(np.uint8)
    return b.reshape(-1)


@pytest.mark.parametrize("formats", [None, {"up": "q6_k"}])
def test_qk_norm_is_per_query_head(hip, formats):
    """A property the oracle does not enter: with QK-norm on, doubling the Q rows of one
    head leaves every output unchanged (the norm is per query head and comes after the
    linear RoPE; only the 1e-6 inside the root differs); without it the same change moves
    the output.  Doubling the K rows of one kv head does move it (K is not normed)."""
    n_layers, hidden, inter, nq, nkv, hd, seq = 1, 512, 1024, 8, 2, 64, 9
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=87, formats=formats)
    x = np.stack([oracle.gauss(890 + p, hidden) for p in range(seq)])
    args = (x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)

    def run(qk, wq=None, wk=None):
        layers = m.hip_layers(10000.0)
        keep = []
        for arr, field in ((wq, "wq"), (wk, "wk")):
            if arr is not None:   # a fresh buffer: the cached model is rebuilt
                keep.append(arr)
                getattr(layers[0], field).data = arr.ctypes.data
        hip.reset_kv_cache()
        return hip.prefill_q4(layers, *args, use_qk_norm=qk)

    wq2 = _double_rows_q4k(m.layers[0]["wq"], 3 * hd, 4 * hd, hidden)
    wk2 = _double_rows_q4k(m.layers[0]["wk"], hd, 2 * hd, hidden)
    base = run(True)
    e_q = rel_err(run(True, wq=wq2), base.astype(np.float64))
    e_k = rel_err(run(True, wk=wk2), base.astype(np.float64))
    e_off = rel_err(run(False, wq=wq2), run(False).astype(np.float64))
    print(f"[qk-norm invariance] formats={formats}: Q head x2 {e_q:.2e}, K head x2 {e_k:.2e}, "
          f"Q head x2 without norm {e_off:.2e}", flush=True)
    assert e_q <= 1e-5 and e_k > 1e-3 and e_off > 1e-3


@pytest.mark.parametrize("formats", [None, {"wv": "q6_k", "down": "q6_k"}])
def test_prefill_q4_uneven_k_splits(hip, formats):
    """hidden 2560 = 10 super-blocks: the small Q|K|V grids split K four ways as 3, 3, 3
    and 1 super-blocks (the last split shorter), summed in split order, for Q4_K and Q6_K
    weights; every position stays within the bar."""
    n_layers, hidden, inter, nq, nkv, hd, seq = 2, 2560, 1024, 8, 2, 64, 20
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=13, formats=formats)
    layers = m.hip_layers(10000.0)
    x = np.stack([oracle.gauss(200 + p, hidden) for p in range(seq)])
    hip.reset_kv_cache()
    got = hip.prefill_q4(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)
    worst = 0.0
    for p in range(seq):
        ref = x[p].copy()
        for L in m.layers:
            ref = oracle.decode_layer(L, ref, p, hidden, inter, nq, nkv, hd, 10000.0)
        worst = max(worst, rel_err(got[p], ref))
    print(f"[prefill splits] hidden {hidden}: worst rel_err={worst:.3e}", flush=True)
    assert worst <= REL_TOL


def test_prefill_q4_deep_model(hip):
    """The batched pass through 16 layers stays within the bar at every position: its
    error must not compound with depth (fp16 GEMM operands reached 1.8e-3 here)."""
    n_layers, hidden, inter, nq, nkv, hd, seq = 16, 512, 1024, 8, 2, 64, 24
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=5)
    layers = m.hip_layers(10000.0)
    x = np.stack([oracle.gauss(100 + p, hidden) for p in range(seq)])
    hip.reset_kv_cache()
    got = hip.prefill_q4(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)
    worst = 0.0
    for p in range(seq):
        ref = x[p].copy()
        for L in m.layers:
            ref = oracle.decode_layer(L, ref, p, hidden, inter, nq, nkv, hd, 10000.0)
        worst = max(worst, rel_err(got[p], ref))
    print(f"[prefill deep] 16 layers, {seq} positions: worst rel_err={worst:.3e}", flush=True)
    assert worst <= REL_TOL


def test_decode_unsupported_layer_returns_none(hip):
    """A supported layer decodes; the same layer struct flipped to LayerNorm (and then to
    biased up projections) returns None even though its weights match the cached model,
    and flipped to GELU-tanh it decodes as the oracle's GELU layer, not the cached SiLU one."""
    be = larql_hip.HipBackend(0, strict=False)
    try:
        m = SmallModel(1, 256, 256, 2, 1, 128, cap=4)
        layers = m.hip_layers(10000.0)
        x = oracle.gauss(17, 256)
        silu = be.decode_token(layers, x, 256, 256, 256, 128, 2, 1, 128, 10000.0)
        assert silu is not None
        layers[0].norm_type = larql_hip.NORM_LAYER
        assert be.decode_token(layers, x, 256, 256, 256, 128, 2, 1, 128, 10000.0) is None
        assert "LayerNorm" in be.last_error()
        layers[0].norm_type = larql_hip.NORM_RMS
        bias = np.zeros(256, np.float32)
        layers[0].ffn_up_bias = bias.ctypes.data
        assert be.decode_token(layers, x, 256, 256, 256, 128, 2, 1, 128, 10000.0) is None
        assert "bias" in be.last_error()
        layers[0].ffn_up_bias = None
        layers[0].activation = larql_hip.ACT_GELU_TANH
        be.reset_kv_cache()
        gelu = be.decode_token(layers, x, 256, 256, 256, 128, 2, 1, 128, 10000.0)
        L = dict(m.layers[0], activation="gelu_tanh")
        L["k_cache"], L["v_cache"] = np.zeros_like(L["k_cache"]), np.zeros_like(L["v_cache"])
        ref = oracle.decode_layer(L, x, 0, 256, 256, 2, 1, 128, 10000.0)
        assert rel_err(gelu, ref) <= REL_TOL and not np.array_equal(gelu, silu)
    finally:
        be.close()


def cpu_logits(host):
    """Oracle decode of the synthetic model on the same bytes: 32 oracle layers at
    pos = kv_len, final RMSNorm, Q6_K head (LI/src/layer_graph/generate.rs:140-143)."""
    c = host["cfg"]
    ones = np.ones(c["hidden"], np.float32)
    h = host["x"].astype(np.float32)
    for L in host["layers"]:
        layer = dict(L, input_norm=ones, post_attn_norm=ones)
        h = oracle.decode_layer(layer, h, host["kv_len"], c["hidden"], c["inter"], c["nq"], c["nkv"], c["hd"],
                                c["rope"])
    hn = oracle.rms_norm(h, ones)
    return oracle.q6k_matvec(host["head"], hn, c["vocab"], c["hidden"])


@pytest.mark.parametrize("formats", [None, {"wv": "q6_k"}])
def test_model_prefill_dev_matches_trait_prefill(hip, formats):
    """larql_hip_model_prefill_dev (a registered model, device buffers) gives the trait
    prefill_q4's hidden states bit for bit (batched pass, or per position for mixed
    formats), leaves the cache at seq_len, and the next decode_dev continues from it."""
    torch = pytest.importorskip("torch")
    n_layers, hidden, inter, nq, nkv, hd, seq = 2, 512, 1024, 8, 2, 64, 20
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=31, formats=formats)
    layers = m.hip_layers(10000.0)
    x = np.stack([oracle.gauss(600 + p, hidden) for p in range(seq)])
    hip.reset_kv_cache()
    ref = hip.prefill_q4(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)
    nxt = oracle.gauss(700, hidden)
    ref_next = hip.decode_token(layers, nxt, hidden, inter, nq * hd, nkv * hd, nq, nkv, hd, 10000.0)
    model = hip.model(layers, hidden, inter, weights_on_device=False)
    try:
        xd = torch.from_numpy(x.astype(np.float32)).cuda()
        out = torch.empty_like(xd)
        model.prefill_dev(xd, seq, out)
        torch.cuda.synchronize()
        assert hip.kv_cache_len() == seq
        assert np.array_equal(out.cpu().numpy(), ref)
        h = torch.empty(hidden, device="cuda", dtype=torch.float32)
        model.decode_dev(torch.from_numpy(nxt.astype(np.float32)).cuda(), hidden_out=h)
        torch.cuda.synchronize()
        assert np.array_equal(h.cpu().numpy(), ref_next)
    finally:
        model.close()


def test_decode_8b_step_matches_cpu():
    """Full Llama-3-8B-shape decode step: 32 layers, d=4096, 32q/8kv heads, hd 128,
    FFN 14336, Q4_K projections, fp16 KV with 2048 prefilled positions, Q6_K head over
    a 128256 vocab.  Weights are generated and quantized on the device; the CPU oracle
    runs on the same downloaded bytes."""
    torch = pytest.importorskip("torch")
    from larql_hip.synth import LLAMA3_8B, build_llama

    be = larql_hip.HipBackend(0, strict=True)
    try:
        print("[8b] building the synthetic model on the device", flush=True)
        sm = build_llama(be, torch, keep_host=True, log=lambda m: print(m, flush=True), **LLAMA3_8B)
        stream = torch.cuda.Stream()
        be.kv_truncate(2048)
        sm.model.decode_dev(sm.x, logits=sm.logits, stream=stream)
        stream.synchronize()
        got = sm.logits.cpu().numpy()
        assert be.kv_cache_len() == 2049
        print("[8b] gpu logits ready; running the CPU oracle (32 layers)", flush=True)
        ref = cpu_logits(sm.host)
        e = rel_err(got, ref)
        print(f"[8b] rel_err={e:.3e} argmax gpu={int(np.argmax(got))} cpu={int(np.argmax(ref))}", flush=True)
        assert e <= REL_TOL
        assert int(np.argmax(got)) == int(np.argmax(ref))
        sm.model.close()
    finally:
        be.close()


@pytest.mark.parametrize("formats", [None, {"wv": "q6_k"}])
def test_vindex_file_layers_match_direct_layers(hip, tmp_path, formats):
    """Layers sliced from vindex files (interleaved_q4k.bin [gate|up|down] per layer,
    attn_weights_q4k.bin + manifest; pipeline_layer.rs:97-152) run prefill_q4 and
    decode_token bit-identically to the same bytes passed as separate arrays."""
    from larql_hip import vindex

    n_layers, hidden, inter, nq, nkv, hd, seq = 2, 512, 1024, 8, 2, 64, 5
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=seq + 2, seed=41, formats=formats)
    (tmp_path / "interleaved_q4k.bin").write_bytes(
        b"".join(L[n].tobytes() for L in m.layers for n in ("gate", "up", "down")))
    blob, man = b"", []
    for L in m.layers:
        for n in ("wq", "wk", "wv", "wo"):
            man.append({"offset": len(blob), "length": L[n].nbytes,
                        "format": "Q6_K" if m.formats.get(n) == "q6_k" else "Q4_K"})
            blob += L[n].tobytes()
    (tmp_path / "attn_weights_q4k.bin").write_bytes(blob)
    (tmp_path / "attn_weights_q4k_manifest.json").write_text(__import__("json").dumps(man))
    v = vindex.Vindex(str(tmp_path), n_layers, hidden, inter)
    vl = v.pipeline_layers([(L["input_norm"], L["post_attn_norm"]) for L in m.layers], head_dim=hd,
                           num_q_heads=nq, num_kv_heads=nkv, rope_base=10000.0)
    x = np.stack([oracle.gauss(300 + p, hidden) for p in range(seq)])
    outs = []
    for layers in (m.hip_layers(10000.0), vl):
        hip.reset_kv_cache()
        pre = hip.prefill_q4(layers, x, hidden, inter, nq * hd, nkv * hd, seq, nq, nkv, hd, 10000.0)
        nxt = hip.decode_token(layers, oracle.gauss(400, hidden), hidden, inter, nq * hd, nkv * hd, nq, nkv, hd,
                               10000.0)
        outs.append((pre, nxt))
    print(f"[vindex] formats={formats}: prefill and next token compared", flush=True)
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


def test_decode_step_inside_cache_capacity_captures_without_allocating(hip):
    """A decode step inside the KV capacity allocates nothing and synchronises nothing, so it
    records into a HIP graph: here the captured step is the first at T = 65, one more
    position split than any step before it (the attention partials are sized by the
    cache capacity, not by T).  Three replays, with eager work and synchronisations
    between them, give the eager step's hidden state bit for bit."""
    torch = pytest.importorskip("torch")
    n_layers, hidden, inter, nq, nkv, hd, T0 = 2, 512, 1024, 8, 2, 64, 63
    m = SmallModel(n_layers, hidden, inter, nq, nkv, hd, cap=T0 + 3, seed=33)
    kvd = nkv * hd
    hip.reset_kv_cache()
    for l in range(n_layers):
        hip.populate_kv_layer(l, oracle.gauss(7000 + l, T0 * kvd), oracle.gauss(7100 + l, T0 * kvd), T0, nkv, hd)
    model = hip.model(m.hip_layers(10000.0), hidden, inter)
    try:
        side = torch.cuda.Stream()
        x1 = torch.from_numpy(oracle.gauss(7200, hidden)).cuda()
        x2 = torch.from_numpy(oracle.gauss(7201, hidden)).cuda()
        h1 = torch.empty(hidden, device="cuda")
        hg = torch.full((hidden,), 7.0, device="cuda")
        href = torch.empty(hidden, device="cuda")
        model.decode_dev(x1, hidden_out=h1, stream=side)   # T = 64: one position split
        side.synchronize()
        print("[decode-graph] capturing the step at T = 65", flush=True)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            model.decode_dev(x2, hidden_out=hg, stream=side)   # T = 65: two splits
        hip.kv_truncate(T0 + 1)
        model.decode_dev(x2, hidden_out=href, stream=side)
        side.synchronize()
        ref = href.cpu().numpy()
        for rep in range(3):
            hip.kv_truncate(T0 + 1)
            hg.fill_(7.0)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(hg.cpu().numpy().view(np.uint32), ref.view(np.uint32))
        del graph
    finally:
        model.close()
        hip.reset_kv_cache()
