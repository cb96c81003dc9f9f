"""CPU oracle for the LARQL quantized compute path — TEST INFRASTRUCTURE ONLY.

A ctypes view of ``liblarql_oracle.so`` (the plain-C restatement of the
reference CPU backend in ``larql_oracle.c``) and of ``_ref/libq4dot_ref.so``
(the reference's own ``larql-compute/csrc/q4_dot.c`` compiled in place).

Only ``tests/``, ``__graft_entry__.smoke()`` and the cpu_baseline leg of
``bench.py`` import this package, and only to check or time the CPU path.
The product (``liblarql_hip.so`` and its Python binding) never imports it.

Parity status of each function (what pins it against the reference) is
listed in the header of ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblarql_oracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libq4dot_ref.so")

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t

_lib = None
_ref = None


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
        lib = ctypes.CDLL(_LIB_PATH)
        sig = {
            "lo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "lo_decode_f16": (ctypes.c_float, [ctypes.c_uint16]),
            "lo_f32_to_f16_trunc": (ctypes.c_uint16, [ctypes.c_float]),
            "lo_f32_to_f16_rne": (ctypes.c_uint16, [ctypes.c_float]),
            "lo_quantize_to_q8": (None, [_P, _SZ, _P, _P]),
            "lo_quantize_q4_0": (None, [_P, _SZ, _P]),
            "lo_quantize_q4_k": (None, [_P, _SZ, _P]),
            "lo_quantize_q6_k": (None, [_P, _SZ, _P]),
            "lo_quantize_weights_q8": (None, [_P, _SZ, _SZ, _P, _P]),
            "lo_q4_0_matvec_x86": (None, [_P, _P, _P, _P, _SZ, _SZ]),
            "lo_q4_0_matvec_blockint": (None, [_P, _P, _P, _P, _SZ, _SZ]),
            "lo_q4_0_block_dots": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_q4_0_vecmat": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_q4k_matvec": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_q6k_matvec": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_q8_matvec": (None, [_P, _P, _P, _P, _P, _SZ, _SZ]),
            "lo_q4kf_gguf_matvec": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_q4_0_f32_matvec": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_q4kf160_matvec": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_gguf_scale_min": (None, [ctypes.c_int, _P, _P, _P]),
            "lo_q4k_to_gguf": (None, [_P, _SZ, _P]),
            "lo_quantize_q4_k_gguf": (None, [_P, _SZ, _P]),
            "lo_q4k_to_q4kf": (None, [_P, _SZ, _P]),
            "lo_q4k_to_gguf_llamacpp": (None, [_P, _SZ, _P]),
            "lo_q8_block_dots": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_topk_abs": (None, [_P, _SZ, _SZ, _P, _P]),
            "lo_topk_signed": (None, [_P, _SZ, _SZ, _P, _P]),
            "lo_gate_scores_f32": (None, [_P, _P, _P, _SZ, _SZ]),
            "lo_rms_norm": (None, [_P, _P, ctypes.c_float, ctypes.c_double, _P, _SZ]),
            "lo_rope_at": (None, [_P, _SZ, _SZ, _SZ, ctypes.c_double, _SZ]),
            "lo_silu_gate_up": (None, [_P, _P, _P, _SZ]),
            "lo_gelu_tanh_gate_up": (None, [_P, _P, _P, _SZ]),
            "lo_rms_norm_heads": (None, [_P, _SZ, _SZ, ctypes.c_double]),
            "lo_attend_f16": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P]),
            "lo_attend_f16_opts": (None, [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, ctypes.c_int,
                                          ctypes.c_float, _P]),
            "lo_qk_norm_heads": (None, [_P, _SZ, _SZ]),
            "lo_decode_layer": (None, [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_double, ctypes.c_double]),
            "lo_decode_layer_mt": (None, [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_double, ctypes.c_double,
                                           ctypes.c_int]),
            "lo_proj_rows_mt": (None, [ctypes.c_int, _P, _P, ctypes.c_int, _P, _P, _SZ, _SZ, ctypes.c_int]),
            "lo_decode_layer_window": (None, [_P, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_double, ctypes.c_double,
                                              _SZ]),
            "lo_gauss_f32": (None, [ctypes.c_uint64, ctypes.c_float, ctypes.c_float, _P, _SZ]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def ref_lib():
    """The reference's own q4_dot.c (x86 scalar path), or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(_REF_PATH):
        lib = ctypes.CDLL(_REF_PATH)
        lib.q4_0_matvec_c.restype = None
        lib.q4_0_matvec_c.argtypes = [_P, _P, _P, _P, _SZ, _SZ]
        lib.q4_0_vecmat_c.restype = None
        lib.q4_0_vecmat_c.argtypes = [_P, _P, _P, _SZ, _SZ]
        _ref = lib
    return _ref


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ── inputs ──────────────────────────────────────────────────────────────
def gauss(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _load().lo_gauss_f32(ctypes.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), mean, std, _ptr(out), n)
    return out


# ── f16 ─────────────────────────────────────────────────────────────────
def f16_to_f32(bits: int) -> float:
    return _load().lo_f16_to_f32(bits)


def decode_f16(bits: int) -> float:
    return _load().lo_decode_f16(bits)


def f32_to_f16_trunc(v: float) -> int:
    return _load().lo_f32_to_f16_trunc(v)


def f32_to_f16_rne(v: float) -> int:
    return _load().lo_f32_to_f16_rne(v)


# ── quantizers ──────────────────────────────────────────────────────────
def quantize_to_q8(x):
    x = _c(x, np.float32)
    assert x.size % 32 == 0
    q = np.empty(x.size, dtype=np.int8)
    s = np.empty(x.size // 32, dtype=np.float32)
    _load().lo_quantize_to_q8(_ptr(x), x.size, _ptr(q), _ptr(s))
    return q, s


def quantize_q4_0(x):
    x = _c(x, np.float32)
    if x.size % 32:
        raise ValueError("data length must be a multiple of 32")
    out = np.empty(x.size // 32 * 18, dtype=np.uint8)
    _load().lo_quantize_q4_0(_ptr(x), x.size, _ptr(out))
    return out


def quantize_q4_k(x):
    x = _c(x, np.float32)
    if x.size % 256:
        raise ValueError("data length must be a multiple of 256")
    out = np.empty(x.size // 256 * 148, dtype=np.uint8)
    _load().lo_quantize_q4_k(_ptr(x), x.size, _ptr(out))
    return out


def quantize_q6_k(x):
    x = _c(x, np.float32)
    if x.size % 256:
        raise ValueError("data length must be a multiple of 256")
    out = np.empty(x.size // 256 * 210, dtype=np.uint8)
    _load().lo_quantize_q6_k(_ptr(x), x.size, _ptr(out))
    return out


def quantize_weights_q8(w, rows: int, cols: int):
    w = _c(w, np.float32)
    assert w.size == rows * cols and cols % 32 == 0
    q = np.empty(rows * cols, dtype=np.int8)
    s = np.empty(rows * cols // 32, dtype=np.float32)
    _load().lo_quantize_weights_q8(_ptr(w), rows, cols, _ptr(q), _ptr(s))
    return q, s


# ── matvecs ─────────────────────────────────────────────────────────────
def q4_0_matvec_x86(q4, q8x, q8s, rows: int, hidden: int):
    q4, q8x, q8s = _c(q4, np.uint8), _c(q8x, np.int8), _c(q8s, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q4_0_matvec_x86(_ptr(q4), _ptr(q8x), _ptr(q8s), _ptr(out), rows, hidden)
    return out


def q4_0_matvec_blockint(q4, q8x, q8s, rows: int, hidden: int):
    q4, q8x, q8s = _c(q4, np.uint8), _c(q8x, np.int8), _c(q8s, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q4_0_matvec_blockint(_ptr(q4), _ptr(q8x), _ptr(q8s), _ptr(out), rows, hidden)
    return out


def q4_0_block_dots(q4, q8x, rows: int, hidden: int):
    q4, q8x = _c(q4, np.uint8), _c(q8x, np.int8)
    out = np.empty(rows * (hidden // 32), dtype=np.int32)
    _load().lo_q4_0_block_dots(_ptr(q4), _ptr(q8x), _ptr(out), rows, hidden)
    return out.reshape(rows, hidden // 32)


def q4_0_vecmat(act, q4, inter: int, hidden: int):
    act, q4 = _c(act, np.float32), _c(q4, np.uint8)
    out = np.empty(hidden, dtype=np.float32)
    _load().lo_q4_0_vecmat(_ptr(act), _ptr(q4), _ptr(out), inter, hidden)
    return out


def q4k_matvec(q4k, x, rows: int, hidden: int):
    q4k, x = _c(q4k, np.uint8), _c(x, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q4k_matvec(_ptr(q4k), _ptr(x), _ptr(out), rows, hidden)
    return out


def q6k_matvec(q6k, x, rows: int, hidden: int):
    q6k, x = _c(q6k, np.uint8), _c(x, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q6k_matvec(_ptr(q6k), _ptr(x), _ptr(out), rows, hidden)
    return out


def q4_0_f32_matvec(q4, x, rows: int, hidden: int):
    """Q4_0 weights x f32 activation (the reference GPU's q4_f32_matvec order)."""
    q4, x = _c(q4, np.uint8), _c(x, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q4_0_f32_matvec(_ptr(q4), _ptr(x), _ptr(out), rows, hidden)
    return out


def q4kf_gguf_matvec(w, x, rows: int, hidden: int):
    """Q4_KF, 144-byte llama.cpp GGUF block (the reference's GPU decode layout)."""
    w, x = _c(w, np.uint8), _c(x, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q4kf_gguf_matvec(_ptr(w), _ptr(x), _ptr(out), rows, hidden)
    return out


def q4kf160_matvec(w, x, rows: int, hidden: int):
    """Q4_KF, 160-byte block with pre-baked half scales (q4k_to_q4kf)."""
    w, x = _c(w, np.uint8), _c(x, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q4kf160_matvec(_ptr(w), _ptr(x), _ptr(out), rows, hidden)
    return out


def gguf_scale_min(j: int, q12):
    q12 = _c(q12, np.uint8)
    sc, mn = ctypes.c_uint8(0), ctypes.c_uint8(0)
    _load().lo_gguf_scale_min(j, _ptr(q12), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value


def _convert(fn, src, nblocks, out_block):
    src = _c(src, np.uint8)
    out = np.empty(nblocks * out_block, dtype=np.uint8)
    getattr(_load(), fn)(_ptr(src), nblocks, _ptr(out))
    return out


def q4k_to_gguf(q4k):
    return _convert("lo_q4k_to_gguf", q4k, np.asarray(q4k).size // 148, 144)


def q4k_to_q4kf(q4k):
    return _convert("lo_q4k_to_q4kf", q4k, np.asarray(q4k).size // 148, 160)


def q4k_to_gguf_llamacpp(q4k):
    return _convert("lo_q4k_to_gguf_llamacpp", q4k, np.asarray(q4k).size // 148, 144)


def quantize_q4_k_gguf(x):
    x = _c(x, np.float32)
    if x.size % 256:
        raise ValueError("length must be a multiple of 256")
    out = np.empty(x.size // 256 * 144, dtype=np.uint8)
    _load().lo_quantize_q4_k_gguf(_ptr(x), x.size, _ptr(out))
    return out


def q8_matvec(wq, ws, xq, xs, rows: int, hidden: int):
    wq, ws, xq, xs = _c(wq, np.int8), _c(ws, np.float32), _c(xq, np.int8), _c(xs, np.float32)
    out = np.empty(rows, dtype=np.float32)
    _load().lo_q8_matvec(_ptr(wq), _ptr(ws), _ptr(xq), _ptr(xs), _ptr(out), rows, hidden)
    return out


def q8_block_dots(wq, xq, rows: int, hidden: int):
    wq, xq = _c(wq, np.int8), _c(xq, np.int8)
    out = np.empty(rows * (hidden // 32), dtype=np.int32)
    _load().lo_q8_block_dots(_ptr(wq), _ptr(xq), _ptr(out), rows, hidden)
    return out.reshape(rows, hidden // 32)


# ── KNN ─────────────────────────────────────────────────────────────────
def topk_abs(scores, k: int):
    s = _c(scores, np.float32)
    k = min(k, s.size)
    idx = np.empty(k, dtype=np.uint32)
    val = np.empty(k, dtype=np.float32)
    _load().lo_topk_abs(_ptr(s), s.size, k, _ptr(idx), _ptr(val))
    return idx, val


def topk_signed(scores, k: int):
    s = _c(scores, np.float32)
    k = min(k, s.size)
    idx = np.empty(k, dtype=np.uint32)
    val = np.empty(k, dtype=np.float32)
    _load().lo_topk_signed(_ptr(s), s.size, k, _ptr(idx), _ptr(val))
    return idx, val


def gate_scores_f32(gate, x, features: int, hidden: int):
    gate, x = _c(gate, np.float32), _c(x, np.float32)
    out = np.empty(features, dtype=np.float32)
    _load().lo_gate_scores_f32(_ptr(gate), _ptr(x), _ptr(out), features, hidden)
    return out


# ── decode numerics ─────────────────────────────────────────────────────
def rms_norm(x, w, offset: float = 0.0, eps: float = 1e-6):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    wk = _c(w, np.float32) if w is not None else None
    _load().lo_rms_norm(_ptr(x), _ptr(wk) if wk is not None else None, offset, eps, _ptr(out), x.size)
    return out


def rope_at(x, num_heads: int, head_dim: int, base: float, pos: int, rotary_dim: int | None = None):
    x = np.array(x, dtype=np.float32, copy=True)
    _load().lo_rope_at(_ptr(x), num_heads, head_dim, rotary_dim or head_dim, base, pos)
    return x


def silu_gate_up(g, u):
    g, u = _c(g, np.float32), _c(u, np.float32)
    out = np.empty_like(g)
    _load().lo_silu_gate_up(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


def gelu_tanh_gate_up(g, u):
    g, u = _c(g, np.float32), _c(u, np.float32)
    out = np.empty_like(g)
    _load().lo_gelu_tanh_gate_up(_ptr(g), _ptr(u), _ptr(out), g.size)
    return out


def rms_norm_heads(x, num_heads: int, head_dim: int, eps: float = 1e-6):
    x = np.array(x, dtype=np.float32, copy=True)
    _load().lo_rms_norm_heads(_ptr(x), num_heads, head_dim, eps)
    return x


def attend_f16(q, kc, vc, T: int, num_q: int, num_kv: int, head_dim: int, scale: float, t_start: int = 0,
               qk_norm: bool = False, softcap: float = 0.0):
    """Attention of the last query row over cache positions t_start .. T-1 (t_start > 0 is
    the sliding window, LC/src/metal/shaders/kv_attention.rs:35); qk_norm / softcap as the
    prompt attention's options (LC/src/metal/shaders/fused_attention.rs:79-88, 132-137)."""
    kvd = num_kv * head_dim
    q = _c(q, np.float32)
    kc = _c(np.asarray(kc)[t_start * kvd:T * kvd], np.uint16)
    vc = _c(np.asarray(vc)[t_start * kvd:T * kvd], np.uint16)
    out = np.empty(num_q * head_dim, dtype=np.float32)
    if qk_norm or softcap != 0.0:
        _load().lo_attend_f16_opts(_ptr(q), _ptr(kc), _ptr(vc), T - t_start, num_q, num_kv, head_dim, scale,
                                   int(bool(qk_norm)), softcap, _ptr(out))
    else:
        _load().lo_attend_f16(_ptr(q), _ptr(kc), _ptr(vc), T - t_start, num_q, num_kv, head_dim, scale, _ptr(out))
    return out


def qk_norm_heads(x, num_heads: int, head_dim: int):
    x = np.array(x, dtype=np.float32, copy=True)
    _load().lo_qk_norm_heads(_ptr(x), num_heads, head_dim)
    return x


_PROJ = ("wq", "wk", "wv", "wo", "gate", "up", "down")


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in _PROJ + ("input_norm", "post_attn_norm", "k_cache", "v_cache")] + \
               [("fmt", ctypes.c_int * 7),
                ("pre_ffn_norm", ctypes.c_void_p), ("post_ffn_norm", ctypes.c_void_p),
                ("norm_offset", ctypes.c_float), ("has_post_norms", ctypes.c_int),
                ("activation", ctypes.c_int), ("has_v_norm", ctypes.c_int),
                ("layer_scalar", ctypes.c_float), ("rotary_dim", ctypes.c_size_t),
                ("attn_scale", ctypes.c_float)] + [(n + "_s", ctypes.c_void_p) for n in _PROJ] + \
               [("qk_norm", ctypes.c_int), ("softcap", ctypes.c_float),
                ("k_cache32", ctypes.c_void_p), ("v_cache32", ctypes.c_void_p)]


def decode_layer(layer: dict, h, pos: int, hidden: int, inter: int, num_q: int, num_kv: int,
                 head_dim: int, rope_base: float, eps: float = 1e-6, window: int = 0, threads: int = 1):
    """One decoder layer on the CPU.  ``layer`` holds numpy arrays keyed as the
    lo_layer_t fields; k_cache / v_cache (uint16 fp16 bits, or float32 for the reference's f32
    cache: the new row stored unrounded) are updated in place.
    window > 0 attends over the last `window` positions only.  ``layer["formats"]``
    (optional) maps a projection name to "q6_k" (Q6_K bytes), "q4_kf" (Q4_KF, 144-byte GGUF),
    "q4_kf160" (Q4_KF, 160-byte), "q8_0" (int8 weights, scales under name + "_s") or "q4_0";
    the default is Q4_K.
    Optional layer variants (FullPipelineLayer, LC/src/pipeline.rs:76-115):
    pre_ffn_norm / post_ffn_norm (arrays or None), norm_offset, has_post_norms,
    activation ("silu" | "gelu_tanh"), has_v_norm, layer_scalar, rotary_dim, attn_scale; and the
    prompt-attention options qk_norm (bool) and softcap (float, 0 = off) of prefill_q4 /
    full_pipeline_q4."""
    keep = {}
    st = _Layer()
    for name, dt in (("wq", np.uint8), ("wk", np.uint8), ("wv", np.uint8), ("wo", np.uint8),
                     ("gate", np.uint8), ("up", np.uint8), ("down", np.uint8),
                     ("input_norm", np.float32), ("post_attn_norm", np.float32)):
        a = _c(layer[name], dt)
        keep[name] = a
        setattr(st, name, a.ctypes.data)
    for name in ("pre_ffn_norm", "post_ffn_norm"):
        if layer.get(name) is not None:
            a = _c(layer[name], np.float32)
            keep[name] = a
            setattr(st, name, a.ctypes.data)
    fm = layer.get("formats", {})
    codes = {"q4_k": 0, "q6_k": 1, "q4_kf": 2, "q4_kf160": 3, "q8_0": 4, "q4_0": 5}
    for i, name in enumerate(_PROJ):
        st.fmt[i] = codes[fm.get(name, "q4_k")]
        if st.fmt[i] == 4:   # Q8_0: int8 bytes in layer[name], f32 scales in layer[name + "_s"]
            a = _c(layer[name + "_s"], np.float32)
            keep[name + "_s"] = a
            setattr(st, name + "_s", a.ctypes.data)
    for name in ("k_cache", "v_cache"):
        a = layer[name]
        assert a.dtype in (np.uint16, np.float32) and a.flags["C_CONTIGUOUS"]
        # uint16: fp16 bits; float32: the f32 cache (the new row stored unrounded)
        setattr(st, name + ("32" if a.dtype == np.float32 else ""), a.ctypes.data)
    st.norm_offset = float(layer.get("norm_offset", 0.0))
    st.has_post_norms = int(bool(layer.get("has_post_norms", False)))
    st.activation = {"silu": 0, "gelu_tanh": 1}[layer.get("activation", "silu")]
    st.has_v_norm = int(bool(layer.get("has_v_norm", False)))
    st.layer_scalar = float(layer.get("layer_scalar", 0.0))
    st.rotary_dim = int(layer.get("rotary_dim", 0))
    st.attn_scale = float(layer.get("attn_scale", 0.0))
    st.qk_norm = int(bool(layer.get("qk_norm", False)))
    st.softcap = float(layer.get("softcap", 0.0))
    h = np.array(h, dtype=np.float32, copy=True)
    if threads > 1:
        assert window == 0
        _load().lo_decode_layer_mt(ctypes.byref(st), _ptr(h), pos, hidden, inter, num_q, num_kv,
                                   head_dim, rope_base, eps, threads)
    else:
        _load().lo_decode_layer_window(ctypes.byref(st), _ptr(h), pos, hidden, inter, num_q, num_kv,
                                       head_dim, rope_base, eps, window)
    return h


_FMT_CODES = {"q4_k": 0, "q6_k": 1, "q4_kf": 2, "q4_kf160": 3, "q8_0": 4, "q4_0": 5}


def proj_rows_mt(fmt: str, w, x, rows: int, cols: int, threads: int, scales=None, q8_input: bool = False):
    """One projection out = W x with its rows split over `threads` threads (the one-thread
    kernel on each contiguous slice: identical output).  fmt as decode_layer's formats;
    Q8_0 takes int8 weights and f32 `scales`; q8_input: Q4_0 against the Q8-quantized x."""
    code = _FMT_CODES[fmt]
    w = _c(w, np.int8 if code == 4 else np.uint8)
    x = _c(x, np.float32)
    sc = _c(scales, np.float32) if scales is not None else None
    out = np.empty(rows, dtype=np.float32)
    _load().lo_proj_rows_mt(code, _ptr(w), _ptr(sc) if sc is not None else None, int(q8_input), _ptr(x),
                            _ptr(out), rows, cols, threads)
    return out


# ── the reference's own C kernel (x86 scalar path), when built ──────────
def ref_q4_0_matvec(q4, q8x, q8s, rows: int, hidden: int):
    lib = ref_lib()
    if lib is None:
        return None
    q4, q8x, q8s = _c(q4, np.uint8), _c(q8x, np.int8), _c(q8s, np.float32)
    out = np.empty(rows, dtype=np.float32)
    lib.q4_0_matvec_c(_ptr(q4), _ptr(q8x), _ptr(q8s), _ptr(out), rows, hidden)
    return out


def ref_q4_0_vecmat(act, q4, inter: int, hidden: int):
    lib = ref_lib()
    if lib is None:
        return None
    act, q4 = _c(act, np.float32), _c(q4, np.uint8)
    out = np.empty(hidden, dtype=np.float32)
    lib.q4_0_vecmat_c(_ptr(act), _ptr(q4), _ptr(out), inter, hidden)
    return out
