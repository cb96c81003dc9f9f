"""Python binding of liblarql_hip — the MI355X backend for LARQL's quantized path.

``HipBackend`` mirrors the reference trait ``ComputeBackend``
(larql-main/crates/larql-compute/src/backend.rs:24-164): the same method names,
argument meaning and ``Option`` behaviour — a method returns ``None`` when the
backend cannot serve the request, and the reason is in ``last_error()``.
Construct with ``strict=True`` to raise ``LarqlHipError`` instead.

Importing this module loads ``liblarql_hip.so`` (built next to this file by
``make -C encoding-experiment_amd``) and raises if it is missing: there is no
CPU fallback behind this binding.

The ``*_dev`` methods take device-resident tensors (anything with
``data_ptr()``, e.g. torch tensors on ``cuda``) and only enqueue work.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liblarql_hip.so")

Q4_0, Q4_K, Q4_KF, Q6_K, Q8_0, F32 = 0, 1, 2, 3, 4, 5
FORMAT_NAMES = {Q4_0: "Q4_0", Q4_K: "Q4_K", Q4_KF: "Q4_KF", Q6_K: "Q6_K", Q8_0: "Q8_0", F32: "F32"}
TOPK_MAX, KNN_MAX_LAYERS = 512, 64
NOALLOC_SCRATCH_BYTES = 8 << 20

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_DEVICE, ERR_NOMEM, ERR_STATE = 0, -1, -2, -3, -4, -5

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_I = ctypes.c_int
_U64 = ctypes.c_uint64


class LarqlHipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


# name -> (restype, argtypes); every symbol declared in include/larql_hip.h
SIGNATURES = {
    "larql_hip_ctx_create": (_I, [_I, ctypes.POINTER(_P)]),
    "larql_hip_ctx_destroy": (None, [_P]),
    "larql_hip_last_error": (ctypes.c_char_p, [_P]),
    "larql_hip_name": (ctypes.c_char_p, []),
    "larql_hip_device_info": (_I, [_P, ctypes.c_char_p, _SZ]),
    "larql_hip_has_q4": (_I, [_P]),
    "larql_hip_has_kv_cache": (_I, [_P]),
    "larql_hip_synchronize": (_I, [_P]),
    "larql_hip_register_weight": (_I, [_P, _I, _P, _SZ, _P, _SZ, _SZ, ctypes.POINTER(_U64)]),
    "larql_hip_register_weight_device": (_I, [_P, _I, _P, _SZ, _P, _SZ, _SZ, ctypes.POINTER(_U64)]),
    "larql_hip_release_weight": (_I, [_P, _U64]),
    "larql_hip_forget_host": (_I, [_P, _P]),
    "larql_hip_weight_device_bytes": (_I, [_P, _U64, ctypes.POINTER(_SZ)]),
    "larql_hip_q4_matvec": (_I, [_P, _P, _SZ, _P, _P, _P, _SZ, _SZ]),
    "larql_hip_q4_vecmat": (_I, [_P, _P, _P, _SZ, _P, _SZ, _SZ]),
    "larql_hip_q4_matvec_pair_batch": (_I, [_P, _P, _SZ, _P, _SZ, _P, _SZ, _P, _P, _SZ, _SZ]),
    "larql_hip_vecmat_dev": (_I, [_P, _U64, _P, _P, _P]),
    "larql_hip_read_floor_dev": (_I, [_P, _U64, ctypes.c_uint, ctypes.c_uint, _P, _SZ, _P]),
    "larql_hip_q4k_launch_shape": (_I, [_P, _U64, _P, _P, _P, _P, _P, _P, _P]),
    "larql_hip_pair_batch_dev": (_I, [_P, _U64, _U64, _P, _SZ, _P, _P, _P]),
    "larql_hip_q4k_matvec": (_I, [_P, _P, _SZ, _P, _P, _SZ, _SZ]),
    "larql_hip_q6k_matvec": (_I, [_P, _P, _SZ, _P, _P, _SZ, _SZ]),
    "larql_hip_q4k_matmul": (_I, [_P, _P, _SZ, _P, _SZ, _P, _SZ, _SZ]),
    "larql_hip_matmul": (_I, [_P, _P, _SZ, _SZ, _P, _SZ, _I, _P]),
    "larql_hip_matmul_dev": (_I, [_P, _P, _SZ, _SZ, _P, _SZ, _I, _P, _P]),
    "larql_hip_quantize_to_q8": (_I, [_P, _P, _SZ, _P, _P]),
    "larql_hip_q8_matvec": (_I, [_P, _P, _SZ, _P, _P, _P, _SZ, _P, _SZ, _SZ]),
    "larql_hip_matvec_dev": (_I, [_P, _U64, _P, _P, _P, _SZ, _P]),
    "larql_hip_quantize_to_q8_dev": (_I, [_P, _P, _SZ, _SZ, _P, _P, _P]),
    "larql_hip_quantize_weights": (_I, [_P, _I, _P, _SZ, _P, _P]),
    "larql_hip_quantize_weights_dev": (_I, [_P, _I, _P, _SZ, _P, _P, _P]),
    # vindex gate-KNN
    "larql_hip_gate_knn": (_I, [_P, _I, _P, _SZ, _SZ, _SZ, _P, _SZ, _SZ, _P, _P]),
    "larql_hip_gate_knn_dev": (_I, [_P, _P, _SZ, _P, _SZ, _SZ, _P, _P, _P]),
    "larql_hip_gate_scores_dev": (_I, [_P, _P, _SZ, _P, _SZ, _P, _P]),
    "larql_hip_topk_dev": (_I, [_P, _P, _SZ, _SZ, _SZ, _I, _P, _P, _P]),
    "larql_hip_lm_head_knn": (_I, [_P, _P, _SZ, _P, _SZ, _SZ, _SZ, _P, _P]),
    "larql_hip_lm_head_knn_dev": (_I, [_P, _U64, _P, _SZ, _SZ, _P, _P, _P]),
    "larql_hip_lm_head_knn_dev_noalloc": (_I, [_P, _U64, _P, _SZ, _SZ, _P, _P, _P]),
    # decode step (structs declared below; pointers passed as void*)
    "larql_hip_decode_token": (_I, [_P, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P]),
    "larql_hip_prefill_q4": (_I, [_P, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float,
                                  ctypes.c_int, ctypes.c_float, _P]),
    "larql_hip_full_pipeline_q4": (_I, [_P, _P, _SZ, _P, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, _SZ, ctypes.c_float,
                                        ctypes.c_int, ctypes.c_float, _P]),
    "larql_hip_multi_layer_q4_ffn": (_I, [_P, _P, _SZ, _P, _SZ, _SZ, _P]),
    "larql_hip_populate_kv_layer": (_I, [_P, _SZ, _P, _P, _SZ, _SZ, _SZ]),
    "larql_hip_reset_kv_cache": (_I, [_P]),
    "larql_hip_kv_cache_len": (_I, [_P, ctypes.POINTER(_SZ)]),
    "larql_hip_kv_truncate": (_I, [_P, _SZ]),
    "larql_hip_populate_kv_layer_f16_dev": (_I, [_P, _SZ, _P, _P, _SZ, _SZ, _SZ]),
    "larql_hip_model_create": (_I, [_P, _P, _SZ, _SZ, _SZ, _I, ctypes.POINTER(_P)]),
    "larql_hip_model_set_head": (_I, [_P, _P, _P, _SZ, _P, ctypes.c_float, _I]),
    "larql_hip_model_destroy": (_I, [_P, _P]),
    "larql_hip_model_decode_dev": (_I, [_P, _P, _P, _P, _P, _P]),
    "larql_hip_model_prefill_dev": (_I, [_P, _P, _P, _SZ, _P, _P]),
}

NORM_RMS, NORM_LAYER = 0, 1
FFN_GATED, FFN_STANDARD = 0, 1
ACT_SILU, ACT_GELU_TANH = 0, 1


class QuantWeight(ctypes.Structure):
    """larql_quant_weight / QuantWeight (larql-compute/src/pipeline.rs:22-27)."""
    _fields_ = [("data", _P), ("len", _SZ), ("scales", _P), ("format", _I)]


class Q4FfnLayer(ctypes.Structure):
    """larql_q4_ffn_layer: one (gate, up, down_t) Q4_0 triple of multi_layer_q4_ffn."""
    _fields_ = [("gate", _P), ("gate_len", _SZ), ("up", _P), ("up_len", _SZ), ("down", _P), ("down_len", _SZ)]


class PipelineLayer(ctypes.Structure):
    """larql_pipeline_layer / FullPipelineLayer (larql-compute/src/pipeline.rs:60-120)."""
    _fields_ = [
        ("wq", QuantWeight), ("wk", QuantWeight), ("wv", QuantWeight), ("wo", QuantWeight),
        ("gate", QuantWeight), ("up", QuantWeight), ("down", QuantWeight),
        ("input_norm", _P), ("post_attn_norm", _P), ("pre_ffn_norm", _P), ("post_ffn_norm", _P),
        ("input_norm_bias", _P), ("post_attn_norm_bias", _P),
        ("norm_offset", ctypes.c_float), ("qk_norm_offset", ctypes.c_float), ("eps", ctypes.c_float),
        ("has_post_norms", _I), ("norm_type", _I), ("ffn_type", _I), ("activation", _I),
        ("attn_scale", ctypes.c_float), ("head_dim", _SZ), ("num_q_heads", _SZ), ("num_kv_heads", _SZ),
        ("rope_base", ctypes.c_float), ("rotary_dim", _SZ), ("sliding_window", _SZ),
        ("has_v_norm", _I), ("layer_scalar", ctypes.c_float),
        ("ffn_up_bias", _P), ("ffn_down_bias", _P),
    ]


def _addr(a):
    """Address of a numpy array (host) or tensor-like (device) or int."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        assert a.flags["C_CONTIGUOUS"]
        return a.ctypes.data
    return a.data_ptr()


def _nbytes(a):
    if isinstance(a, np.ndarray):
        return a.nbytes
    return a.numel() * a.element_size()


def make_layer(wq, wk, wv, wo, gate, up, down, input_norm, post_attn_norm, *, head_dim, num_q_heads,
               num_kv_heads, rope_base, eps=1e-6, attn_scale=None, fmt=Q4_K, formats=None,
               rotary_dim=0, sliding_window=0, norm_offset=0.0, has_post_norms=False, pre_ffn_norm=None,
               post_ffn_norm=None, activation=ACT_SILU, has_v_norm=False, layer_scalar=0.0, scales=None):
    """A FullPipelineLayer over numpy (host) or device tensors of reference-layout bytes:
    the Llama layer by default, or the variants of larql-compute/src/pipeline.rs:76-115
    (norm offset, post-norms with pre/post-FFN norm weights, GELU-tanh, V-norm, layer
    scalar).  scales: projection name -> f32 scales of a Q8_0 weight (QuantWeight.scales).
    Keep the source arrays alive while the struct is in use."""
    L = PipelineLayer()
    names = ("wq", "wk", "wv", "wo", "gate", "up", "down")
    for name, arr in zip(names, (wq, wk, wv, wo, gate, up, down)):
        f = (formats or {}).get(name, fmt)
        setattr(L, name, QuantWeight(_addr(arr), _nbytes(arr), _addr((scales or {}).get(name)), f))
    L.input_norm = _addr(input_norm)
    L.post_attn_norm = _addr(post_attn_norm)
    L.pre_ffn_norm = _addr(pre_ffn_norm)
    L.post_ffn_norm = _addr(post_ffn_norm)
    L.norm_offset = norm_offset
    L.has_post_norms = int(bool(has_post_norms))
    L.has_v_norm = int(bool(has_v_norm))
    L.layer_scalar = layer_scalar
    L.eps = eps
    L.norm_type = NORM_RMS
    L.ffn_type = FFN_GATED
    L.activation = activation
    L.attn_scale = attn_scale if attn_scale is not None else float(1.0 / np.sqrt(head_dim))
    L.head_dim, L.num_q_heads, L.num_kv_heads = head_dim, num_q_heads, num_kv_heads
    L.rope_base = rope_base
    L.rotary_dim = rotary_dim
    L.sliding_window = sliding_window
    return L

QUANT_BYTES = {Q4_0: (32, 18), Q4_K: (256, 148), Q6_K: (256, 210), Q8_0: (32, 32)}

_lib = None


def _share_torch_hip_runtime():
    """PyTorch-ROCm ships its own libamdhip64 (soname libamdhip64.so.7).  If it is
    loaded first, liblarql_hip binds to that copy; if liblarql_hip loaded the system
    copy first, torch would load a second HIP/HSA runtime that cannot open the device.
    Importing torch first keeps one runtime per process."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load_library():
    """Load liblarql_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"liblarql_hip.so not built at {LIB_PATH}; run `make -C encoding-experiment_amd`")
        _share_torch_hip_runtime()
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


load_library()


def _arr(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data_as(_P)


def _dptr(t):
    """Device pointer of a tensor-like object (torch.Tensor or an int address)."""
    if t is None:
        return None
    if isinstance(t, int):
        return _P(t)
    return _P(t.data_ptr())


def _stream_ptr(stream):
    """hipStream_t of a torch stream (or a raw handle).  None selects the context's
    own stream.  The legacy default stream (handle 0) is rejected: NULL means
    "context stream" in the C ABI, so work would silently leave the caller's order."""
    if stream is None:
        return None
    h = stream if isinstance(stream, int) else stream.cuda_stream
    if h == 0:
        raise ValueError("pass a non-default stream (e.g. torch.cuda.Stream()); handle 0 means the context stream")
    return _P(h)


class HipBackend:
    """ComputeBackend over liblarql_hip (one context = one device + stream)."""

    def __init__(self, device: int = 0, strict: bool = False):
        self._lib = load_library()
        self.strict = strict
        ctx = _P()
        rc = self._lib.larql_hip_ctx_create(device, ctypes.byref(ctx))
        if rc != OK:
            raise LarqlHipError(rc, f"larql_hip_ctx_create(device={device}) failed")
        self._ctx = ctx
        self.device = device

    # ── lifecycle ──────────────────────────────────────────────────────
    def close(self):
        if getattr(self, "_ctx", None):
            self._lib.larql_hip_ctx_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def last_error(self) -> str:
        return self._lib.larql_hip_last_error(self._ctx).decode()

    def _ok(self, rc: int) -> bool:
        if rc == OK:
            return True
        if self.strict:
            raise LarqlHipError(rc, self.last_error())
        return False

    def _check(self, rc: int):
        if rc != OK:
            raise LarqlHipError(rc, self.last_error())

    # ── metadata (backend.rs:155-163) ──────────────────────────────────
    def name(self) -> str:
        return self._lib.larql_hip_name().decode()

    def device_info(self) -> str:
        buf = ctypes.create_string_buffer(256)
        self._check(self._lib.larql_hip_device_info(self._ctx, buf, 256))
        return buf.value.decode()

    def has_q4(self) -> bool:
        return bool(self._lib.larql_hip_has_q4(self._ctx))

    def has_kv_cache(self) -> bool:
        return bool(self._lib.larql_hip_has_kv_cache(self._ctx))

    def synchronize(self):
        self._check(self._lib.larql_hip_synchronize(self._ctx))

    # ── weight registry ────────────────────────────────────────────────
    def register_weight(self, fmt: int, data, rows: int, cols: int, q8_scales=None) -> int:
        """Upload + repack reference-layout bytes (host numpy) -> handle."""
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        sc_ptr = None
        if q8_scales is not None:
            sc, sc_ptr = _arr(q8_scales, np.float32)
        h = _U64()
        self._check(self._lib.larql_hip_register_weight(
            self._ctx, fmt, raw.ctypes.data_as(_P), raw.size, sc_ptr, rows, cols, ctypes.byref(h)))
        return h.value

    def register_weight_device(self, fmt: int, dev_data, nbytes: int, rows: int, cols: int,
                               dev_q8_scales=None) -> int:
        h = _U64()
        self._check(self._lib.larql_hip_register_weight_device(
            self._ctx, fmt, _dptr(dev_data), nbytes, _dptr(dev_q8_scales), rows, cols, ctypes.byref(h)))
        return h.value

    def release_weight(self, handle: int):
        self._check(self._lib.larql_hip_release_weight(self._ctx, handle))

    def forget_host(self, data: np.ndarray):
        self._check(self._lib.larql_hip_forget_host(self._ctx, data.ctypes.data_as(_P)))

    def weight_device_bytes(self, handle: int) -> int:
        n = _SZ()
        self._check(self._lib.larql_hip_weight_device_bytes(self._ctx, handle, ctypes.byref(n)))
        return n.value

    # ── trait methods (backend.rs) ─────────────────────────────────────
    def q4_matvec(self, q4_data, q8_x, q8_scales, num_rows: int, hidden: int):
        """backend.rs:49-53 — scores[N] = Q4_0[N,K] @ Q8_x[K]."""
        q4, q4p = _arr(q4_data, np.uint8)
        qx, qxp = _arr(q8_x, np.int8)
        qs, qsp = _arr(q8_scales, np.float32)
        out = np.empty(num_rows, dtype=np.float32)
        rc = self._lib.larql_hip_q4_matvec(self._ctx, q4p, q4.size, qxp, qsp, out.ctypes.data_as(_P), num_rows, hidden)
        return out if self._ok(rc) else None

    def q4_vecmat(self, activation, q4_data, intermediate: int, hidden: int):
        """backend.rs:56-60 — out[hidden] = activation[intermediate] @ Q4_0[intermediate, hidden]."""
        a, ap = _arr(activation, np.float32)
        q4, q4p = _arr(q4_data, np.uint8)
        out = np.empty(hidden, dtype=np.float32)
        rc = self._lib.larql_hip_q4_vecmat(self._ctx, ap, q4p, q4.size, out.ctypes.data_as(_P), intermediate, hidden)
        return out if self._ok(rc) else None

    def q4_matvec_pair_batch(self, gate_q4, up_q4, x_matrix, seq_len: int, num_rows: int, hidden: int):
        """backend.rs:64-69 — per position: quantize_to_q8, then gate and up Q4_0 matvecs.
        Returns (gate [seq_len, num_rows], up [seq_len, num_rows])."""
        g, gp = _arr(gate_q4, np.uint8)
        u, up = _arr(up_q4, np.uint8)
        x, xp = _arr(x_matrix, np.float32)
        go = np.empty((seq_len, num_rows), dtype=np.float32)
        uo = np.empty((seq_len, num_rows), dtype=np.float32)
        rc = self._lib.larql_hip_q4_matvec_pair_batch(self._ctx, gp, g.size, up, u.size, xp, seq_len,
                                                      go.ctypes.data_as(_P), uo.ctypes.data_as(_P), num_rows, hidden)
        return (go, uo) if self._ok(rc) else None

    def q4k_matvec(self, q4k_data, x, num_rows: int, hidden: int):
        """backend.rs:126-130 — scores[N] = Q4_K[N,K] @ f32_x[K]."""
        q, qp = _arr(q4k_data, np.uint8)
        xv, xp = _arr(x, np.float32)
        out = np.empty(num_rows, dtype=np.float32)
        rc = self._lib.larql_hip_q4k_matvec(self._ctx, qp, q.size, xp, out.ctypes.data_as(_P), num_rows, hidden)
        return out if self._ok(rc) else None

    def q4k_matmul(self, q4k_data, x, num_rows: int, hidden: int):
        """Prefill projection (Metal prefill loop, LC/src/metal/prefill.rs:21-110):
        x f32 [m, hidden] -> out f32 [m, num_rows] = x . deq(Q4_K)^T (MFMA GEMM)."""
        q, qp = _arr(q4k_data, np.uint8)
        xv = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, hidden)
        m = xv.shape[0]
        out = np.empty((m, num_rows), dtype=np.float32)
        rc = self._lib.larql_hip_q4k_matmul(self._ctx, qp, q.size, xv.ctypes.data_as(_P), m, out.ctypes.data_as(_P),
                                            num_rows, hidden)
        return out if self._ok(rc) else None

    def _matmul(self, a, b, transpose_b: bool):
        av = np.ascontiguousarray(a, dtype=np.float32)
        bv = np.ascontiguousarray(b, dtype=np.float32)
        if av.ndim != 2 or bv.ndim != 2:
            raise ValueError("matmul takes 2-D arrays")
        m, k = av.shape
        n = bv.shape[0] if transpose_b else bv.shape[1]
        if (bv.shape[1] if transpose_b else bv.shape[0]) != k:
            raise ValueError(f"matmul: inner dimensions differ ({av.shape} x {bv.shape}, transpose_b={transpose_b})")
        out = np.empty((m, n), dtype=np.float32)
        rc = self._lib.larql_hip_matmul(self._ctx, av.ctypes.data_as(_P), m, k, bv.ctypes.data_as(_P), n,
                                        int(bool(transpose_b)), out.ctypes.data_as(_P))
        return out if self._ok(rc) else None

    def matmul(self, a, b):
        """backend.rs:27-28 — C = A [m, k] x B [k, n] (f32)."""
        return self._matmul(a, b, False)

    def matmul_transb(self, a, b):
        """backend.rs:30-31 — C = A [m, k] x B [n, k]^T (f32)."""
        return self._matmul(a, b, True)

    def matmul_batch(self, ops):
        """backend.rs:33-43 — ops: (a, b, transpose_b) triples, run in order."""
        return [self._matmul(a, b, tb) for a, b, tb in ops]

    def matmul_dev(self, a, b, out, m: int, k: int, n: int, transpose_b: bool = False, stream=None):
        """Device form of matmul / matmul_transb: a [m, k], b [k, n] or [n, k], out [m, n]."""
        self._check(self._lib.larql_hip_matmul_dev(self._ctx, _dptr(a), m, k, _dptr(b), n, int(bool(transpose_b)),
                                                   _dptr(out), _stream_ptr(stream)))

    def q6k_matvec(self, q6k_data, x, num_rows: int, hidden: int):
        """backend.rs:133-137 — scores[N] = Q6_K[N,K] @ f32_x[K]."""
        q, qp = _arr(q6k_data, np.uint8)
        xv, xp = _arr(x, np.float32)
        out = np.empty(num_rows, dtype=np.float32)
        rc = self._lib.larql_hip_q6k_matvec(self._ctx, qp, q.size, xp, out.ctypes.data_as(_P), num_rows, hidden)
        return out if self._ok(rc) else None

    # ── reference free functions (extensions) ──────────────────────────
    def quantize_to_q8(self, x):
        """q4_common.rs:28-44 on the device (bit-exact)."""
        xv, xp = _arr(x, np.float32)
        q8 = np.empty(xv.size, dtype=np.int8)
        sc = np.empty(xv.size // 32, dtype=np.float32)
        rc = self._lib.larql_hip_quantize_to_q8(self._ctx, xp, xv.size, q8.ctypes.data_as(_P), sc.ctypes.data_as(_P))
        return (q8, sc) if self._ok(rc) else None

    def q8_matvec(self, w_q8, w_scales, x_q8, x_scales, num_rows: int, hidden: int):
        """q8_matvec.rs:36-62, batched: x_q8 is [m, hidden] (or [hidden]); returns [m, num_rows]."""
        wq, wqp = _arr(w_q8, np.int8)
        ws, wsp = _arr(w_scales, np.float32)
        xq, xqp = _arr(x_q8, np.int8)
        xs, xsp = _arr(x_scales, np.float32)
        m = xq.size // hidden
        out = np.empty((m, num_rows), dtype=np.float32)
        rc = self._lib.larql_hip_q8_matvec(self._ctx, wqp, wq.size, wsp, xqp, xsp, m, out.ctypes.data_as(_P), num_rows, hidden)
        return out if self._ok(rc) else None

    def quantize_weights(self, fmt: int, x):
        """Reference weight quantizers on the device: returns the reference layout bytes
        (and, for Q8_0, (int8 values, f32 scales))."""
        xv, xp = _arr(x, np.float32)
        per, nbytes = QUANT_BYTES[fmt]
        out = np.empty(xv.size // per * nbytes, dtype=np.uint8)
        sc = np.empty(xv.size // 32, dtype=np.float32) if fmt == Q8_0 else None
        rc = self._lib.larql_hip_quantize_weights(self._ctx, fmt, xp, xv.size, out.ctypes.data_as(_P),
                                                  sc.ctypes.data_as(_P) if sc is not None else None)
        if not self._ok(rc):
            return None
        return (out.view(np.int8), sc) if fmt == Q8_0 else out

    # ── decode step (backend.rs:99-123) ───────────────────────────────
    def has_kv(self) -> bool:
        return self.has_kv_cache()

    def decode_token(self, layers, x, hidden: int, inter: int, q_dim: int, kv_dim: int, num_q_heads: int,
                     num_kv_heads: int, head_dim: int, rope_base: float):
        """backend.rs:115-123: one token through all layers with the KV cache; returns the
        final hidden state (before the final norm) or None."""
        arr = (PipelineLayer * len(layers))(*layers)
        xv, xp = _arr(x, np.float32)
        out = np.empty(hidden, dtype=np.float32)
        rc = self._lib.larql_hip_decode_token(self._ctx, ctypes.cast(arr, _P), len(layers), xp, hidden, inter, q_dim,
                                              kv_dim, num_q_heads, num_kv_heads, head_dim, rope_base,
                                              out.ctypes.data_as(_P))
        return out if self._ok(rc) else None

    def prefill_q4(self, layers, x, hidden: int, inter: int, q_dim: int, kv_dim: int, seq_len: int,
                   num_q_heads: int, num_kv_heads: int, head_dim: int, rope_base: float, use_qk_norm: bool = False,
                   softcap: float = 0.0):
        """backend.rs:139-152: a prompt [seq_len, hidden] through all layers at positions
        0..seq_len-1, filling the KV cache; returns the final hidden states [seq_len, hidden]
        or None."""
        arr = (PipelineLayer * len(layers))(*layers)
        xv, xp = _arr(x, np.float32)
        out = np.empty(seq_len * hidden, dtype=np.float32)
        rc = self._lib.larql_hip_prefill_q4(self._ctx, ctypes.cast(arr, _P), len(layers), xp, hidden, inter, q_dim,
                                            kv_dim, seq_len, num_q_heads, num_kv_heads, head_dim, rope_base,
                                            1 if use_qk_norm else 0, softcap, out.ctypes.data_as(_P))
        return out.reshape(seq_len, hidden) if self._ok(rc) else None

    def full_pipeline_q4(self, layers, x, hidden: int, inter: int, q_dim: int, kv_dim: int, seq_len: int,
                         num_q_heads: int, num_kv_heads: int, head_dim: int, rope_base: float,
                         use_qk_norm: bool = False, softcap: float = 0.0):
        """backend.rs:71-84: positions 0..seq_len-1 through all layers with causal attention
        among them only (the decode cache untouched); returns [seq_len, hidden] or None."""
        arr = (PipelineLayer * len(layers))(*layers)
        xv, xp = _arr(x, np.float32)
        out = np.empty(seq_len * hidden, dtype=np.float32)
        rc = self._lib.larql_hip_full_pipeline_q4(self._ctx, ctypes.cast(arr, _P), len(layers), xp, hidden, inter,
                                                  q_dim, kv_dim, seq_len, num_q_heads, num_kv_heads, head_dim,
                                                  rope_base, 1 if use_qk_norm else 0, softcap,
                                                  out.ctypes.data_as(_P))
        return out.reshape(seq_len, hidden) if self._ok(rc) else None

    def multi_layer_q4_ffn(self, layers_q4, x, inter: int, hidden: int):
        """backend.rs:86-96: layers_q4 = [(gate, up, down_t) Q4_0 byte arrays]; returns the
        chained FFN output [hidden] or None."""
        keep = [tuple(np.ascontiguousarray(a, dtype=np.uint8) for a in t) for t in layers_q4]
        arr = (Q4FfnLayer * len(keep))(*[Q4FfnLayer(g.ctypes.data, g.nbytes, u.ctypes.data, u.nbytes, d.ctypes.data,
                                                    d.nbytes) for g, u, d in keep])
        xv, xp = _arr(x, np.float32)
        out = np.empty(hidden, dtype=np.float32)
        rc = self._lib.larql_hip_multi_layer_q4_ffn(self._ctx, ctypes.cast(arr, _P), len(keep), xp, inter, hidden,
                                                    out.ctypes.data_as(_P))
        return out if self._ok(rc) else None

    def populate_kv_layer(self, layer: int, k_data, v_data, seq_len: int, num_kv_heads: int, head_dim: int):
        """backend.rs:103-107 (K/V f32 [seq_len, num_kv*head_dim], stored as fp16)."""
        k, kp = _arr(k_data, np.float32)
        v, vp = _arr(v_data, np.float32)
        self._check(self._lib.larql_hip_populate_kv_layer(self._ctx, layer, kp, vp, seq_len, num_kv_heads, head_dim))

    def populate_kv_layer_f16_dev(self, layer: int, k_dev, v_dev, seq_len: int, num_kv_heads: int, head_dim: int):
        self._check(self._lib.larql_hip_populate_kv_layer_f16_dev(self._ctx, layer, _dptr(k_dev), _dptr(v_dev),
                                                                  seq_len, num_kv_heads, head_dim))

    def reset_kv_cache(self):
        """backend.rs:110."""
        self._check(self._lib.larql_hip_reset_kv_cache(self._ctx))

    def kv_cache_len(self) -> int:
        n = _SZ()
        self._check(self._lib.larql_hip_kv_cache_len(self._ctx, ctypes.byref(n)))
        return n.value

    def kv_truncate(self, n: int):
        self._check(self._lib.larql_hip_kv_truncate(self._ctx, n))

    def model(self, layers, hidden: int, inter: int, weights_on_device: bool = False) -> DeviceModel:
        """weights_on_device: the layers' weight and norm pointers are device addresses
        (else host memory, uploaded once)."""
        return DeviceModel(self, layers, hidden, inter, weights_on_device)

    # ── device-resident fast path ──────────────────────────────────────
    def matvec_dev(self, handle: int, x, out, m: int = 1, x_scales=None, stream=None):
        self._check(self._lib.larql_hip_matvec_dev(self._ctx, handle, _dptr(x), _dptr(x_scales), _dptr(out), m,
                                                   _stream_ptr(stream)))

    def quantize_weights_dev(self, fmt: int, x, n: int, out, q8_scales=None, stream=None):
        self._check(self._lib.larql_hip_quantize_weights_dev(self._ctx, fmt, _dptr(x), n, _dptr(out),
                                                             _dptr(q8_scales), _stream_ptr(stream)))

    def quantize_to_q8_dev(self, x, n: int, m: int, q8, scales, stream=None):
        self._check(self._lib.larql_hip_quantize_to_q8_dev(self._ctx, _dptr(x), n, m, _dptr(q8), _dptr(scales),
                                                           _stream_ptr(stream)))

    # ── vindex gate-KNN (LV/src/index/gate.rs) ─────────────────────────
    def gate_knn(self, gate, features: int, hidden: int, queries, top_k: int, fmt: int = F32):
        """gate_knn (gate.rs:108-134) per query, or gate_knn_q4 (:711-731) with fmt=Q4_0.
        queries: f32 [nq, hidden] (or [hidden]).  Returns (idx u32 [nq, k], scores f32
        [nq, k]) by |score| descending, ties in index order; None if unsupported."""
        g, gp = _arr(gate, np.float32 if fmt == F32 else np.uint8)
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, hidden)
        nq = q.shape[0]
        idx = np.empty((nq, top_k), dtype=np.uint32)
        val = np.empty((nq, top_k), dtype=np.float32)
        rc = self._lib.larql_hip_gate_knn(self._ctx, fmt, gp, g.nbytes, features, hidden, q.ctypes.data_as(_P), nq,
                                          top_k, idx.ctypes.data_as(_P), val.ctypes.data_as(_P))
        return (idx, val) if self._ok(rc) else None

    def lm_head_knn(self, lm_head_q4, vocab: int, hidden: int, query, top_k: int):
        """lm_head_knn_backend's Q4 path (LV/src/index/walk.rs:549-583): top_k (token, score)
        by signed score descending, ties in index order; None if unsupported."""
        w, wp = _arr(lm_head_q4, np.uint8)
        q, qp = _arr(query, np.float32)
        idx = np.empty(top_k, dtype=np.uint32)
        val = np.empty(top_k, dtype=np.float32)
        rc = self._lib.larql_hip_lm_head_knn(self._ctx, wp, w.nbytes, qp, vocab, hidden, top_k,
                                             idx.ctypes.data_as(_P), val.ctypes.data_as(_P))
        return (idx, val) if self._ok(rc) else None

    def lm_head_knn_dev(self, handle: int, queries, nq: int, top_k: int, idx, scores, stream=None):
        self._check(self._lib.larql_hip_lm_head_knn_dev(self._ctx, handle, _dptr(queries), nq, top_k, _dptr(idx),
                                                        _dptr(scores), _stream_ptr(stream)))

    def lm_head_knn_dev_noalloc(self, handle: int, queries, nq: int, top_k: int, idx, scores, stream=None):
        """lm_head_knn_dev with its work buffers in the library's fixed device array (no
        allocation); nq * (vocab * 4 + hidden * 9 / 8) must fit NOALLOC_SCRATCH_BYTES."""
        self._check(self._lib.larql_hip_lm_head_knn_dev_noalloc(self._ctx, handle, _dptr(queries), nq, top_k,
                                                                _dptr(idx), _dptr(scores), _stream_ptr(stream)))

    @staticmethod
    def _handle_array(handles):
        arr = (_U64 * len(handles))(*handles)
        return arr, ctypes.cast(arr, _P)

    def vecmat_dev(self, handle: int, activation, out, stream=None):
        self._check(self._lib.larql_hip_vecmat_dev(self._ctx, handle, _dptr(activation), _dptr(out),
                                                   _stream_ptr(stream)))

    def read_floor_dev(self, handle: int, out, workgroups: int = 0, threads: int = 0, stream=None):
        """Plain read of a registered weight's device bytes (a measurement of the memory
        floor): in its matvec's launch shape by default (Q4_K-family weights), else
        `workgroups` x `threads` (any format).
        out: device int32/uint32 tensor, one XOR fold per workgroup."""
        self._check(self._lib.larql_hip_read_floor_dev(self._ctx, handle, workgroups, threads, _dptr(out),
                                                       out.numel(), _stream_ptr(stream)))

    def q4k_launch_shape(self, handle: int) -> dict:
        """The launch configuration of a registered Q4_K / Q4_KF weight's matvec: ur, tiles,
        pre, xb, rounds (q4k_mfma_kernel<ur, tiles, norm, header, pre, xb>) and its grid."""
        v = [ctypes.c_int() for _ in range(5)]
        g, t = ctypes.c_uint(), ctypes.c_uint()
        self._check(self._lib.larql_hip_q4k_launch_shape(self._ctx, handle, *[ctypes.byref(x) for x in v],
                                                         ctypes.byref(g), ctypes.byref(t)))
        d = dict(zip(("ur", "tiles", "pre", "xb", "rounds"), (x.value for x in v)))
        d.update(workgroups=g.value, threads=t.value)
        return d

    def pair_batch_dev(self, gate: int, up: int, x, seq_len: int, gate_out, up_out, stream=None):
        self._check(self._lib.larql_hip_pair_batch_dev(self._ctx, gate, up, _dptr(x), seq_len, _dptr(gate_out),
                                                       _dptr(up_out), _stream_ptr(stream)))

    def gate_knn_dev(self, handles, queries, nq: int, top_k: int, idx, scores, stream=None):
        arr, ap = self._handle_array(handles)
        self._check(self._lib.larql_hip_gate_knn_dev(self._ctx, ap, len(handles), _dptr(queries), nq, top_k,
                                                     _dptr(idx), _dptr(scores), _stream_ptr(stream)))

    def gate_scores_dev(self, handles, queries, nq: int, scores, stream=None):
        arr, ap = self._handle_array(handles)
        self._check(self._lib.larql_hip_gate_scores_dev(self._ctx, ap, len(handles), _dptr(queries), nq,
                                                        _dptr(scores), _stream_ptr(stream)))

    def topk_dev(self, scores, rows: int, n: int, k: int, idx, vals, signed: bool = False, stream=None):
        self._check(self._lib.larql_hip_topk_dev(self._ctx, _dptr(scores), rows, n, k, int(signed), _dptr(idx),
                                                 _dptr(vals), _stream_ptr(stream)))


class DeviceModel:
    """Device-resident decoder (larql_hip_model): registered once, decoded per token."""

    def __init__(self, backend: "HipBackend", layers, hidden: int, inter: int, weights_on_device: bool):
        self.be = backend
        arr = (PipelineLayer * len(layers))(*layers)
        h = _P()
        backend._check(backend._lib.larql_hip_model_create(backend._ctx, ctypes.cast(arr, _P), len(layers), hidden,
                                                           inter, int(weights_on_device), ctypes.byref(h)))
        self._h = h
        self.hidden = hidden

    def set_head(self, head, vocab: int, final_norm, eps: float = 1e-6, fmt: int = Q6_K, on_device: bool = True):
        qw = QuantWeight(_addr(head), _nbytes(head), None, fmt)
        self.be._check(self.be._lib.larql_hip_model_set_head(self.be._ctx, self._h, ctypes.byref(qw), vocab,
                                                             _P(_addr(final_norm)), eps, int(on_device)))

    def decode_dev(self, x, hidden_out=None, logits=None, stream=None):
        self.be._check(self.be._lib.larql_hip_model_decode_dev(self.be._ctx, self._h, _dptr(x), _dptr(hidden_out),
                                                               _dptr(logits), _stream_ptr(stream)))

    def prefill_dev(self, x, seq_len: int, out, stream=None):
        """A prompt [seq_len][hidden] from position 0 (device tensors); resets the KV cache
        and leaves it at seq_len; out gets every position's hidden state."""
        self.be._check(self.be._lib.larql_hip_model_prefill_dev(self.be._ctx, self._h, _dptr(x), seq_len,
                                                                _dptr(out), _stream_ptr(stream)))

    def close(self):
        if self._h:
            self.be._lib.larql_hip_model_destroy(self.be._ctx, self._h)
            self._h = None


def default_backend(device: int = 0, strict: bool = False) -> HipBackend:
    """lib.rs:68-78 analogue: the HIP backend on `device` (raises if no device)."""
    return HipBackend(device, strict=strict)
