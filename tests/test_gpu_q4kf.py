"""GPU parity of the Q4_KF format (QuantFormat::Q4_KF, larql-compute/src/pipeline.rs:15) in
its two byte layouts, against the CPU oracle:

  * 144-byte GGUF block as the reference's GPU decode reads it (llama.cpp block_q4_K:
    6-bit scales and mins packed in 12 bytes, chunk c of 32 bytes holding sub-block 2c in
    the low and 2c + 1 in the high nibbles; LC/src/metal/shaders/q4kf_qkv_proj.rs:87-119);
  * 160-byte block with pre-baked half scales (q4k_to_q4kf, LC/src/cpu/ops/q4_common.rs:370-413).

Bar: max|gpu - cpu| / max|cpu| <= 1e-3 (floating-point outputs).  Test data: Q4_K blocks
converted losslessly into the GGUF layout with the 6-bit min fields' top bits set at random
(so mins above 15 occur), fuzzed bytes, and the reference's q4k_to_q4kf.
"""
import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def gguf_weights(rows, cols, seed, std=0.02):
    """llama.cpp-layout GGUF blocks from quantized Q4_K, with random bits 4..5 of every 6-bit min."""
    q = oracle.quantize_q4_k(oracle.gauss(seed, rows * cols, 0.0, std))
    g = oracle.q4k_to_gguf_llamacpp(q).reshape(-1, 144)
    rng = np.random.default_rng(seed)
    n = g.shape[0]
    # packed byte k sits at block offset 4 + k: bytes 4..7 = m_j | (m_{j+4} >> 4) << 6 (j < 4)
    g[:, 8:12] |= (rng.integers(0, 4, (n, 4)) << 4).astype(np.uint8)   # bits 4..5 of m_0..m_3
    g[:, 8:12] |= (rng.integers(0, 4, (n, 4)) << 6).astype(np.uint8)   # bits 4..5 of m_4..m_7
    return g.reshape(-1)


def fuzz_gguf(rows, cols, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, rows * cols // 256 * 144, dtype=np.uint8).reshape(-1, 144)
    b[:, 0:2] = np.frombuffer(rng.uniform(1e-4, 0.05, b.shape[0]).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
    b[:, 2:4] = np.frombuffer(rng.uniform(0, 0.02, b.shape[0]).astype(np.float16).tobytes(), np.uint8).reshape(-1, 2)
    return b.reshape(-1)


def kf160_weights(rows, cols, seed, std=0.02):
    return oracle.q4k_to_q4kf(oracle.quantize_q4_k(oracle.gauss(seed, rows * cols, 0.0, std)))


def fuzz_kf160(rows, cols, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, rows * cols // 256 * 160, dtype=np.uint8).reshape(-1, 160)
    b[:, 0:32] = np.frombuffer(rng.uniform(-0.2, 0.2, b.shape[0] * 16).astype(np.float16).tobytes(),
                               np.uint8).reshape(-1, 32)
    return b.reshape(-1)


def _dev_matvec(hip, torch, raw, rows, cols, x):
    h = hip.register_weight(larql_hip.Q4_KF, raw, rows, cols)
    try:
        xd = torch.from_numpy(x).cuda()
        out = torch.empty(rows, device="cuda", dtype=torch.float32)
        hip.matvec_dev(h, xd, out)
        hip.synchronize()
        return out.cpu().numpy()
    finally:
        hip.release_weight(h)


@pytest.mark.parametrize("layout", ["gguf", "gguf_fuzz", "kf160", "kf160_fuzz"])
@pytest.mark.parametrize("rows,cols", [(5, 256), (1000, 2560), (14336, 4096), (4096, 14336)])
def test_q4kf_matvec_matches_oracle(hip, layout, rows, cols):
    torch = pytest.importorskip("torch")
    print(f"[q4kf] {layout} [{rows}x{cols}]", flush=True)
    make = {"gguf": gguf_weights, "gguf_fuzz": fuzz_gguf, "kf160": kf160_weights, "kf160_fuzz": fuzz_kf160}[layout]
    raw = make(rows, cols, 100 + rows)
    x = oracle.gauss(200 + cols, cols)
    got = _dev_matvec(hip, torch, raw, rows, cols, x)
    ref = (oracle.q4kf_gguf_matvec if layout.startswith("gguf") else oracle.q4kf160_matvec)(raw, x, rows, cols)
    e = rel_err(got, ref)
    print(f"  rel_err {e:.2e}", flush=True)
    assert e <= REL_TOL


def test_q4kf_gguf_equals_q4k_on_converted_blocks(hip):
    """The same Q4_K bytes registered as Q4_K and, converted losslessly, as Q4_KF (GGUF) give
    the same matvec to within the kernel's own rounding (one shared kernel, two headers)."""
    torch = pytest.importorskip("torch")
    rows, cols = 2048, 4096
    q = oracle.quantize_q4_k(oracle.gauss(7, rows * cols, 0.0, 0.02))
    x = oracle.gauss(8, cols)
    a = _dev_matvec(hip, torch, oracle.q4k_to_gguf_llamacpp(q), rows, cols, x)
    b = hip.q4k_matvec(q, x, rows, cols)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("nbytes", [10 * 143, 10 * 160 + 16, 10 * 144 + 16, 10 * 160 + 160, 10 * 152])
def test_q4kf_wrong_length_is_an_error(nbytes):
    """A Q4_KF buffer is exactly 144 or exactly 160 bytes per block: shorter, or either form
    with trailing slack (which would otherwise read a 160-byte buffer as GGUF blocks), is an
    error, not a silent misread."""
    be = larql_hip.HipBackend(0, strict=False)
    try:
        raw = np.zeros(nbytes, np.uint8)   # 10 rows of one 256-element block
        with pytest.raises(larql_hip.LarqlHipError, match="Q4_KF buffer"):
            be.register_weight(larql_hip.Q4_KF, raw, 10, 256)
    finally:
        be.close()
