"""GPU parity of the trait's f32 products ComputeBackend::matmul / matmul_transb /
matmul_batch (LC/src/backend.rs:27-43; Metal LC/src/metal/f32_ops.rs:93-140).

Bar: BIT-EXACT with the oracle's canonical order (one f32 fma chain per element over k
from +0, lo_gate_scores_f32, pinned in test_oracle.py); the reference's CPU sgemm
(matrixmultiply) sums in its own blocked order, so against float64 the bar is the f32
rounding of a K-term sum.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _ref_transb(a, b):
    """C[i] = canonical chains of row i of a against every row of b."""
    n, k = b.shape
    return np.stack([oracle.gate_scores_f32(b, a[i], n, k) for i in range(a.shape[0])])


def _rand(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


# (m, k, n): m = 1 (the gemv callers), k not a multiple of 16 or of 4, m < n (the
# product stored transposed) and m > n, tiles with ragged edges on both sides
SHAPES = [(1, 2560, 300), (1, 7, 5), (3, 17, 1), (5, 33, 70), (64, 16, 64), (300, 100, 7), (257, 129, 65),
          (31, 1000, 513), (700, 48, 2)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_transb_bit_exact(hip, m, k, n):
    rng = np.random.default_rng(m * 1000 + k + n)
    a, b = _rand(rng, m, k), _rand(rng, n, k)
    got = hip.matmul_transb(a, b)
    ref = _ref_transb(a, b)
    assert got.shape == (m, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (m, k, n)
    exact = a.astype(np.float64) @ b.astype(np.float64).T
    assert np.max(np.abs(got - exact)) <= 1e-5 * max(1.0, np.max(np.abs(exact))) * np.sqrt(k)


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_matmul_bit_exact(hip, m, k, n):
    rng = np.random.default_rng(m * 2000 + k + n)
    a, b = _rand(rng, m, k), _rand(rng, k, n)
    got = hip.matmul(a, b)
    ref = _ref_transb(a, np.ascontiguousarray(b.T))
    assert got.shape == (m, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (m, k, n)


def test_matmul_edge_cases(hip):
    """k = 0 gives zeros; special values propagate as the chain propagates them; a
    batch equals its calls in order; mismatched inner dimensions raise."""
    rng = np.random.default_rng(7)
    z = hip.matmul_transb(np.zeros((3, 0), np.float32), np.zeros((4, 0), np.float32))
    assert z.shape == (3, 4) and not np.any(z) and not np.any(np.signbit(z))
    a, b = _rand(rng, 5, 40), _rand(rng, 9, 40)
    a[1, 3], a[2, 5], b[4, 0] = np.inf, np.nan, -np.inf
    got, ref = hip.matmul_transb(a, b), _ref_transb(a, b)
    nan = np.isnan(ref)
    assert nan.any() and np.array_equal(np.isnan(got), nan)          # NaN payloads may differ
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    ops = [(a, b, True), (_rand(rng, 2, 9), _rand(rng, 9, 6), False)]
    batch = hip.matmul_batch(ops)
    assert np.array_equal(batch[0], hip.matmul_transb(a, b), equal_nan=True)
    assert np.array_equal(batch[1], hip.matmul(ops[1][0], ops[1][1]))
    with pytest.raises(ValueError):
        hip.matmul(a, b)


def test_matmul_gate_shape_and_device_entry(hip):
    """The vindex score shape (LV/src/index/gate.rs:14-29): 256 queries against a gate
    [10240 x 2560], through the device entry on torch buffers.  Rows sampled across the
    output against the oracle bit for bit; the swapped product (gate against queries) is
    the exact transpose; the host entry gives the same bits."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    q, g = _rand(rng, 256, 2560), (0.02 * _rand(rng, 10240, 2560)).astype(np.float32)
    dev = torch.device("cuda:0")
    tq, tg = torch.from_numpy(q).to(dev), torch.from_numpy(g).to(dev)
    out = torch.empty(256 * 10240, device=dev)
    outt = torch.empty(10240 * 256, device=dev)
    hip.matmul_dev(tq, tg, out, 256, 2560, 10240, transpose_b=True)
    hip.matmul_dev(tg, tq, outt, 10240, 2560, 256, transpose_b=True)
    torch.cuda.synchronize()
    c = out.cpu().numpy().reshape(256, 10240)
    ct = outt.cpu().numpy().reshape(10240, 256)
    assert np.array_equal(c, ct.T)
    rows = [0, 1, 97, 128, 255]
    ref = _ref_transb(q[rows], g)
    assert np.array_equal(c[rows].view(np.uint32), ref.view(np.uint32))
    host = hip.matmul_transb(q[:8], g)
    assert np.array_equal(host, c[:8])
