"""GPU parity of the quantized prefill projection (Q4_K GEMM on the matrix cores)
against the CPU oracle: prefill = the Q4_K matvec applied per token
(LC/src/cpu/ops/q4k_matvec.rs:31-90, the Metal prefill loop LC/src/metal/prefill.rs:21-110).

Bar: max|gpu - cpu| / max|cpu| <= 1e-3 over the checked token rows (fp16 operands with
f32 accumulation; measured ~1e-4)."""
import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def check_rows(q4k, x, got, rows, cols, token_rows):
    errs = []
    for t in token_rows:
        ref = oracle.q4k_matvec(q4k, x[t], rows, cols)
        errs.append(rel_err(got[t], ref))
    e = max(errs)
    print(f"  rel_err max over {len(token_rows)} tokens = {e:.3e}", flush=True)
    assert e <= REL_TOL, e


@pytest.mark.parametrize("rows,cols,m", [(300, 512, 37), (1000, 2560, 130), (64, 256, 2), (129, 768, 129),
                                         (300, 512, 700), (72, 256, 1030), (1000, 2560, 513)])
def test_q4k_matmul_small_shapes(hip, rows, cols, m):
    print(f"[prefill] rows={rows} cols={cols} m={m}", flush=True)
    w = oracle.gauss(61, rows * cols, 0.0, 0.02)
    q4k = oracle.quantize_q4_k(w)
    x = oracle.gauss(62, m * cols).reshape(m, cols)
    got = hip.q4k_matmul(q4k, x, rows, cols)
    check_rows(q4k, x, got, rows, cols, range(m))


def test_q4k_matmul_fuzzed_bytes(hip):
    """Random 148-byte blocks (all nibbles and scale codes), bounded f16 d / dmin."""
    rows, cols, m = 200, 1024, 70
    rng = np.random.default_rng(63)
    q4k = rng.integers(0, 256, size=rows * cols // 256 * 148, dtype=np.uint8)
    blocks = q4k.reshape(-1, 148)
    dd = rng.uniform(-0.01, 0.01, size=(blocks.shape[0], 2)).astype(np.float16)
    blocks[:, 0:4] = dd.view(np.uint8).reshape(-1, 4)
    x = oracle.gauss(64, m * cols).reshape(m, cols)
    got = hip.q4k_matmul(q4k, x, rows, cols)
    check_rows(q4k, x, got, rows, cols, range(m))


def test_q4k_prefill_512_tokens_full_shape(hip):
    """The prefill workload: Q4_K W [10240 x 2560] from N(0, 0.02), X [512 x 2560] N(0,1),
    through the device path (matvec_dev with m = 512); every token row is checked against
    the oracle (its matvecs spread over the host's threads)."""
    torch = pytest.importorskip("torch")
    rows, cols, m = 10240, 2560, 512
    w = oracle.gauss(71, rows * cols, 0.0, 0.02)
    q4k = oracle.quantize_q4_k(w)
    x = oracle.gauss(72, m * cols).reshape(m, cols)
    h = hip.register_weight(larql_hip.Q4_K, q4k, rows, cols)
    try:
        dx = torch.from_numpy(x).cuda()
        dy = torch.empty(m * rows, device="cuda", dtype=torch.float32)
        hip.matvec_dev(h, dx, dy, m=m)
        hip.synchronize()
        got = dy.cpu().numpy().reshape(m, rows)
        assert np.all(np.isfinite(got))
        import os
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max(1, min(16, len(os.sched_getaffinity(0))))) as pool:
            errs = list(pool.map(lambda t: rel_err(got[t], oracle.q4k_matvec(q4k, x[t], rows, cols)), range(m)))
        e = max(errs)
        print(f"  rel_err max over all {m} tokens = {e:.3e}", flush=True)
        assert e <= REL_TOL, e
    finally:
        hip.release_weight(h)


def test_q4k_matmul_m1_equals_matvec(hip):
    rows, cols = 512, 1024
    q4k = oracle.quantize_q4_k(oracle.gauss(81, rows * cols, 0.0, 0.02))
    x = oracle.gauss(82, cols)
    a = hip.q4k_matmul(q4k, x[None, :], rows, cols)[0]
    b = hip.q4k_matvec(q4k, x, rows, cols)
    np.testing.assert_array_equal(a, b)


# (4096, 14336, 64): the Llama-3-8B down projection; (300, 512, 37): a ragged tile; (70, 1024,
# 9, scaled): token rows scaled by 1e6 .. 1e-30, far outside fp16 (the GEMM's operand pairs
# are fp16: each row must be brought into range by its own power of two), and a zero row
@pytest.mark.parametrize("rows,cols,m,scaled", [(4096, 14336, 64, False), (300, 512, 37, False), (70, 1024, 9, True)])
def test_q6k_gemm_rows_match_matvec_oracle(hip, rows, cols, m, scaled):
    """The Q6_K f32-accuracy GEMM of the prompt pass (matvec_dev with m > 1 on a Q6_K handle)
    at the Llama-3-8B down-projection shape: every token row against the oracle's Q6_K
    matvec (LC/src/cpu/ops/q6k_matvec.rs), within 1e-3 (fp16 operand pairs: measured ~1e-6)."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    torch = pytest.importorskip("torch")
    print(f"[q6k gemm] rows={rows} cols={cols} m={m} scaled={scaled}", flush=True)
    q6k = oracle.quantize_q6_k(oracle.gauss(91, rows * cols, 0.0, 0.02))
    x = oracle.gauss(92, m * cols).reshape(m, cols)
    if scaled:
        f = np.array([1e6, 1e3, 3e4, 1.0, 1e-3, 1e-8, 1e-20, 1e-30, 0.0], np.float32)
        x = (x * f[:, None]).astype(np.float32)
    h = hip.register_weight(larql_hip.Q6_K, q6k, rows, cols)
    try:
        dx = torch.from_numpy(x).cuda()
        dy = torch.empty(m * rows, device="cuda", dtype=torch.float32)
        hip.matvec_dev(h, dx, dy, m=m)
        hip.synchronize()
        got = dy.cpu().numpy().reshape(m, rows)
        with ThreadPoolExecutor(max(1, min(16, len(os.sched_getaffinity(0))))) as pool:
            refs = list(pool.map(lambda t: oracle.q6k_matvec(q6k, x[t], rows, cols), range(m)))
        errs = [rel_err(got[t], refs[t]) if np.any(refs[t]) else float(np.max(np.abs(got[t]))) for t in range(m)]
        e = max(errs)
        print(f"  rel_err max over all {m} tokens = {e:.3e}", flush=True)
        assert e <= REL_TOL, e
    finally:
        hip.release_weight(h)
        hip.forget_host(q6k)
