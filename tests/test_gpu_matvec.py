"""GPU parity: HIP matvec kernels (through the C ABI) vs the CPU oracle on the
same seeded inputs.

Bars (parity targets of the quantized compute path):
  * Q4_0 x Q8 and Q8_0 x Q8: BIT-EXACT outputs.  The reference's int32 block
    dot is exact and its block accumulation order (acc += (float)isum_b * cs_b,
    LC/csrc/q4_dot.c:58-89, LC/src/cpu/ops/q8_matvec.rs:44-57) is reproduced.
  * quantize_to_q8 on the device: bit-exact bytes and scales.
  * Q4_K / Q6_K (f32 activations): relative error
        max|gpu - cpu| / max|cpu|  <=  1e-3
    (the reference's own metric, LC/tests/test_q4_x86_correctness.rs:65-71).
"""
import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def weights(fmt, rows, cols, seed, std=0.02):
    w = oracle.gauss(seed, rows * cols, 0.0, std)
    if fmt == "q4k":
        return oracle.quantize_q4_k(w)
    if fmt == "q6k":
        return oracle.quantize_q6_k(w)
    if fmt == "q4_0":
        return oracle.quantize_q4_0(w)
    raise ValueError(fmt)


def fuzz_q4k(rows, cols, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (rows * cols // 256, 148), dtype=np.uint8)
    d = rng.uniform(1e-4, 2e-2, b.shape[0]).astype(np.float16)
    dmin = rng.uniform(0, 2e-2, b.shape[0]).astype(np.float16)
    d[::17] = np.float16(3e-6)                     # f16 subnormal d must decode, not flush
    b[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    b[:, 2:4] = dmin.view(np.uint8).reshape(-1, 2)
    return b.reshape(-1)


def fuzz_q6k(rows, cols, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (rows * cols // 256, 210), dtype=np.uint8)
    d = rng.uniform(1e-4, 2e-3, b.shape[0]).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(-1, 2)
    return b.reshape(-1)


Q4K_SHAPES = [(1, 256), (7, 256), (64, 512), (300, 4096), (1000, 2560), (14336, 4096), (4096, 14336), (100, 20480),
              (28672, 4096), (6144, 4096)]


@pytest.mark.parametrize("rows,cols", Q4K_SHAPES)
def test_q4k_matvec_quantized(hip, rows, cols):
    print(f"[q4k] rows={rows} cols={cols}", flush=True)
    q = weights("q4k", rows, cols, seed=100 + rows)
    x = oracle.gauss(200 + cols, cols)
    ref = oracle.q4k_matvec(q, x, rows, cols)
    got = hip.q4k_matvec(q, x, rows, cols)
    e = rel_err(got, ref)
    print(f"  rel_err={e:.3e}", flush=True)
    assert e <= REL_TOL


@pytest.mark.parametrize("rows,cols", [(5, 256), (129, 1024), (2048, 4096)])
def test_q4k_matvec_fuzzed_bytes(hip, rows, cols):
    print(f"[q4k fuzz] rows={rows} cols={cols}", flush=True)
    q = fuzz_q4k(rows, cols, seed=rows)
    x = oracle.gauss(7 + rows, cols)
    ref = oracle.q4k_matvec(q, x, rows, cols)
    got = hip.q4k_matvec(q, x, rows, cols)
    assert rel_err(got, ref) <= REL_TOL


Q6K_SHAPES = [(1, 256), (9, 512), (300, 4096), (14336, 4096), (4096, 14336), (128256, 4096), (70, 20480), (50, 2560)]


@pytest.mark.parametrize("rows,cols", Q6K_SHAPES)
def test_q6k_matvec_quantized(hip, rows, cols):
    print(f"[q6k] rows={rows} cols={cols}", flush=True)
    q = weights("q6k", rows, cols, seed=300 + rows)
    x = oracle.gauss(400 + cols, cols)
    ref = oracle.q6k_matvec(q, x, rows, cols)
    got = hip.q6k_matvec(q, x, rows, cols)
    e = rel_err(got, ref)
    print(f"  rel_err={e:.3e}", flush=True)
    assert e <= REL_TOL


@pytest.mark.parametrize("rows,cols", [(3, 256), (200, 2048)])
def test_q6k_matvec_fuzzed_bytes(hip, rows, cols):
    q = fuzz_q6k(rows, cols, seed=rows)
    x = oracle.gauss(11 + rows, cols)
    ref = oracle.q6k_matvec(q, x, rows, cols)
    got = hip.q6k_matvec(q, x, rows, cols)
    assert rel_err(got, ref) <= REL_TOL


@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 64), (257, 256), (10240, 2560), (1000, 4096)])
def test_q4_0_matvec_bit_exact(hip, rows, cols):
    print(f"[q4_0] rows={rows} cols={cols}", flush=True)
    q = weights("q4_0", rows, cols, seed=500 + rows)
    q8, s8 = oracle.quantize_to_q8(oracle.gauss(600 + cols, cols))
    ref = oracle.q4_0_matvec_blockint(q, q8, s8, rows, cols)
    got = hip.q4_matvec(q, q8, s8, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # and within tolerance of the x86 scalar order the reference's C kernel uses on this host
    x86 = oracle.q4_0_matvec_x86(q, q8, s8, rows, cols)
    assert rel_err(got, x86) <= REL_TOL


def test_q4_0_matvec_fuzzed_bytes_bit_exact(hip):
    rng = np.random.default_rng(21)
    rows, cols = 777, 1024
    q = rng.integers(0, 256, rows * cols // 32 * 18, dtype=np.uint8)
    q.reshape(-1, 18)[:, 1] &= 0x3B
    q8 = rng.integers(-128, 128, cols, dtype=np.int8)
    s8 = rng.uniform(0, 0.05, cols // 32).astype(np.float32)
    ref = oracle.q4_0_matvec_blockint(q, q8, s8, rows, cols)
    got = hip.q4_matvec(q, q8, s8, rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_f16_decode_all_codes_on_device(hip):
    """Every finite f16 code as a Q4_0 block scale; nibbles 0x99 (q = +1) and x = 1:
    score = 32 * f16(code) exactly — the device decodes subnormals like the reference."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(codes.view(np.float16))
    codes = codes[finite]
    rows = codes.size
    blocks = np.empty((rows, 18), np.uint8)
    blocks[:, 0:2] = codes.view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = 0x99
    q8 = np.ones(32, np.int8)
    s8 = np.ones(1, np.float32)
    got = hip.q4_matvec(blocks.reshape(-1), q8, s8, rows, 32)
    # the reference accumulates from +0.0 (acc = 0.0 + p), which maps -0.0 to +0.0
    want = np.float32(0.0) + codes.view(np.float16).astype(np.float32) * np.float32(32.0)
    ref = oracle.q4_0_matvec_blockint(blocks.reshape(-1), q8, s8, rows, 32)
    assert np.array_equal(ref.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m", [1, 4, 8])
@pytest.mark.parametrize("rows,cols", [(100, 256), (14336, 4096)])
def test_q8_matvec_bit_exact(hip, m, rows, cols):
    print(f"[q8] m={m} rows={rows} cols={cols}", flush=True)
    w = oracle.gauss(700 + rows, rows * cols, 0.0, 0.02)
    wq, ws = oracle.quantize_weights_q8(w, rows, cols)
    xs = [oracle.quantize_to_q8(oracle.gauss(800 + i, cols)) for i in range(m)]
    xq = np.concatenate([a for a, _ in xs])
    xsc = np.concatenate([b for _, b in xs])
    got = hip.q8_matvec(wq, ws, xq, xsc, rows, cols)
    for i in range(m):
        ref = oracle.q8_matvec(wq, ws, xs[i][0], xs[i][1], rows, cols)
        assert np.array_equal(got[i].view(np.uint32), ref.view(np.uint32)), i


@pytest.mark.parametrize("m,rows,cols", [(3, 37, 160), (5, 250, 544), (8, 17, 14336), (2, 1, 32)])
def test_q8_matvec_ragged_bit_exact(hip, m, rows, cols):
    """Odd batch sizes (run as 8/4/2/1 chunks), block counts that leave part of the last
    16-block step empty, row counts off the 16-row tile, and a hidden size whose x image
    only fits LDS two activation rows at a time."""
    print(f"[q8 ragged] m={m} rows={rows} cols={cols}", flush=True)
    w = oracle.gauss(710 + rows, rows * cols, 0.0, 0.02)
    wq, ws = oracle.quantize_weights_q8(w, rows, cols)
    xs = [oracle.quantize_to_q8(oracle.gauss(810 + i, cols)) for i in range(m)]
    got = hip.q8_matvec(wq, ws, np.concatenate([a for a, _ in xs]), np.concatenate([b for _, b in xs]), rows, cols)
    for i in range(m):
        ref = oracle.q8_matvec(wq, ws, xs[i][0], xs[i][1], rows, cols)
        assert np.array_equal(got[i].view(np.uint32), ref.view(np.uint32)), i


@pytest.mark.parametrize("m,rows,cols", [(3, 1000, 2560), (2, 17, 64), (11, 1000, 2560), (9, 300, 4096),
                                         (5, 64, 4096), (8, 33, 160), (2, 200, 384), (6, 100, 1152),
                                         (7, 4100, 2688), (4, 1, 512), (3, 70, 8192)])
def test_q4_0_matvec_batched_dev_bit_exact(hip, m, rows, cols):
    """Q4_0 x Q8 over several activation rows through the device entry point: each row
    equals the single-row block-integer order.  Passes of up to 8 rows (11 rows: 8 + 3;
    9 rows: 8 + 1), a partial workgroup of rows (17), hidden 64 .. 8192, an odd block
    count (8, 33, 160), and on the matrix-core kernel (hidden a multiple of 128) odd
    counts of four-block quads (3, 9, 21: the last pair of quads half past the row), a
    single row and a padded row count; hidden 8192 has an x image too large for its LDS
    and takes the lane-group kernel."""
    torch = pytest.importorskip("torch")
    print(f"[q4_0 batched] m={m} rows={rows} cols={cols}", flush=True)
    q = weights("q4_0", rows, cols, seed=520 + rows)
    xs = [oracle.quantize_to_q8(oracle.gauss(620 + i, cols)) for i in range(m)]
    h = hip.register_weight(larql_hip.Q4_0, q, rows, cols)
    try:
        dq = torch.from_numpy(np.concatenate([a for a, _ in xs])).cuda()
        ds = torch.from_numpy(np.concatenate([b for _, b in xs])).cuda()
        dy = torch.empty(m * rows, device="cuda", dtype=torch.float32)
        hip.matvec_dev(h, dq, dy, m=m, x_scales=ds)
        hip.synchronize()
        got = dy.cpu().numpy().reshape(m, rows)
    finally:
        hip.release_weight(h)
    for i in range(m):
        ref = oracle.q4_0_matvec_blockint(q, xs[i][0], xs[i][1], rows, cols)
        assert np.array_equal(got[i].view(np.uint32), ref.view(np.uint32)), i


def test_quantize_to_q8_bit_exact(hip):
    x = oracle.gauss(901, 32 * 1000)
    x[:32] = 0.0                                     # zero block -> scale 0, q 0
    x[32:64] = np.linspace(-127, 127, 32, dtype=np.float32)
    x[64:96] = np.float32(1e-30)
    x[96:128] *= np.float32(1e4)
    x[128] = 2.5
    x[160:192] = np.nan                              # all-NaN block -> scale 0 (the fold starts at 0)
    x[200] = np.nan                                  # one NaN -> code 0, the scale from the rest
    x[224:256] = np.float32(3.0)
    x[230] = np.inf                                  # scale inf, inv 0: finite -> 0, inf * 0 = NaN -> 0
    x[262] = -np.inf
    q, s = hip.quantize_to_q8(x)
    rq, rs = oracle.quantize_to_q8(x)
    assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


def test_invalid_shapes_return_none(hip):
    be = larql_hip.HipBackend(0, strict=False)
    try:
        q = np.zeros(148, np.uint8)
        assert be.q4k_matvec(q, np.zeros(100, np.float32), 1, 100) is None
        assert "multiple of 256" in be.last_error()
        assert be.q4k_matvec(q, np.zeros(256, np.float32), 2, 256) is None   # buffer too small
        assert "too small" in be.last_error()
    finally:
        be.close()


def test_weight_cache_reuse_and_forget(hip):
    rows, cols = 64, 512
    q = weights("q4k", rows, cols, seed=1)
    x = oracle.gauss(2, cols)
    a = hip.q4k_matvec(q, x, rows, cols)
    b = hip.q4k_matvec(q, x, rows, cols)              # served from the cache
    assert np.array_equal(a, b)
    q[20:40] ^= 0x5A                                   # rewrite in place -> must forget first
    hip.forget_host(q)
    c = hip.q4k_matvec(q, x, rows, cols)
    ref = oracle.q4k_matvec(q, x, rows, cols)
    assert rel_err(c, ref) <= REL_TOL


@pytest.mark.parametrize("fmt", ["q4_0", "q4k", "q6k", "q8"])
def test_device_weight_quantizers_bit_exact(hip, fmt):
    """Device quantizers produce the reference quantizers' bytes (q4_common.rs:50-239,
    q8_matvec.rs:11-34), including zero blocks, constant blocks and large magnitudes."""
    rows, cols = 96, 2048
    w = oracle.gauss(1000, rows * cols, 0.0, 0.02)
    w[:256] = 0.0
    w[256:512] = 0.5
    w[512:768] *= np.float32(1e3)
    w[768:1024] = np.abs(w[768:1024])
    if fmt == "q4_0":
        assert np.array_equal(hip.quantize_weights(larql_hip.Q4_0, w), oracle.quantize_q4_0(w))
    elif fmt == "q4k":
        assert np.array_equal(hip.quantize_weights(larql_hip.Q4_K, w), oracle.quantize_q4_k(w))
    elif fmt == "q6k":
        assert np.array_equal(hip.quantize_weights(larql_hip.Q6_K, w), oracle.quantize_q6_k(w))
    else:
        q, s = hip.quantize_weights(larql_hip.Q8_0, w)
        rq, rs = oracle.quantize_weights_q8(w, rows, cols)
        assert np.array_equal(q, rq) and np.array_equal(s.view(np.uint32), rs.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(300, 4096), (14336, 4096), (4096, 14336), (28672, 4096)])
def test_read_floor_reads_every_block(hip, rows, cols):
    """The plain-read floor kernel folds the weight's device bytes by XOR, a linear map:
    one nibble bit flipped in the first or the last super-block of the host bytes flips
    exactly one bit of the total fold (so both ends of the allocation are read), the total
    does not depend on the launch shape (every byte read exactly once in each), and the
    same bytes give the same fold on every call."""
    import torch

    print(f"[read floor] rows={rows} cols={cols}", flush=True)
    q = weights("q4k", rows, cols, seed=7 + rows)
    words = 4 * ((rows + 63) // 64)

    def fold(raw, shapes=((0, 0),)):
        h = hip.register_weight(larql_hip.Q4_K, raw, rows, cols)
        res = []
        for g, t in shapes:
            out = torch.zeros(max(words, g), dtype=torch.int32, device="cuda")
            hip.read_floor_dev(h, out, g, t)
            hip.read_floor_dev(h, out, g, t)
            torch.cuda.synchronize()
            res.append(int(np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))))
        hip.release_weight(h)
        hip.forget_host(raw)
        return res

    base = fold(q.copy(), ((0, 0), (2048, 256), (37, 1024), (7, 192)))
    assert len(set(base)) == 1, [hex(v) for v in base]
    assert fold(q.copy())[0] == base[0]
    for pos in (20 + 5, q.size - 1):
        m = q.copy()
        m[pos] ^= 0x10
        d = fold(m)[0] ^ base[0]
        assert bin(d).count("1") == 1, (pos, hex(d))
    h = hip.register_weight(larql_hip.Q4_K, q, rows, cols)
    try:
        for g, t, n in ((64, 256, 63), (8, 100, 8), (8, 2048, 8)):
            with pytest.raises(larql_hip.LarqlHipError):
                hip.read_floor_dev(h, torch.zeros(n, dtype=torch.int32, device="cuda"), g, t)
    finally:
        hip.release_weight(h)
        hip.forget_host(q)


def test_read_floor_other_formats_explicit_shapes(hip):
    """Weights of the other formats are read in explicit launch shapes only: the fold is
    the same in every shape (each device byte read once) and changes when one weight byte
    does; the matvec's own shape (0, 0) is known for Q4_K-family weights alone."""
    import torch

    rows, cols = 1000, 2560
    w = oracle.gauss(901, rows * cols, 0.0, 0.02)
    wq, ws = oracle.quantize_weights_q8(w, rows, cols)

    def folds(qbytes):
        h = hip.register_weight(larql_hip.Q8_0, qbytes, rows, cols, q8_scales=ws)
        try:
            res = []
            for g, t in ((64, 256), (300, 128), (7, 1024)):
                out = torch.zeros(g, dtype=torch.int32, device="cuda")
                hip.read_floor_dev(h, out, g, t)
                torch.cuda.synchronize()
                res.append(int(np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))))
            with pytest.raises(larql_hip.LarqlHipError):
                hip.read_floor_dev(h, torch.zeros(64, dtype=torch.int32, device="cuda"), 0, 0)
            return res
        finally:
            hip.release_weight(h)
            hip.forget_host(qbytes)

    base = folds(wq.copy())
    assert len(set(base)) == 1, [hex(v) for v in base]
    m = wq.copy()
    m[12345] ^= 0x04
    assert bin(folds(m)[0] ^ base[0]).count("1") == 1
