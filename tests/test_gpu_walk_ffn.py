"""GPU parity of the Q4_0 walk-FFN pair: q4_vecmat (LC/src/backend.rs:56-60 ->
LC/csrc/q4_dot.c:201-232) and q4_matvec_pair_batch (backend.rs:64-69, Metal
LC/src/metal/ops/q4_batched.rs:19-80), as the vindex walk FFN calls them
(LI/src/vindex/walk_ffn.rs:233-330).

Bars:
  * vecmat: max|gpu - cpu| / max|cpu| <= 1e-3 against the oracle's x86 order (the
    reference sums each column over the rows in one serial chain; the kernel sums row
    chunks and adds the chunk totals in order, so only f32 rounding differs — measured
    ~1e-7).  The skip of rows with |act| < 1e-10 is checked with rows whose weights
    would dominate the result if they were not skipped.
  * pair batch: BIT-EXACT with quantize_to_q8 + the block-integer Q4_0 matvec per row.
"""
import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu

REL_TOL = 1e-3


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


# (20000, 8192): 32 column tiles, few chunks of many rows
@pytest.mark.parametrize("inter,hidden", [(10240, 2560), (1, 32), (7, 64), (300, 544), (14336, 4096), (4099, 1056),
                                          (20000, 8192)])
def test_q4_vecmat_matches_oracle(hip, inter, hidden):
    print(f"[vecmat] inter={inter} hidden={hidden}", flush=True)
    q4 = oracle.quantize_q4_0(oracle.gauss(900 + inter, inter * hidden, 0.0, 0.02))
    act = oracle.gauss(901 + hidden, inter)
    act[::5] = 0.0                      # the walk FFN's activations are mostly zero
    got = hip.q4_vecmat(act, q4, inter, hidden)
    ref = oracle.q4_0_vecmat(act, q4, inter, hidden)
    e = rel_err(got, ref)
    print(f"  rel_err {e:.2e}", flush=True)
    assert e <= REL_TOL, e


def test_q4_vecmat_skips_tiny_activations(hip):
    """Rows with |act| just below 1e-10 carry scales of 6e4 (f16 max): if they were added,
    they would outweigh every other row by ~1e4."""
    inter, hidden = 1000, 256
    rng = np.random.default_rng(7)
    q4 = oracle.quantize_q4_0(oracle.gauss(17, inter * hidden, 0.0, 0.02))
    blocks = q4.reshape(inter, hidden // 32, 18)
    act = oracle.gauss(18, inter)
    tiny = rng.choice(inter, 50, replace=False)
    act[tiny[:25]] = 9.9e-11
    act[tiny[25:]] = -9.9e-11
    blocks[tiny, :, 0:2] = np.frombuffer(np.float16(65504.0).tobytes(), np.uint8)
    blocks[tiny, :, 2:] = 0xFF
    act[3] = 1.0001e-10               # just outside the band: kept
    got = hip.q4_vecmat(act, q4, inter, hidden)
    ref = oracle.q4_0_vecmat(act, q4, inter, hidden)
    assert rel_err(got, ref) <= REL_TOL
    # and the big rows really are absent from both
    assert np.max(np.abs(ref)) < 100.0


def test_q4_vecmat_all_zero_activation(hip):
    inter, hidden = 64, 128
    q4 = oracle.quantize_q4_0(oracle.gauss(19, inter * hidden))
    got = hip.q4_vecmat(np.zeros(inter, np.float32), q4, inter, hidden)
    assert np.array_equal(got, np.zeros(hidden, np.float32))


def test_q4_vecmat_fuzzed_bytes(hip):
    inter, hidden = 777, 1024
    rng = np.random.default_rng(23)
    q4 = rng.integers(0, 256, inter * hidden // 32 * 18, dtype=np.uint8)
    blocks = q4.reshape(-1, 18)
    blocks[:, 0:2] = np.frombuffer(rng.uniform(-0.05, 0.05, blocks.shape[0]).astype(np.float16).tobytes(),
                                   np.uint8).reshape(-1, 2)
    act = oracle.gauss(24, inter)
    got = hip.q4_vecmat(act, q4, inter, hidden)
    ref = oracle.q4_0_vecmat(act, q4, inter, hidden)
    assert rel_err(got, ref) <= REL_TOL


def test_vecmat_dev_matches_host_entry(hip):
    torch = pytest.importorskip("torch")
    inter, hidden = 10240, 2560
    q4 = oracle.quantize_q4_0(oracle.gauss(31, inter * hidden, 0.0, 0.02))
    act = oracle.gauss(32, inter)
    h = hip.register_weight(larql_hip.Q4_0, q4, inter, hidden)
    try:
        da = torch.from_numpy(act).cuda()
        do = torch.empty(hidden, device="cuda", dtype=torch.float32)
        hip.vecmat_dev(h, da, do)
        hip.synchronize()
        dev = do.cpu().numpy()
    finally:
        hip.release_weight(h)
    host = hip.q4_vecmat(act, q4, inter, hidden)
    assert np.array_equal(dev.view(np.uint32), host.view(np.uint32))   # same kernels, same order


def test_vecmat_dev_graph_replays_and_shape_changes(hip):
    """The vecmat's chunk partials live in one context buffer that grows with the shape:
    eager calls over shapes with more and fewer column tiles and chunks, then a captured
    graph of two calls replayed three times with eager calls between, all bit-identical
    to the first eager results (the summation order is fixed)."""
    torch = pytest.importorskip("torch")
    shapes = [(4096, 1024), (2048, 8192), (10240, 2560)]
    hs, acts, outs, ref = [], [], [], []
    try:
        for i, (inter, hidden) in enumerate(shapes):
            q4 = oracle.quantize_q4_0(oracle.gauss(60 + i, inter * hidden, 0.0, 0.02))
            hs.append(hip.register_weight(larql_hip.Q4_0, q4, inter, hidden))
            acts.append(torch.from_numpy(oracle.gauss(70 + i, inter)).cuda())
            outs.append(torch.empty(hidden, device="cuda", dtype=torch.float32))
            hip.vecmat_dev(hs[-1], acts[-1], outs[-1])
            hip.synchronize()
            ref.append(outs[-1].cpu().numpy().copy())
            e = rel_err(ref[-1], oracle.q4_0_vecmat(acts[-1].cpu().numpy(), q4, inter, hidden))
            assert e <= REL_TOL, (inter, hidden, e)
        for i in (1, 0, 2):   # again, in another order
            outs[i].fill_(7.0)
            hip.vecmat_dev(hs[i], acts[i], outs[i])
            hip.synchronize()
            assert np.array_equal(outs[i].cpu().numpy().view(np.uint32), ref[i].view(np.uint32)), i
        side = torch.cuda.Stream()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            hip.vecmat_dev(hs[2], acts[2], outs[2], stream=side)
            hip.vecmat_dev(hs[0], acts[0], outs[0], stream=side)
        for rep in range(3):
            outs[0].fill_(7.0)
            outs[2].fill_(7.0)
            hip.vecmat_dev(hs[1], acts[1], outs[1])
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for i in range(3):
                assert np.array_equal(outs[i].cpu().numpy().view(np.uint32), ref[i].view(np.uint32)), (rep, i)
        del graph
    finally:
        for h in hs:
            hip.release_weight(h)


# (6, 10240, 2560), (17, 300, 576), (130, 200, 128): several positions (one launch per pass of
# up to 8, ragged row tiles); (1, 64, 32): one position; (9, 300, 544): hidden not a multiple
# of 64; (9, 640, 256): the matrix-core kernel, passes of 8 and 1 rows; (5, 1000, 1152),
# (3, 130, 384): the matrix-core kernel with an odd count of four-block quads (9, 3) over
# both matrices of one launch
@pytest.mark.parametrize("seq,rows,hidden", [(6, 10240, 2560), (17, 300, 576), (130, 200, 128), (1, 64, 32),
                                             (9, 300, 544), (9, 640, 256), (5, 1000, 1152), (3, 130, 384)])
def test_pair_batch_bit_exact(hip, seq, rows, hidden):
    print(f"[pair batch] seq={seq} rows={rows} hidden={hidden}", flush=True)
    gate = oracle.quantize_q4_0(oracle.gauss(41 + seq, rows * hidden, 0.0, 0.02))
    up = oracle.quantize_q4_0(oracle.gauss(42 + seq, rows * hidden, 0.0, 0.02))
    x = oracle.gauss(43, seq * hidden).reshape(seq, hidden)
    g, u = hip.q4_matvec_pair_batch(gate, up, x, seq, rows, hidden)
    for s in range(seq):
        q8, q8s = oracle.quantize_to_q8(x[s])
        rg = oracle.q4_0_matvec_blockint(gate, q8, q8s, rows, hidden)
        ru = oracle.q4_0_matvec_blockint(up, q8, q8s, rows, hidden)
        assert np.array_equal(g[s].view(np.uint32), rg.view(np.uint32)), s
        assert np.array_equal(u[s].view(np.uint32), ru.view(np.uint32)), s


def test_pair_batch_dev(hip):
    torch = pytest.importorskip("torch")
    seq, rows, hidden = 4, 2048, 1024
    gate = oracle.quantize_q4_0(oracle.gauss(51, rows * hidden, 0.0, 0.02))
    up = oracle.quantize_q4_0(oracle.gauss(52, rows * hidden, 0.0, 0.02))
    x = oracle.gauss(53, seq * hidden).reshape(seq, hidden)
    hg = hip.register_weight(larql_hip.Q4_0, gate, rows, hidden)
    hu = hip.register_weight(larql_hip.Q4_0, up, rows, hidden)
    try:
        dx = torch.from_numpy(x).cuda()
        dg = torch.empty(seq * rows, device="cuda", dtype=torch.float32)
        du = torch.empty(seq * rows, device="cuda", dtype=torch.float32)
        hip.pair_batch_dev(hg, hu, dx, seq, dg, du)
        hip.synchronize()
        g = dg.cpu().numpy().reshape(seq, rows)
        u = du.cpu().numpy().reshape(seq, rows)
    finally:
        hip.release_weight(hg)
        hip.release_weight(hu)
    for s in range(seq):
        q8, q8s = oracle.quantize_to_q8(x[s])
        assert np.array_equal(g[s].view(np.uint32), oracle.q4_0_matvec_blockint(gate, q8, q8s, rows, hidden).view(np.uint32))
        assert np.array_equal(u[s].view(np.uint32), oracle.q4_0_matvec_blockint(up, q8, q8s, rows, hidden).view(np.uint32))


@pytest.mark.parametrize("offset", [0, 1])
def test_pair_batch_dev_quantizes_like_quantize_to_q8(hip, offset):
    """The device pair batch quantizes f32 rows inside the matrix-core kernel (x 16-byte
    aligned) or through the separate quantizer (offset 1: x one float past an aligned
    address): both bit-exact with quantize_to_q8 + the block-integer matvec, over zero, NaN,
    tiny, huge and half-way activations."""
    torch = pytest.importorskip("torch")
    seq, rows, hidden = 7, 1280, 512
    gate = oracle.quantize_q4_0(oracle.gauss(55, rows * hidden, 0.0, 0.02))
    up = oracle.quantize_q4_0(oracle.gauss(56, rows * hidden, 0.0, 0.02))
    x = oracle.gauss(57, seq * hidden).reshape(seq, hidden)
    x[0, :32] = 0.0
    x[1, 32:64] = np.nan
    x[1, 70] = np.nan
    x[2, :32] = np.float32(1e-30)
    x[3, 96:128] *= np.float32(1e4)
    x[4, :32] = np.arange(-16, 16, dtype=np.float32) + np.float32(0.5)
    x[4, 31] = np.float32(127.0)                     # scale 1: the others are rounding ties
    x[5, 64:96] = np.float32(127.0)
    x[6, :] = -x[6, :]
    hg = hip.register_weight(larql_hip.Q4_0, gate, rows, hidden)
    hu = hip.register_weight(larql_hip.Q4_0, up, rows, hidden)
    try:
        buf = torch.zeros(seq * hidden + 4, device="cuda", dtype=torch.float32)
        buf[offset:offset + seq * hidden] = torch.from_numpy(x.reshape(-1)).cuda()
        dx = buf[offset:offset + seq * hidden]
        dg = torch.empty(seq * rows, device="cuda", dtype=torch.float32)
        du = torch.empty(seq * rows, device="cuda", dtype=torch.float32)
        hip.pair_batch_dev(hg, hu, dx, seq, dg, du)
        hip.synchronize()
        g = dg.cpu().numpy().reshape(seq, rows)
        u = du.cpu().numpy().reshape(seq, rows)
    finally:
        hip.release_weight(hg)
        hip.release_weight(hu)
    for s in range(seq):
        q8, q8s = oracle.quantize_to_q8(x[s])
        assert np.array_equal(g[s].view(np.uint32), oracle.q4_0_matvec_blockint(gate, q8, q8s, rows, hidden).view(np.uint32)), s
        assert np.array_equal(u[s].view(np.uint32), oracle.q4_0_matvec_blockint(up, q8, q8s, rows, hidden).view(np.uint32)), s


def test_pair_batch_shape_mismatch_is_an_error():
    be = larql_hip.HipBackend(0, strict=False)
    try:
        g = oracle.quantize_q4_0(oracle.gauss(1, 64 * 64))
        u = oracle.quantize_q4_0(oracle.gauss(2, 32 * 64))
        x = np.zeros((1, 64), np.float32)
        assert be.q4_matvec_pair_batch(g, u, x, 1, 64, 64) is None   # up is too short for 64 rows
    finally:
        be.close()
