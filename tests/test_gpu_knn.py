"""GPU parity of the vindex gate-KNN (LV/src/index/gate.rs) against the CPU oracle.

Bars:
  * f32 gate scores: BIT-EXACT with the oracle's canonical order (one fma chain per
    (feature, query) over k from +0, lo_gate_scores_f32).  The reference hands the
    order to matrixmultiply (parity of its bit patterns is unpinned); the kernel and
    the oracle fix the same order, so indices are comparable bit for bit.
  * Q4_0 gate scores (gate_knn_q4, gate.rs:711-731): BIT-EXACT with quantize_to_q8 +
    q4_0 block-integer matvec (LC/csrc/q4_dot.c:58-89 order).
  * top-k (top_k_from_scores, gate.rs:307-316; signed: walk.rs:563-580): indices and
    values BIT-EXACT with the oracle's selection, ties in index order.
"""
import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu


def oracle_knn_f32(gate, queries, features, hidden, k):
    idx, val = [], []
    for q in queries:
        s = oracle.gate_scores_f32(gate, q, features, hidden)
        i, v = oracle.topk_abs(s, k)
        idx.append(i)
        val.append(v)
    return np.array(idx), np.array(val)


def oracle_knn_q4(q4, queries, features, hidden, k):
    idx, val = [], []
    for q in queries:
        q8, q8s = oracle.quantize_to_q8(q)
        s = oracle.q4_0_matvec_blockint(q4, q8, q8s, features, hidden)
        i, v = oracle.topk_abs(s, k)
        idx.append(i)
        val.append(v)
    return np.array(idx), np.array(val)


@pytest.mark.parametrize("features,hidden,nq,k", [(1000, 2560, 37, 32), (10240, 2560, 8, 32), (64, 256, 300, 64),
                                                  (130, 64, 3, 1)])
def test_gate_knn_f32_bit_exact(hip, features, hidden, nq, k):
    print(f"[knn f32] F={features} K={hidden} nq={nq} k={k}", flush=True)
    gate = oracle.gauss(11, features * hidden, 0.0, 0.02).reshape(features, hidden)
    queries = oracle.gauss(12, nq * hidden).reshape(nq, hidden)
    got = hip.gate_knn(gate, features, hidden, queries, k, fmt=larql_hip.F32)
    ref_i, ref_v = oracle_knn_f32(gate, queries, features, hidden, k)
    np.testing.assert_array_equal(got[0], ref_i)
    np.testing.assert_array_equal(got[1].view(np.uint32), ref_v.view(np.uint32))


def test_gate_scores_f32_bit_exact(hip):
    torch = pytest.importorskip("torch")
    features, hidden, nq = 200, 512, 257   # partial feature tile and two query tiles
    gate = oracle.gauss(21, features * hidden, 0.0, 0.02).reshape(features, hidden)
    queries = oracle.gauss(22, nq * hidden).reshape(nq, hidden)
    h = hip.register_weight(larql_hip.F32, gate, features, hidden)
    try:
        dq = torch.from_numpy(queries).cuda()
        ds = torch.empty(nq * features, device="cuda", dtype=torch.float32)
        hip.gate_scores_dev([h], dq, nq, ds)
        hip.synchronize()
        got = ds.cpu().numpy().reshape(nq, features)
        ref = np.stack([oracle.gate_scores_f32(gate, q, features, hidden) for q in queries])
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        hip.release_weight(h)


@pytest.mark.parametrize("features,hidden,nq,k", [(10240, 2560, 6, 32), (1000, 2560, 130, 17), (64, 64, 2, 64)])
def test_gate_knn_q4_bit_exact(hip, features, hidden, nq, k):
    print(f"[knn q4] F={features} K={hidden} nq={nq} k={k}", flush=True)
    gate = oracle.gauss(31, features * hidden, 0.0, 0.02)
    q4 = oracle.quantize_q4_0(gate)
    queries = oracle.gauss(32, nq * hidden).reshape(nq, hidden)
    got = hip.gate_knn(q4, features, hidden, queries, k, fmt=larql_hip.Q4_0)
    ref_i, ref_v = oracle_knn_q4(q4, queries, features, hidden, k)
    np.testing.assert_array_equal(got[0], ref_i)
    np.testing.assert_array_equal(got[1].view(np.uint32), ref_v.view(np.uint32))


def test_gate_knn_q4_fuzzed_bytes(hip):
    """Random Q4_0 bytes (all nibbles, scales from a bounded f16 range)."""
    features, hidden, nq, k = 300, 512, 5, 32
    rng = np.random.default_rng(41)
    q4 = rng.integers(0, 256, size=features * hidden // 32 * 18, dtype=np.uint8)
    blocks = q4.reshape(-1, 18)
    blocks[:, 0:2] = np.frombuffer(rng.uniform(-0.05, 0.05, blocks.shape[0]).astype(np.float16).tobytes(),
                                   np.uint8).reshape(-1, 2)
    queries = oracle.gauss(42, nq * hidden).reshape(nq, hidden)
    got = hip.gate_knn(q4, features, hidden, queries, k, fmt=larql_hip.Q4_0)
    ref_i, ref_v = oracle_knn_q4(q4, queries, features, hidden, k)
    np.testing.assert_array_equal(got[0], ref_i)
    np.testing.assert_array_equal(got[1].view(np.uint32), ref_v.view(np.uint32))


def _q4_scores(hip, torch, q4, queries, features, hidden):
    h = hip.register_weight(larql_hip.Q4_0, q4, features, hidden)
    try:
        nq = queries.shape[0]
        dq = torch.from_numpy(np.ascontiguousarray(queries, dtype=np.float32)).cuda()
        ds = torch.empty(nq * features, device="cuda", dtype=torch.float32)
        hip.gate_scores_dev([h], dq, nq, ds)
        hip.synchronize()
        return ds.cpu().numpy().reshape(nq, features)
    finally:
        hip.release_weight(h)


def _q4_scores_ref(q4, queries, features, hidden):
    out = []
    for q in queries:
        q8, q8s = oracle.quantize_to_q8(q)
        out.append(oracle.q4_0_matvec_blockint(q4, q8, q8s, features, hidden))
    return np.stack(out)


@pytest.mark.parametrize("features,hidden,nq", [(200, 192, 257), (130, 2560, 33), (16, 64, 1), (1000, 512, 129)])
def test_gate_scores_q4_bit_exact(hip, features, hidden, nq):
    """Every score: hidden sizes of an odd number of block pairs, partial feature tiles,
    query counts off the 8-query groups and the 16-group tiles."""
    torch = pytest.importorskip("torch")
    print(f"[knn q4 scores] F={features} K={hidden} nq={nq}", flush=True)
    q4 = oracle.quantize_q4_0(oracle.gauss(61, features * hidden, 0.0, 0.02))
    queries = oracle.gauss(62, nq * hidden).reshape(nq, hidden)
    got = _q4_scores(hip, torch, q4, queries, features, hidden)
    ref = _q4_scores_ref(q4, queries, features, hidden)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("nibble", [0x00, 0xFF, 0x0F])
def test_gate_scores_q4_extreme_codes(hip, nibble):
    """Block dots at their largest magnitudes: every code 0 or 15 against queries whose
    int8 values are all +-127 (constant rows and alternating signs); the int32 dots and
    their conversion to f32 are exact there."""
    torch = pytest.importorskip("torch")
    features, hidden = 48, 2560
    print(f"[knn q4 extreme] nibble byte {nibble:#x}", flush=True)
    blocks = np.zeros((features * hidden // 32, 18), dtype=np.uint8)
    blocks[:, 2:] = nibble
    blocks[:, 0:2] = np.frombuffer(np.full(blocks.shape[0], 0.03, dtype=np.float16).tobytes(), np.uint8).reshape(-1, 2)
    q4 = blocks.reshape(-1)
    queries = np.stack([np.full(hidden, 1.0), np.full(hidden, -2.5), np.tile([3.0, -3.0], hidden // 2),
                        oracle.gauss(63, hidden)]).astype(np.float32)
    got = _q4_scores(hip, torch, q4, queries, features, hidden)
    ref = _q4_scores_ref(q4, queries, features, hidden)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def _topk_rows(hip, torch, rows, k, signed):
    n = rows.shape[1]
    ds = torch.from_numpy(np.ascontiguousarray(rows, dtype=np.float32)).cuda()
    di = torch.empty(rows.shape[0] * k, device="cuda", dtype=torch.int32)
    dv = torch.empty(rows.shape[0] * k, device="cuda", dtype=torch.float32)
    hip.topk_dev(ds, rows.shape[0], n, k, di, dv, signed=signed)
    hip.synchronize()
    return di.cpu().numpy().view(np.uint32).reshape(-1, k), dv.cpu().numpy().reshape(-1, k)


@pytest.mark.parametrize("signed", [False, True])
def test_topk_ties_zeros_and_sizes(hip, signed):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(51)
    cases = []
    # duplicates, +-0, all equal, sign pairs with equal magnitude, huge values
    r = rng.standard_normal(1000).astype(np.float32)
    r[::7] = 0.0
    r[3::11] = -0.0
    r[5::13] = 1.5
    r[6::13] = -1.5
    cases.append(r)
    cases.append(np.zeros(777, np.float32))
    cases.append(np.full(500, -2.0, np.float32))
    cases.append(np.concatenate([rng.standard_normal(300), [np.inf, -np.inf, 3e38, -3e38]]).astype(np.float32))
    for n in (64, 12288, 12289, 128256):   # register path limit is 48 * 256 = 12288
        cases.append(rng.standard_normal(n).astype(np.float32))
    for row in cases:
        for k in (1, 32, 64, 300, 512):
            if k > row.size:
                continue
            gi, gv = _topk_rows(hip, torch, row[None, :], k, signed)
            ri, rv = (oracle.topk_signed if signed else oracle.topk_abs)(row, k)
            np.testing.assert_array_equal(gi[0], ri, err_msg=f"n={row.size} k={k} signed={signed}")
            np.testing.assert_array_equal(gv[0].view(np.uint32), rv.view(np.uint32))


@pytest.mark.parametrize("signed", [False, True])
def test_topk_mass_ties_linear_time(hip, signed):
    """More than the 2048 LDS candidates tie at the k-th key: all-zero rows of the lm-head
    (128256) and gate (10240) widths, and a row with 5000 equal values under 100 larger
    ones.  Ties resolve in index order by a select over their indices (linear time)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(52)
    spiky = rng.uniform(-0.5, 0.5, 20000).astype(np.float32)
    spiky[rng.choice(20000, 5000, replace=False)] = 1.0
    spiky[rng.choice(20000, 100, replace=False)] = 2.0 + rng.uniform(0, 1, 100).astype(np.float32)
    for row in (np.zeros(128256, np.float32), np.zeros(10240, np.float32), spiky):
        for k in (1, 64, 512):
            print(f"[topk ties] n={row.size} k={k} signed={signed}", flush=True)
            gi, gv = _topk_rows(hip, torch, np.stack([row, row[::-1].copy()]), k, signed)
            for r, rr in enumerate((row, row[::-1].copy())):
                ri, rv = (oracle.topk_signed if signed else oracle.topk_abs)(rr, k)
                np.testing.assert_array_equal(gi[r], ri, err_msg=f"n={row.size} k={k}")
                np.testing.assert_array_equal(gv[r].view(np.uint32), rv.view(np.uint32))


@pytest.mark.parametrize("signed", [False, True])
def test_topk_wave_rows_every_path(hip, signed):
    """Rows with k <= 64 and n <= 14336 take one wave per row: row lengths that fill the
    lane registers exactly (4096, 10240, 14336) or leave a partial last register (40, 65,
    4097, 10241), five rows per launch (a partial last workgroup of four rows), and rows
    whose candidate list overflows (600 equal largest values; an all-zero row), which
    select over the whole row again."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(53)
    for n in (40, 65, 4096, 4097, 10240, 10241, 14336):
        rows = rng.standard_normal((5, n)).astype(np.float32)
        rows[1, rng.choice(n, min(n, 600), replace=False)] = 7.0    # > 512 tied candidates
        rows[2] = 0.0
        rows[3, ::5] = -rows[3, ::5]                                   # equal magnitudes
        rows[3, 1::5] = rows[3, ::5][: rows[3, 1::5].size]
        for k in (1, 7, 32, 64):
            if k > n:
                continue
            print(f"[topk wave] n={n} k={k} signed={signed}", flush=True)
            gi, gv = _topk_rows(hip, torch, rows, k, signed)
            for r in range(rows.shape[0]):
                ri, rv = (oracle.topk_signed if signed else oracle.topk_abs)(rows[r], k)
                np.testing.assert_array_equal(gi[r], ri, err_msg=f"n={n} k={k} row={r}")
                np.testing.assert_array_equal(gv[r].view(np.uint32), rv.view(np.uint32))


def test_topk_k_above_row_length_is_clamped(hip):
    """top_k.min(len) (LV/src/index/walk.rs:569): a request for more entries than the row has
    returns the whole row ranked; the slots past it hold index 0xFFFFFFFF and score 0."""
    gate = oracle.gauss(61, 8 * 64).reshape(8, 64)
    q = oracle.gauss(62, 64)
    got = hip.gate_knn(gate, 8, 64, q, 11, fmt=larql_hip.F32)
    ri, rv = oracle_knn_f32(gate, q[None, :], 8, 64, 8)
    np.testing.assert_array_equal(got[0][0, :8], ri[0])
    np.testing.assert_array_equal(got[1][0, :8].view(np.uint32), rv[0].view(np.uint32))
    assert np.all(got[0][0, 8:] == 0xFFFFFFFF) and np.all(got[1][0, 8:] == 0.0)


@pytest.mark.parametrize("signed", [False, True])
def test_topk_k_above_selection_bound_sorts(hip, signed):
    """A top_k above LARQL_HIP_TOPK_MAX (512) is taken, as the reference clamps k only to the
    row length (gate.rs:307-316; range-filtered callers ask for top_k * 10, gate.rs:300):
    rows are ranked by a stable sort in the same order (key descending, index ascending).
    Random rows of the gate and lm-head widths, rows with mass ties and +-0, k up to and
    past the row length."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(54)
    for n in (10240, 128256, 700):
        rows = rng.standard_normal((3, n)).astype(np.float32)
        rows[1, ::3] = 0.0
        rows[1, 1::7] = -0.0
        rows[2, rng.choice(n, n // 2, replace=False)] = 1.25   # ties across the k-th place
        rows[2, ::11] = -1.25
        for k in (513, 600, 1000, n, n + 37):
            print(f"[topk sort] n={n} k={k} signed={signed}", flush=True)
            gi, gv = _topk_rows(hip, torch, rows, k, signed)
            for r in range(rows.shape[0]):
                ri, rv = (oracle.topk_signed if signed else oracle.topk_abs)(rows[r], k)
                m = min(k, n)
                np.testing.assert_array_equal(gi[r, :m], ri, err_msg=f"n={n} k={k} row={r}")
                np.testing.assert_array_equal(gv[r, :m].view(np.uint32), rv.view(np.uint32))
                assert np.all(gi[r, m:] == 0xFFFFFFFF) and np.all(gv[r, m:] == 0.0)


@pytest.mark.parametrize("signed", [False, True])
def test_topk_long_rows_in_chunks(hip, signed):
    """Rows longer than one selection kernel's registers are ranked in chunks on many CUs and
    then over the chunks' candidates: row lengths whose last chunk is shorter than k (its
    empty slots must rank after every real score, also when all scores are negative),
    exact multiples of the chunk, mass ties across chunk boundaries, k = 1 .. 512."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(55)
    for n, k in ((4096 * 4 + 3, 32), (4096 * 4, 64), (12288 * 2 + 5, 100), (12288 * 3, 512), (128256, 5),
                 (14337, 1), (40000, 300)):
        rows = rng.standard_normal((3, n)).astype(np.float32)
        rows[1] = -np.abs(rows[1]) - 1.0                  # every score negative
        rows[2, rng.choice(n, n // 3, replace=False)] = -3.0
        rows[2, rng.choice(n, 50, replace=False)] = 3.0    # ties straddle chunk boundaries
        print(f"[topk chunks] n={n} k={k} signed={signed}", flush=True)
        gi, gv = _topk_rows(hip, torch, rows, k, signed)
        for r in range(rows.shape[0]):
            ri, rv = (oracle.topk_signed if signed else oracle.topk_abs)(rows[r], k)
            np.testing.assert_array_equal(gi[r], ri, err_msg=f"n={n} k={k} row={r}")
            np.testing.assert_array_equal(gv[r].view(np.uint32), rv.view(np.uint32))


def test_gate_knn_k_above_selection_bound(hip):
    """gate_knn with top_k = 320 and 1000 (the reference's top_k * 10 fallback sizes) through
    the host and device entry points, f32 and Q4_0, bit-exact with the oracle."""
    torch = pytest.importorskip("torch")
    features, hidden, nq = 4000, 256, 5
    gate = oracle.gauss(91, features * hidden, 0.0, 0.02).reshape(features, hidden)
    queries = oracle.gauss(92, nq * hidden).reshape(nq, hidden)
    q4 = oracle.quantize_q4_0(gate.reshape(-1))
    for k in (320, 1000):
        print(f"[knn sort] F={features} K={hidden} nq={nq} k={k}", flush=True)
        got = hip.gate_knn(gate, features, hidden, queries, k, fmt=larql_hip.F32)
        ri, rv = oracle_knn_f32(gate, queries, features, hidden, k)
        np.testing.assert_array_equal(got[0], ri)
        np.testing.assert_array_equal(got[1].view(np.uint32), rv.view(np.uint32))
        got = hip.gate_knn(q4, features, hidden, queries, k, fmt=larql_hip.Q4_0)
        ri, rv = oracle_knn_q4(q4, queries, features, hidden, k)
        np.testing.assert_array_equal(got[0], ri)
        np.testing.assert_array_equal(got[1].view(np.uint32), rv.view(np.uint32))
    h = hip.register_weight(larql_hip.Q4_0, q4, features, hidden)
    try:
        dq = torch.from_numpy(np.ascontiguousarray(queries, dtype=np.float32)).cuda()
        k = 777
        di = torch.empty(2 * nq * k, device="cuda", dtype=torch.int32)
        dv = torch.empty(2 * nq * k, device="cuda", dtype=torch.float32)
        hip.gate_knn_dev([h, h], dq, nq, k, di, dv)
        hip.synchronize()
        ri, rv = oracle_knn_q4(q4, queries, features, hidden, k)
        gi = di.cpu().numpy().view(np.uint32).reshape(2, nq, k)
        gv = dv.cpu().numpy().reshape(2, nq, k)
        for l in range(2):
            np.testing.assert_array_equal(gi[l], ri)
            np.testing.assert_array_equal(gv[l].view(np.uint32), rv.view(np.uint32))
    finally:
        hip.release_weight(h)


def test_topk_invalid_k_returns_none():
    be = larql_hip.HipBackend(0, strict=False)
    try:
        gate = np.zeros((8, 64), np.float32)
        q = np.zeros(64, np.float32)
        assert be.gate_knn(gate, 8, 64, q, 0, fmt=larql_hip.F32) is None          # k = 0
        assert be.gate_knn(gate, 8, 64, q, 1 << 31, fmt=larql_hip.F32) is None    # rows x k >= 2^31
        assert be.gate_knn(gate, 8, 64, q, 4, fmt=larql_hip.Q4_K) is None         # unsupported format
    finally:
        be.close()


def _pool_map(fn, items):
    """The oracle's ctypes calls run without the GIL: map them over the host's threads."""
    import os
    from concurrent.futures import ThreadPoolExecutor

    n = max(1, min(16, len(os.sched_getaffinity(0))))
    with ThreadPoolExecutor(n) as pool:
        return list(pool.map(fn, items))


def test_gate_knn_34_layers_full_size(hip):
    """The vindex walk shape: 34 layers x gate [10240 x 2560], 256 queries, top-32, in
    f32 and Q4_0, one launch each.  Every list of layers 0 and 33 (2 x 256 of each format)
    is checked against the oracle bit for bit; every list of all 34 layers is checked
    for the selection invariants.  For Q4_0 the same lists are also ranked by the
    reference's x86 order (per-element accumulation, LC/csrc/q4_dot.c:183-195): lists
    whose index sets differ must differ only across a near-tie at the k-th score (a gap
    below twice the largest score difference between the two orders in that row), and
    the counts are printed."""
    torch = pytest.importorskip("torch")
    L, F, K, Q, k = 34, 10240, 2560, 256, 32
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gates, handles_f32, handles_q4, q4_host = [], [], [], {}
    print("[knn 34] building gates", flush=True)
    for l in range(L):
        gen.manual_seed(9000 + l)
        g = torch.randn(F, K, generator=gen, device=dev, dtype=torch.float32) * 0.02
        handles_f32.append(hip.register_weight_device(larql_hip.F32, g, g.numel() * 4, F, K))
        raw = torch.empty(F * K // 32 * 18, dtype=torch.uint8, device=dev)
        hip.quantize_weights_dev(larql_hip.Q4_0, g, F * K, raw)
        hip.synchronize()
        handles_q4.append(hip.register_weight_device(larql_hip.Q4_0, raw, raw.numel(), F, K))
        if l in (0, 33):
            gates.append((l, g.cpu().numpy()))
            q4_host[l] = raw.cpu().numpy()
        del g, raw
    gen.manual_seed(4)
    queries = torch.randn(Q, K, generator=gen, device=dev, dtype=torch.float32)
    qn = queries.cpu().numpy()
    q8 = [oracle.quantize_to_q8(qn[qi]) for qi in range(Q)]
    try:
        for fmt, handles in (("f32", handles_f32), ("q4_0", handles_q4)):
            di = torch.empty(L * Q * k, device=dev, dtype=torch.int32)
            dv = torch.empty(L * Q * k, device=dev, dtype=torch.float32)
            hip.gate_knn_dev(handles, queries, Q, k, di, dv)
            hip.synchronize()
            gi = di.cpu().numpy().view(np.uint32).reshape(L, Q, k)
            gv = dv.cpu().numpy().reshape(L, Q, k)
            print(f"[knn 34] {fmt}: checking invariants", flush=True)
            a = np.abs(gv)
            assert np.all(a[..., :-1] >= a[..., 1:])
            assert all(len(set(r)) == k for r in gi.reshape(-1, k))
            assert gi.max() < F
            for l, g in gates:
                print(f"[knn 34] {fmt}: layer {l}, all {Q} queries against the oracle", flush=True)

                def scores(qi, l=l, g=g):
                    if fmt == "f32":
                        return oracle.gate_scores_f32(g, qn[qi], F, K)
                    return oracle.q4_0_matvec_blockint(q4_host[l], q8[qi][0], q8[qi][1], F, K)

                def check(qi):
                    ri, rv = oracle.topk_abs(scores(qi), k)
                    return (np.array_equal(gi[l, qi], ri) and np.array_equal(gv[l, qi].view(np.uint32), rv.view(np.uint32)))

                ok = _pool_map(check, range(Q))
                bad = [qi for qi in range(Q) if not ok[qi]]
                assert not bad, f"{fmt} layer {l}: queries {bad[:8]} differ from the oracle"
                if fmt != "q4_0":
                    continue

                def x86_cmp(qi, l=l):
                    sb = scores(qi)
                    sx = oracle.q4_0_matvec_x86(q4_host[l], q8[qi][0], q8[qi][1], F, K)
                    delta = float(np.max(np.abs(sx.astype(np.float64) - sb)))
                    xi, _ = oracle.topk_abs(sx, k)
                    srt = np.sort(np.abs(sx.astype(np.float64)))[::-1]
                    gap = srt[k - 1] - srt[k]
                    same = set(xi.tolist()) == set(gi[l, qi].tolist())
                    explained = same
                    if not same:
                        diff = set(xi.tolist()) ^ set(gi[l, qi].tolist())
                        explained = all(abs(abs(float(sx[f])) - srt[k - 1]) <= 2 * delta for f in diff)
                    return same, explained, gap <= 2 * delta

                res = _pool_map(x86_cmp, range(Q))
                n_same = sum(r[0] for r in res)
                n_near = sum(r[2] for r in res)
                print(f"[knn 34] q4_0 layer {l}: x86-order top-{k} index sets identical in {n_same}/{Q} lists; "
                      f"near-ties at the k-th score in {n_near}/{Q}", flush=True)
                assert all(r[1] for r in res), f"layer {l}: an x86-order difference not explained by a near-tie"
    finally:
        for h in handles_f32 + handles_q4:
            hip.release_weight(h)


@pytest.mark.parametrize("vocab,hidden,k", [(10007, 512, 5), (32000, 1024, 64), (64, 64, 64)])
def test_lm_head_knn_q4_bit_exact(hip, vocab, hidden, k):
    """lm_head_knn_backend's Q4 path (LV/src/index/walk.rs:549-583): quantize_to_q8, the
    Q4_0 matvec over the vocab, top-k by signed score (ties in index order)."""
    print(f"[lm-head knn] vocab={vocab} hidden={hidden} k={k}", flush=True)
    head = oracle.quantize_q4_0(oracle.gauss(51, vocab * hidden, 0.0, 0.02))
    query = oracle.gauss(52, hidden)
    got = hip.lm_head_knn(head, vocab, hidden, query, k)
    q8, q8s = oracle.quantize_to_q8(query)
    scores = oracle.q4_0_matvec_blockint(head, q8, q8s, vocab, hidden)
    ref_i, ref_v = oracle.topk_signed(scores, k)
    np.testing.assert_array_equal(got[0], ref_i)
    np.testing.assert_array_equal(got[1].view(np.uint32), ref_v.view(np.uint32))


def test_lm_head_knn_dev_batch(hip):
    """Device form over several queries equals the host form query by query."""
    torch = pytest.importorskip("torch")
    vocab, hidden, nq, k = 5000, 256, 3, 10
    head = oracle.quantize_q4_0(oracle.gauss(53, vocab * hidden, 0.0, 0.02))
    queries = oracle.gauss(54, nq * hidden).reshape(nq, hidden)
    h = hip.register_weight(larql_hip.Q4_0, head, vocab, hidden)
    try:
        dq = torch.from_numpy(queries).cuda()
        di = torch.empty(nq * k, device="cuda", dtype=torch.int32)
        dv = torch.empty(nq * k, device="cuda", dtype=torch.float32)
        hip.lm_head_knn_dev(h, dq, nq, k, di, dv)
        hip.synchronize()
        gi = di.cpu().numpy().view(np.uint32).reshape(nq, k)
        gv = dv.cpu().numpy().reshape(nq, k)
        for i in range(nq):
            ri, rv = hip.lm_head_knn(head, vocab, hidden, queries[i], k)
            np.testing.assert_array_equal(gi[i], ri)
            np.testing.assert_array_equal(gv[i].view(np.uint32), rv.view(np.uint32))
    finally:
        hip.release_weight(h)
