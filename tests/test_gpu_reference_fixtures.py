"""The reference's own fixtures fed straight into the HIP path (the other GPU tests compare
with the oracle, which these fixtures pin; here the fixtures meet the device kernels):

* the f32 gate known answers of larql-vindex/tests/test_vindex.rs:27-60 (the 2-layer,
  3-feature, hidden-4 test index), :134-160 (gate_knn_finds_best_match,
  gate_knn_top_k_ordering) and :2474-2488 (gate_walk_matches_gate_knn);
* the fixture vindex larql-python/tests/fixtures/ui_walk_trace_vindex (f32 gates of 2
  layers x 4 features x hidden 8, its 16 embeddings as queries), copied as data into
  tests/golden/ui_walk_trace_vindex.npz;
* the Q4_K and Q6_K hand blocks of larql-compute/tests/test_metal_shaders.rs:1301-1361,
  whose products have closed forms;
* tests/golden/q4_0_ref.npz: what the reference's compiled x86 kernel
  (larql-compute/csrc/q4_dot.c) returns for LCG inputs of its own tests.

Bars: top-k indices exact; f32 gate scores bit-exact with the oracle's fma chain (and
equal to the exact dot products rounded once to f32, which these sparse inputs give);
K-quant closed forms and the
compiled x86 outputs within 1e-5 relative (different accumulation orders).
"""
import json
import os

import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def known():
    with open(os.path.join(GOLD, "known_answers.json")) as f:
        return json.load(f)


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def test_gate_knn_test_index_known_answers(hip):
    """test_vindex.rs:27-60,134-160,2474-2488 through the HIP gate-KNN (hidden 4)."""
    ka = known()["gate_knn_orthogonal"]
    gates = [np.array(ka["gate0"], np.float32), np.array(ka["gate1"], np.float32)]
    for case in ka["cases"]:
        g = gates[case["layer"]]
        q = np.array(case["query"], np.float32)
        idx, val = hip.gate_knn(g, g.shape[0], g.shape[1], q, case["k"], fmt=larql_hip.F32)
        print(f"[fixtures] test index layer {case['layer']} q={case['query']}: {idx[0].tolist()} {val[0].tolist()}",
              flush=True)
        assert idx.shape == (1, case["k"])
        if "idx" in case:
            assert idx[0].tolist() == case["idx"]
            assert np.all(np.abs(val[0] - np.array(case["score"], np.float32)) < 0.01)
        if "idx_prefix" in case:
            assert idx[0, : len(case["idx_prefix"])].tolist() == case["idx_prefix"]
    # gate_walk_matches_gate_knn: the same features in the same order, scores within 1e-5
    w = ka["walk_case"]
    g = gates[w["layer"]]
    q = np.array(w["query"], np.float32)
    idx, val = hip.gate_knn(g, g.shape[0], g.shape[1], q, w["k"], fmt=larql_hip.F32)
    s = g.astype(np.float64) @ q.astype(np.float64)
    order = np.argsort(-np.abs(s), kind="stable")[: w["k"]]
    assert idx[0].tolist() == order.tolist()
    assert np.all(np.abs(val[0] - s[order]) < 1e-5)
    # both layers in one device call, every one-hot and mixed query, k up to the feature count
    torch = pytest.importorskip("torch")
    hs = [hip.register_weight(larql_hip.F32, g, g.shape[0], g.shape[1]) for g in gates]
    try:
        qs = np.concatenate([np.eye(4, dtype=np.float32), np.array([[0.8, 0.6, 0, 0], [1, 0.5, 0, 0],
                                                                      [0, 0, 1, 1], [-1, 2, -3, 0.5]], np.float32)])
        dq = torch.from_numpy(qs).cuda()
        k = 3
        di = torch.empty(2 * len(qs) * k, device="cuda", dtype=torch.int32)
        dv = torch.empty(2 * len(qs) * k, device="cuda", dtype=torch.float32)
        hip.gate_knn_dev(hs, dq, len(qs), k, di, dv)
        hip.synchronize()
        gi = di.cpu().numpy().view(np.uint32).reshape(2, len(qs), k)
        gv = dv.cpu().numpy().reshape(2, len(qs), k)
        for l, g in enumerate(gates):
            for j, qq in enumerate(qs):
                ri, rv = oracle.topk_abs(oracle.gate_scores_f32(g, qq, 3, 4), k)
                np.testing.assert_array_equal(gi[l, j], ri)
                np.testing.assert_array_equal(gv[l, j].view(np.uint32), rv.view(np.uint32))
                # at most two nonzero products per score, each exact: the chain rounds once
                s = g.astype(np.float64) @ qq.astype(np.float64)
                np.testing.assert_array_equal(gv[l, j], s[ri].astype(np.float32))
    finally:
        for h in hs:
            hip.release_weight(h)


def test_gate_knn_fixture_vindex(hip):
    """The fixture vindex's gate vectors (hidden 8) with its embeddings as queries: every
    layer's top-k (k = 1, 3, all 4 features, and 6 > features, clamped) from one device call
    over both layers equals the oracle's, and the scores equal gate . embedding exactly."""
    torch = pytest.importorskip("torch")
    fv = np.load(os.path.join(GOLD, "ui_walk_trace_vindex.npz"))
    gates, emb = fv["gates"], fv["embeddings"]
    L, F, H = gates.shape
    hs = [hip.register_weight(larql_hip.F32, np.ascontiguousarray(gates[l]), F, H) for l in range(L)]
    try:
        dq = torch.from_numpy(np.ascontiguousarray(emb, dtype=np.float32)).cuda()
        nq = emb.shape[0]
        for k in (1, 3, F, F + 2):
            print(f"[fixtures] ui_walk_trace_vindex: {L} layers x {F} x {H}, {nq} queries, k={k}", flush=True)
            di = torch.empty(L * nq * k, device="cuda", dtype=torch.int32)
            dv = torch.empty(L * nq * k, device="cuda", dtype=torch.float32)
            hip.gate_knn_dev(hs, dq, nq, k, di, dv)
            hip.synchronize()
            gi = di.cpu().numpy().view(np.uint32).reshape(L, nq, k)
            gv = dv.cpu().numpy().reshape(L, nq, k)
            m = min(k, F)
            for l in range(L):
                for j in range(nq):
                    ri, rv = oracle.topk_abs(oracle.gate_scores_f32(gates[l], emb[j], F, H), k)
                    np.testing.assert_array_equal(gi[l, j, :m], ri)
                    np.testing.assert_array_equal(gv[l, j, :m].view(np.uint32), rv.view(np.uint32))
                    s = gates[l].astype(np.float64) @ emb[j].astype(np.float64)   # one nonzero term
                    np.testing.assert_array_equal(gv[l, j, :m], s[ri].astype(np.float32))
                    assert np.all(gi[l, j, m:] == 0xFFFFFFFF)
    finally:
        for h in hs:
            hip.release_weight(h)


def _hand_x(hidden):
    return np.sin(np.arange(hidden, dtype=np.float32) * np.float32(0.01)).astype(np.float32)


def test_q4k_hand_block_closed_form(hip):
    """test_metal_shaders.rs:1301-1331: d = 1.0, scale 0 = 1, every nibble 1, the rest 0, so
    every row is sum(x[0:32])."""
    ka = known()["q4k_hand_block"]
    rows, hidden = 64, 256
    blk = np.zeros((rows, 148), np.uint8)
    blk[:, 0:2] = ka["d_bytes"]
    blk[:, 4] = ka["scale0"]
    blk[:, 20:148] = ka["nibble_byte"]
    x = _hand_x(hidden)
    got = hip.q4k_matvec(blk.reshape(-1), x, rows, hidden)
    ref = np.full(rows, np.sum(x[:32].astype(np.float64)))
    e = rel_err(got, ref)
    print(f"[fixtures] q4k hand block: rel_err={e:.2e}", flush=True)
    assert e <= 1e-5


def test_q6k_hand_block_closed_form(hip):
    """test_metal_shaders.rs:1334-1361: d = 1.0, scale 0 = 1, every low nibble 3, high bits 0,
    so every row is (3 - 32) * sum(x[0:16])."""
    ka = known()["q6k_hand_block"]
    rows, hidden = 64, 256
    blk = np.zeros((rows, 210), np.uint8)
    blk[:, 208:210] = ka["d_bytes"]
    blk[:, 192] = ka["scale0"]
    blk[:, 0:128] = ka["ql_byte"]
    x = _hand_x(hidden)
    got = hip.q6k_matvec(blk.reshape(-1), x, rows, hidden)
    ref = np.full(rows, -29.0 * np.sum(x[:16].astype(np.float64)))
    e = rel_err(got, ref)
    print(f"[fixtures] q6k hand block: rel_err={e:.2e}", flush=True)
    assert e <= 1e-5


def test_q4_0_compiled_reference_outputs(hip):
    """q4_0_ref.npz: q4_matvec and q4_vecmat of the reference's compiled x86 kernel on LCG
    inputs of its own tests; the GPU's block-integer order is within 1e-5 of its
    per-element float order."""
    d = np.load(os.path.join(GOLD, "q4_0_ref.npz"))
    for tag in ("small", "mid"):
        rows, hidden = int(d[f"{tag}_rows"]), int(d[f"{tag}_hidden"])
        got = hip.q4_matvec(d[f"{tag}_q4"], d[f"{tag}_q8"], d[f"{tag}_q8s"], rows, hidden)
        e = rel_err(got, d[f"{tag}_matvec_out"])
        print(f"[fixtures] q4_0 matvec {tag} [{rows}x{hidden}]: rel_err={e:.2e}", flush=True)
        assert e <= 1e-5
    inter, hidden = int(d["vecmat_inter"]), int(d["vecmat_hidden"])
    got = hip.q4_vecmat(d["vecmat_act"], d["vecmat_q4"], inter, hidden)
    e = rel_err(got, d["vecmat_out"])
    print(f"[fixtures] q4_0 vecmat [{inter}x{hidden}]: rel_err={e:.2e}", flush=True)
    assert e <= 1e-5
