"""larql_hip_lm_head_knn_dev_noalloc — no counterpart in the reference; for callers that
cannot allocate device memory.  Through the C ABI it gives larql_hip_lm_head_knn_dev's
indices and scores bit for bit on two calls in a row (the second with a smaller head and
fewer queries), and rejects a request beyond its fixed device array with an error."""
import numpy as np
import pytest

import larql_hip
import oracle

pytestmark = pytest.mark.gpu


def _both(hip, torch, handle, queries, k):
    nq = queries.shape[0]
    dq = torch.from_numpy(np.ascontiguousarray(queries, dtype=np.float32)).cuda()
    outs = []
    for fn in (hip.lm_head_knn_dev, hip.lm_head_knn_dev_noalloc):
        di = torch.full((nq * k,), -7, device="cuda", dtype=torch.int32)
        dv = torch.full((nq * k,), 7.0, device="cuda", dtype=torch.float32)
        fn(handle, dq, nq, k, di, dv)
        hip.synchronize()
        outs.append((di.cpu().numpy().view(np.uint32).reshape(nq, k), dv.cpu().numpy().reshape(nq, k)))
    return outs


def test_lm_head_knn_noalloc_matches_allocating_entry_point(hip):
    torch = pytest.importorskip("torch")
    cases = [(128256, 1024, 4, 40, 71), (10007, 256, 2, 5, 72)]   # second call: smaller head, fewer queries
    for vocab, hidden, nq, k, seed in cases:
        print(f"[noalloc] vocab={vocab} hidden={hidden} nq={nq} k={k}", flush=True)
        head = oracle.quantize_q4_0(oracle.gauss(seed, vocab * hidden, 0.0, 0.02))
        queries = oracle.gauss(seed + 100, nq * hidden).reshape(nq, hidden)
        h = hip.register_weight(larql_hip.Q4_0, head, vocab, hidden)
        try:
            (ri, rv), (gi, gv) = _both(hip, torch, h, queries, k)
            np.testing.assert_array_equal(gi, ri)
            np.testing.assert_array_equal(gv.view(np.uint32), rv.view(np.uint32))
            # and the reference selection on the oracle's scores, query 0
            q8, q8s = oracle.quantize_to_q8(queries[0])
            oi, ov = oracle.topk_signed(oracle.q4_0_matvec_blockint(head, q8, q8s, vocab, hidden), k)
            np.testing.assert_array_equal(gi[0], oi)
        finally:
            hip.release_weight(h)


def test_lm_head_knn_noalloc_rejects_oversized_requests():
    torch = pytest.importorskip("torch")
    be = larql_hip.HipBackend(0, strict=False)
    try:
        vocab, hidden = 128256, 1024
        head = np.zeros(vocab * hidden // 32 * 18, np.uint8)
        h = be.register_weight(larql_hip.Q4_0, head, vocab, hidden)
        nq = 17   # 17 * (513024 + 1152) bytes > 8 MiB
        dq = torch.zeros(nq * hidden, device="cuda", dtype=torch.float32)
        di = torch.zeros(nq * 4, device="cuda", dtype=torch.int32)
        dv = torch.zeros(nq * 4, device="cuda", dtype=torch.float32)
        with pytest.raises(larql_hip.LarqlHipError, match="fixed scratch"):
            be.lm_head_knn_dev_noalloc(h, dq, nq, 4, di, dv)
        be.release_weight(h)
    finally:
        be.close()


def test_lm_head_knn_noalloc_first_call_is_captured_without_allocating():
    """On a fresh context the allocation-free entry point runs before any allocating KNN
    call, and inside a stream capture, where a device allocation or synchronisation would
    fail the capture.  The captured graph, replayed three times with eager work and
    synchronisations between the replays, gives the allocating entry point's indices and
    scores bit for bit (that one runs after the capture, so nothing it allocates can have
    served the captured call)."""
    torch = pytest.importorskip("torch")
    be = larql_hip.HipBackend(0, strict=True)
    try:
        vocab, hidden, nq, k = 32768, 512, 2, 16
        head = oracle.quantize_q4_0(oracle.gauss(81, vocab * hidden, 0.0, 0.02))
        h = be.register_weight(larql_hip.Q4_0, head, vocab, hidden)
        queries = oracle.gauss(82, nq * hidden).reshape(nq, hidden)
        dq = torch.from_numpy(np.ascontiguousarray(queries, dtype=np.float32)).cuda()
        gi = torch.full((nq * k,), -7, device="cuda", dtype=torch.int32)
        gv = torch.full((nq * k,), 7.0, device="cuda", dtype=torch.float32)
        side = torch.cuda.Stream()
        torch.cuda.synchronize()
        print(f"[noalloc] capture: vocab={vocab} hidden={hidden} nq={nq} k={k}", flush=True)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            be.lm_head_knn_dev_noalloc(h, dq, nq, k, gi, gv, stream=side)
        ri = torch.empty_like(gi)
        rv = torch.empty_like(gv)
        be.lm_head_knn_dev(h, dq, nq, k, ri, rv)
        be.synchronize()
        ref_i, ref_v = ri.cpu().numpy(), rv.cpu().numpy()
        for rep in range(3):
            gi.fill_(-7)
            gv.fill_(7.0)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            np.testing.assert_array_equal(gi.cpu().numpy(), ref_i)
            np.testing.assert_array_equal(gv.cpu().numpy().view(np.uint32), ref_v.view(np.uint32))
        del graph
        be.release_weight(h)
    finally:
        be.close()
