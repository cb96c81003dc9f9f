"""Vindex file slicing (larql_hip.vindex) against the reference's layouts: the interleaved
FFN file (LI/src/layer_graph/pipeline_layer.rs:119-133, generate.rs:60-64), the attention
file + manifest (LV/src/index/walk.rs:401-445, pipeline_layer.rs:97-99) and the Q4_0
gate-vector file (walk.rs:303-345).  Host-only: no GPU calls."""
import json

import numpy as np
import pytest

import larql_hip
import oracle
from larql_hip import vindex


def write_vindex(d, mats, attn, manifest_extra=None, gates=None):
    """mats: per layer (gate, up, down) bytes; attn: per layer [(bytes, format)] x 4."""
    (d / "interleaved_q4k.bin").write_bytes(b"".join(m.tobytes() for L in mats for m in L))
    blob, man = b"", []
    for L in attn:
        for data, fmt in L:
            man.append({"key": "w", "shape": [1, 1], "format": fmt, "offset": len(blob), "length": data.nbytes})
            blob += data.tobytes()
    man += manifest_extra or []
    (d / "attn_weights_q4k.bin").write_bytes(blob)
    (d / "attn_weights_q4k_manifest.json").write_text(json.dumps(man))
    if gates is not None:
        (d / "gate_vectors_q4.bin").write_bytes(b"".join(g.tobytes() for g in gates))


def test_ffn_per_matrix_closed_forms():
    # ceil(inter * hidden / 256) * 148 (Q4_K); inter * hidden / 32 * 18 (Q4_0)
    assert vindex.ffn_per_matrix(14336, 4096) == 14336 * 4096 // 256 * 148
    assert vindex.ffn_per_matrix(10, 100) == 4 * 148  # 1000 elements -> 4 super-blocks
    assert vindex.ffn_per_matrix(14336, 4096, q4k=False) == 14336 * 4096 // 32 * 18


def test_manifest_defaults_and_formats():
    m = vindex.parse_attn_manifest([{"offset": 5, "length": 7, "format": "Q6_K"}, {"length": 3}, {}])
    assert m == [(5, 7, "Q6_K"), (0, 3, "Q4_K"), (0, 0, "Q4_K")]
    assert vindex.attn_format("Q6_K") == larql_hip.Q6_K
    for s in ("Q4_K", "Q8_0", ""):  # every other string is Q4_K
        assert vindex.attn_format(s) == larql_hip.Q4_K


def test_vindex_slices_match_the_written_matrices(tmp_path):
    n_layers, hidden, inter, hd, nq, nkv = 3, 256, 512, 64, 4, 2
    mats, attn, norms = [], [], []
    for l in range(n_layers):
        mats.append([oracle.quantize_q4_k(oracle.gauss(10 * l + i, r * c, 0.0, 0.02))
                     for i, (r, c) in enumerate([(inter, hidden), (inter, hidden), (hidden, inter)])])
        shapes = [(nq * hd, hidden, "Q4_K"), (nkv * hd, hidden, "Q4_K"), (nkv * hd, hidden, "Q6_K"),
                  (hidden, nq * hd, "Q4_K")]
        attn.append([((oracle.quantize_q6_k if f == "Q6_K" else oracle.quantize_q4_k)(
            oracle.gauss(500 + 10 * l + i, r * c, 0.0, 0.02)), f) for i, (r, c, f) in enumerate(shapes)])
        norms.append((np.ones(hidden, np.float32), np.ones(hidden, np.float32)))
    feats = [64, 0, 32]
    gates = [oracle.quantize_q4_0(oracle.gauss(900 + l, nf * hidden)) for l, nf in enumerate(feats)]
    write_vindex(tmp_path, mats, attn, manifest_extra=[{"offset": 0, "length": 4}], gates=gates)

    v = vindex.Vindex(str(tmp_path), n_layers, hidden, inter)
    assert v.ffn_format == larql_hip.Q4_K and v.per_matrix == mats[0][0].nbytes
    for l in range(n_layers):
        for got, ref in zip(v.ffn_weights(l), mats[l]):
            assert np.array_equal(got, ref)
        for (got, fmt), (ref, rfmt) in zip(v.attn_q4k_layer_data(l), attn[l]):
            assert fmt == rfmt and np.array_equal(got, ref)
    # one stray entry after the last layer: not a fourth layer (base + 3 >= len)
    assert v.attn_q4k_layer_data(n_layers) is None
    with pytest.raises(IndexError):
        v.ffn_weights(n_layers)
    assert np.array_equal(v.gate_q4(0, feats), gates[0])
    assert v.gate_q4(1, feats) is None  # no features: no data
    assert np.array_equal(v.gate_q4(2, feats), gates[2])
    assert v.gate_q4(3, feats) is None

    layers = v.pipeline_layers(norms, head_dim=hd, num_q_heads=nq, num_kv_heads=nkv, rope_base=10000.0)
    L = layers[1]
    q, k, vv, o = v.attn_q4k_layer_data(1)
    assert (L.wq.data, L.wq.len, L.wq.format) == (q[0].ctypes.data, q[0].nbytes, larql_hip.Q4_K)
    assert (L.wv.data, L.wv.format) == (vv[0].ctypes.data, larql_hip.Q6_K)
    gate, up, down = v.ffn_weights(1)
    assert (L.down.data, L.down.len, L.down.format) == (down.ctypes.data, down.nbytes, larql_hip.Q4_K)
    assert L.num_q_heads == nq and L.num_kv_heads == nkv and L.head_dim == hd


def test_attention_entry_past_the_file_is_an_error(tmp_path):
    write_vindex(tmp_path, [[np.zeros(148, np.uint8)] * 3], [[(np.zeros(148, np.uint8), "Q4_K")] * 4])
    v = vindex.Vindex(str(tmp_path), 1, 256, 1)
    v.manifest[2] = (500, 200, "Q4_K")  # ends at 700 > 4 x 148
    with pytest.raises(IndexError):
        v.attn_q4k_layer_data(0)
