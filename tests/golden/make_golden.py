"""Writes the golden fixtures under tests/golden/.

  known_answers.json  Known-answer data copied (as data) from the reference's own
                      unit tests, each entry citing its source file:line.
  ui_walk_trace_vindex.npz
                      The f32 gate vectors [2 layers][4 features][hidden 8] and the
                      embeddings [16][8] of the reference's fixture vindex
                      (larql-python/tests/fixtures/ui_walk_trace_vindex/, gate_vectors.bin
                      and embeddings.bin as index.json lays them out), copied as data.
  q4_0_ref.npz        Inputs and outputs of the reference's own C kernel
                      (larql-compute/csrc/q4_dot.c, x86 scalar path), compiled in
                      place by oracle/Makefile into oracle/_ref/libq4dot_ref.so.
                      Inputs use the reference tests' LCG generator
                      (LC/tests/test_q4_x86_correctness.rs:73-80) and the oracle's
                      Q4_0/Q8 quantizers; outputs are what q4_0_matvec_c and
                      q4_0_vecmat_c return for those bytes.

Run from the repo root after `make -C oracle`:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def lcg_synth(n: int, seed: int, inc: int = 1442695040888963407) -> np.ndarray:
    """LC/tests/test_q4_x86_correctness.rs:73-80 (inc=1 in test_metal_shaders.rs:18-24)."""
    out = np.empty(n, dtype=np.float32)
    s = seed & 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        s = (s * 6364136223846793005 + inc) & 0xFFFFFFFFFFFFFFFF
        out[i] = np.float32(np.float32(s >> 33) / np.float32(4294967295.0) * np.float32(2.0) - np.float32(1.0))
    return out


KNOWN = {
    "f16": {
        "source": "larql-models/src/quant/ggml.rs:388-473 (scales 0x3C00=1.0, 0x4000=2.0, 0x3800=0.5, 0x0000=0)",
        "pairs": [[0x3C00, 1.0], [0x4000, 2.0], [0x3800, 0.5], [0x0000, 0.0], [0x8000, -0.0],
                  [0xBC00, -1.0], [0x7BFF, 65504.0], [0x0001, 5.960464477539063e-08], [0x03FF, 6.097555160522461e-05]],
    },
    "q4_0_basic": {
        "source": "larql-models/src/quant/ggml.rs:388-397",
        "block": [0x00, 0x3C] + [0x12] * 16,
        "expect": {"0": -6.0, "1": -7.0},
    },
    "q4_0_zero_scale": {
        "source": "larql-models/src/quant/ggml.rs:400-406",
        "block": [0x00, 0x00] + [0xFF] * 16,
        "expect_all": 0.0,
    },
    "q4_0_two_blocks": {
        "source": "larql-models/src/quant/ggml.rs:408-418",
        "blocks": [0x00, 0x3C] + [0x88] * 16 + [0x00, 0x40] + [0x19] * 16,
        "expect": {"0": 0.0, "32": 2.0, "33": -14.0},
    },
    "q4_0_zero_input": {
        "source": "larql-compute/src/cpu/ops/q4_common.rs:557-569",
        "scale_bytes": [0, 0],
        "nibble_byte": 0x88,
    },
    "q4_0_sizes": {
        "source": "larql-compute/src/cpu/ops/q4_common.rs:545-555",
        "cases": [[64, 36], [256, 144]],
    },
    "q8_zero_input": {
        "source": "larql-compute/src/cpu/ops/q4_common.rs:535-541",
        "n": 32,
    },
    "q4k_hand_block": {
        "source": "larql-compute/tests/test_metal_shaders.rs:1301-1331",
        "d_bytes": [0x00, 0x3C], "scale0": 1, "nibble_byte": 0x11,
        "expect": "out[r] = sum(x[0:32]) for every row (sc0 = 1, q = 1; other sub-blocks have sc = 0)",
    },
    "q6k_hand_block": {
        "source": "larql-compute/tests/test_metal_shaders.rs:1334-1361",
        "d_bytes": [0x00, 0x3C], "scale0": 1, "ql_byte": 0x33,
        "expect": "out[r] = -29 * sum(x[0:16]) (q = 3 + 16*0 - 32; other sub-blocks have sc = 0)",
    },
    "gate_knn_orthogonal": {
        "source": "larql-vindex/tests/test_vindex.rs:27-60,134-160",
        "gate0": [[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 0]],
        "gate1": [[0, 0, 0, 1], [0.5, 0.5, 0, 0], [0, 0, -1, 0]],
        "cases": [
            {"layer": 0, "query": [1, 0, 0, 0], "k": 1, "idx": [0], "score": [1.0]},
            {"layer": 0, "query": [0.8, 0.6, 0, 0], "k": 3, "idx_prefix": [0, 1]},
        ],
        # gate_walk_matches_gate_knn (test_vindex.rs:2474-2488): the same features in the
        # same order as gate_knn, scores within 1e-5
        "walk_case": {"source": "larql-vindex/tests/test_vindex.rs:2474-2488", "layer": 0,
                      "query": [1.0, 0.5, 0.0, 0.0], "k": 3},
    },
}

FIXTURE_VINDEX = "/root/reference/larql-main/crates/larql-python/tests/fixtures/ui_walk_trace_vindex"


def fixture_vindex():
    """The fixture vindex's gate vectors and embeddings (f32 files laid out by index.json:
    layer l's gates at its byte offset, num_features x hidden_size; embeddings vocab x
    hidden), or None when the reference tree is absent."""
    if not os.path.isdir(FIXTURE_VINDEX):
        return None
    with open(os.path.join(FIXTURE_VINDEX, "index.json")) as f:
        idx = json.load(f)
    hidden, vocab = idx["hidden_size"], idx["vocab_size"]
    raw = np.fromfile(os.path.join(FIXTURE_VINDEX, "gate_vectors.bin"), dtype=np.float32)
    gates = np.stack([raw[L["offset"] // 4: (L["offset"] + L["length"]) // 4].reshape(L["num_features"], hidden)
                      for L in idx["layers"]])
    emb = np.fromfile(os.path.join(FIXTURE_VINDEX, "embeddings.bin"), dtype=np.float32).reshape(vocab, hidden)
    return {"gates": gates, "embeddings": emb, "hidden": np.int64(hidden)}


def main():
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(KNOWN, f, indent=1)
    fv = fixture_vindex()
    if fv is not None:
        np.savez_compressed(os.path.join(HERE, "ui_walk_trace_vindex.npz"), **fv)

    if oracle.ref_lib() is None:
        print("oracle/_ref/libq4dot_ref.so not built; skipping q4_0_ref.npz")
        return
    data = {}
    # test_q4_x86_correctness.rs:82-114 shape (rows 4, hidden 64) and a larger one.
    for tag, rows, hidden, sw, sx in (("small", 4, 64, 0xC0FFEE, 0xBEEF), ("mid", 96, 512, 0x1234, 0x5678)):
        w = lcg_synth(rows * hidden, sw)
        x = lcg_synth(hidden, sx)
        q4 = oracle.quantize_q4_0(w)
        q8, s8 = oracle.quantize_to_q8(x)
        out = oracle.ref_q4_0_matvec(q4, q8, s8, rows, hidden)
        data[f"{tag}_rows"] = np.int64(rows)
        data[f"{tag}_hidden"] = np.int64(hidden)
        if tag == "small":
            data[f"{tag}_w"] = w
        data[f"{tag}_x"] = x
        data[f"{tag}_q4"] = q4
        data[f"{tag}_q8"] = q8
        data[f"{tag}_q8s"] = s8
        data[f"{tag}_matvec_out"] = out
    # vecmat, test_q4_x86_correctness.rs:116-143 shape (intermediate 8, hidden 64)
    inter, hidden = 8, 64
    act = lcg_synth(inter, 0xDEADBEEF)
    w = lcg_synth(inter * hidden, 0xFEEDFACE)
    q4 = oracle.quantize_q4_0(w)
    data["vecmat_inter"] = np.int64(inter)
    data["vecmat_hidden"] = np.int64(hidden)
    data["vecmat_act"] = act
    data["vecmat_q4"] = q4
    data["vecmat_out"] = oracle.ref_q4_0_vecmat(act, q4, inter, hidden)
    np.savez_compressed(os.path.join(HERE, "q4_0_ref.npz"), **data)
    print("wrote known_answers.json and q4_0_ref.npz")


if __name__ == "__main__":
    main()
