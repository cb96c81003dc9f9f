"""The vindex files that feed the decode/prefill path, as zero-copy host views.

The reference hands the GPU backend byte slices of memory-mapped vindex files; this module
opens the same files with numpy.memmap and slices them the same way, so the slices go to
`make_layer` / `HipBackend.prefill_q4` / `decode_token` (and `HipBackend.model`, which
copies them to the device once) without an intermediate copy:

  * interleaved_q4k.bin (or interleaved_q4.bin): per layer [gate | up | down], each
    `per_matrix` bytes (LI/src/layer_graph/pipeline_layer.rs:119-133); per_matrix is
    ceil(inter * hidden / 256) * 148 for Q4_K, inter * hidden / 32 * 18 for Q4_0
    (LI/src/layer_graph/generate.rs:60-64);
  * attn_weights_q4k.bin + attn_weights_q4k_manifest.json: a JSON list of
    {offset, length, format} entries, four per layer in the order Q, K, V, O; a missing
    offset or length reads as 0 and a missing format as "Q4_K"; "Q6_K" selects Q6_K and
    any other string Q4_K (LV/src/index/walk.rs:401-445, pipeline_layer.rs:97-99);
  * gate_vectors_q4.bin: layers back to back, layer l = [num_features(l) x hidden] Q4_0,
    18 bytes per 32 elements; a layer with no features has no data
    (LV/src/index/walk.rs:303-345).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import numpy as np

from . import Q4_0, Q4_K, Q6_K, make_layer


def ffn_per_matrix(inter: int, hidden: int, q4k: bool = True) -> int:
    """Bytes of one FFN matrix in the interleaved file (generate.rs:60-64)."""
    return -(-(inter * hidden) // 256) * 148 if q4k else inter * hidden // 32 * 18


def attn_format(name: str) -> int:
    """Manifest format string -> weight format (pipeline_layer.rs:97-99)."""
    return Q6_K if name == "Q6_K" else Q4_K


def _map(path: str) -> np.ndarray:
    if os.path.getsize(path) == 0:
        return np.zeros(0, np.uint8)
    return np.memmap(path, dtype=np.uint8, mode="r")


def resolve_ffn_weights(ffn: np.ndarray, layer: int, per_matrix: int):
    """(gate, up, down) byte views of one layer (pipeline_layer.rs:119-133)."""
    fs = layer * 3 * per_matrix
    if fs + 3 * per_matrix > len(ffn):
        raise IndexError(f"layer {layer}: interleaved FFN file holds {len(ffn)} bytes, needs {fs + 3 * per_matrix}")
    return ffn[fs:fs + per_matrix], ffn[fs + per_matrix:fs + 2 * per_matrix], ffn[fs + 2 * per_matrix:fs + 3 * per_matrix]


def parse_attn_manifest(entries) -> list[tuple[int, int, str]]:
    """The manifest's (offset, length, format) per entry (walk.rs:417-425)."""
    out = []
    for e in entries:
        out.append((int(e.get("offset", 0) or 0), int(e.get("length", 0) or 0), str(e.get("format", "Q4_K"))))
    return out


def attn_layer_data(attn: np.ndarray, manifest: list[tuple[int, int, str]], layer: int):
    """[(bytes, format string)] for Q, K, V, O of `layer`, or None when the manifest has no
    four entries for it (walk.rs:433-445)."""
    base = layer * 4
    if base + 3 >= len(manifest):
        return None
    out = []
    for off, length, fmt in manifest[base:base + 4]:
        if off + length > len(attn):
            raise IndexError(f"manifest entry [{off}, {off + length}) past the {len(attn)}-byte attention file")
        out.append((attn[off:off + length], fmt))
    return out


@dataclass
class GateQ4Slice:
    byte_offset: int
    byte_len: int
    num_features: int


def gate_q4_slices(num_features: list[int], hidden: int) -> list[GateQ4Slice]:
    """Per-layer slices of gate_vectors_q4.bin (walk.rs:313-325)."""
    slices, off = [], 0
    for nf in num_features:
        n = nf * hidden // 32 * 18
        slices.append(GateQ4Slice(off, n, nf))
        off += n
    return slices


def gate_q4_data(gates: np.ndarray, slices: list[GateQ4Slice], layer: int):
    """Q4_0 bytes of one layer's gate vectors, or None (walk.rs:336-343)."""
    if layer >= len(slices):
        return None
    s = slices[layer]
    if s.byte_len == 0 or s.byte_offset + s.byte_len > len(gates):
        return None
    return gates[s.byte_offset:s.byte_offset + s.byte_len]


class Vindex:
    """The weight files of one vindex directory, memory-mapped.  Keep the object alive while
    layers built from it are in use (they point into its maps)."""

    def __init__(self, path: str, num_layers: int, hidden: int, inter: int):
        self.path, self.num_layers, self.hidden, self.inter = path, num_layers, hidden, inter
        q4k = os.path.exists(os.path.join(path, "interleaved_q4k.bin"))
        self.ffn_format = Q4_K if q4k else Q4_0
        self.ffn = _map(os.path.join(path, "interleaved_q4k.bin" if q4k else "interleaved_q4.bin"))
        self.per_matrix = ffn_per_matrix(inter, hidden, q4k)
        self.attn = _map(os.path.join(path, "attn_weights_q4k.bin"))
        man = os.path.join(path, "attn_weights_q4k_manifest.json")
        self.manifest = None
        if os.path.exists(man):
            with open(man) as f:
                self.manifest = parse_attn_manifest(json.load(f))
        self.gates = None
        gp = os.path.join(path, "gate_vectors_q4.bin")
        if os.path.exists(gp):
            self.gates = _map(gp)

    def attn_q4k_layer_data(self, layer: int):
        return None if self.manifest is None else attn_layer_data(self.attn, self.manifest, layer)

    def ffn_weights(self, layer: int):
        return resolve_ffn_weights(self.ffn, layer, self.per_matrix)

    def gate_q4(self, layer: int, num_features: list[int]):
        if self.gates is None:
            return None
        return gate_q4_data(self.gates, gate_q4_slices(num_features, self.hidden), layer)

    def pipeline_layers(self, norms, *, head_dim: int, num_q_heads: int, num_kv_heads: int, rope_base: float,
                        eps: float = 1e-6, sliding_window: int = 0):
        """FullPipelineLayers for every layer (pipeline_layer.rs:138-152); `norms` holds one
        (input_norm, post_attn_norm) pair of f32 arrays per layer."""
        layers = []
        for l in range(self.num_layers):
            attn = self.attn_q4k_layer_data(l)
            if attn is None:
                raise ValueError(f"no attention weights for layer {l}")
            gate, up, down = self.ffn_weights(l)
            fm = {n: attn_format(f) for n, (_, f) in zip(("wq", "wk", "wv", "wo"), attn)}
            fm.update(gate=self.ffn_format, up=self.ffn_format, down=self.ffn_format)
            layers.append(make_layer(attn[0][0], attn[1][0], attn[2][0], attn[3][0], gate, up, down, norms[l][0],
                                     norms[l][1], head_dim=head_dim, num_q_heads=num_q_heads,
                                     num_kv_heads=num_kv_heads, rope_base=rope_base, eps=eps, formats=fm,
                                     sliding_window=sliding_window))
        return layers
