"""Synthetic Llama-style decoder on the device, for benchmarks and tests.

Weights are drawn N(0, std) with torch's device RNG and quantized on the device by
the library's ports of the reference quantizers (148-byte Q4_K projections, 210-byte
Q6_K output head); norms are 1.0; the fp16 KV cache is prefilled with N(0, 1) rows.
No checkpoint or dataset is involved.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import Q4_K, Q6_K, HipBackend, make_layer

LLAMA3_8B = dict(n_layers=32, hidden=4096, inter=14336, nq=32, nkv=8, hd=128, vocab=128256, rope=500000.0)


@dataclass
class SynthModel:
    model: object                 # larql_hip.DeviceModel
    x: object                     # device f32 [hidden]: embedding row of `token`
    logits: object                # device f32 [vocab]
    hidden_out: object            # device f32 [hidden]
    cfg: dict
    kv_len: int
    host: dict = field(default_factory=dict)   # reference-layout bytes etc. when keep_host
    keep: list = field(default_factory=list)   # device buffers the model's structs point at


def _quantized(be: HipBackend, torch, gen, rows, cols, fmt, std):
    dev = gen.device
    w = torch.randn(rows, cols, generator=gen, device=dev, dtype=torch.float32) * std
    per, nbytes = (256, 148) if fmt == Q4_K else (256, 210)
    raw = torch.empty(rows * cols // per * nbytes, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    be.quantize_weights_dev(fmt, w, rows * cols, raw)
    be.synchronize()
    del w
    return raw


def build_llama(be: HipBackend, torch, *, n_layers=32, hidden=4096, inter=14336, nq=32, nkv=8, hd=128,
                vocab=128256, rope=500000.0, kv_len=2048, token=1, std=0.02, seed=0, keep_host=False,
                log=None, q6k=()) -> SynthModel:
    """q6k: projection names quantized to Q6_K instead of Q4_K (("wv", "down") is the
    Q4_K_M mix of llama.cpp files: attention V and FFN down in Q6_K)."""
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    qd, kvd = nq * hd, nkv * hd
    cfg = dict(n_layers=n_layers, hidden=hidden, inter=inter, nq=nq, nkv=nkv, hd=hd, vocab=vocab, rope=rope)
    ones = torch.ones(hidden, device=dev, dtype=torch.float32)
    host = {"layers": []} if keep_host else {}
    structs, raws_all = [], []
    shapes = (("wq", qd, hidden), ("wk", kvd, hidden), ("wv", kvd, hidden), ("wo", hidden, qd),
              ("gate", inter, hidden), ("up", inter, hidden), ("down", hidden, inter))
    for l in range(n_layers):
        raws = {}
        for i, (name, rows, cols) in enumerate(shapes):
            gen.manual_seed(seed * 1_000_003 + l * 16 + i)
            raws[name] = _quantized(be, torch, gen, rows, cols, Q6_K if name in q6k else Q4_K, std)
        structs.append(make_layer(raws["wq"], raws["wk"], raws["wv"], raws["wo"], raws["gate"], raws["up"],
                                  raws["down"], ones, ones, head_dim=hd, num_q_heads=nq, num_kv_heads=nkv,
                                  rope_base=rope, formats={n: Q6_K for n in q6k}))
        raws_all.append(raws)
        if keep_host:
            host["layers"].append({k: v.cpu().numpy() for k, v in raws.items()})
        if log and (l + 1) % 8 == 0:
            log(f"[synth] quantized {l + 1}/{n_layers} layers")
    model = be.model(structs, hidden, inter, weights_on_device=True)
    torch.cuda.synchronize()
    del raws_all, structs            # the model holds its own repacked copies
    gen.manual_seed(seed * 1_000_003 + 9999)
    head = _quantized(be, torch, gen, vocab, hidden, Q6_K, std)
    model.set_head(head, vocab, ones, eps=1e-6, fmt=Q6_K, on_device=True)
    if keep_host:
        host["head"] = head.cpu().numpy()
    del head
    gen.manual_seed(seed * 1_000_003 + 7777)
    embed = torch.randn(vocab, hidden, generator=gen, device=dev, dtype=torch.float32) * std
    x = embed[token].clone()
    del embed
    be.reset_kv_cache()
    for l in range(n_layers):
        gen.manual_seed(seed * 1_000_003 + 100_000 + l)
        k = torch.randn(kv_len, kvd, generator=gen, device=dev, dtype=torch.float32).half()
        v = torch.randn(kv_len, kvd, generator=gen, device=dev, dtype=torch.float32).half()
        torch.cuda.synchronize()
        be.populate_kv_layer_f16_dev(l, k, v, kv_len, nkv, hd)
        if keep_host:
            kc = np.zeros((kv_len + 1) * kvd, np.uint16)
            vc = np.zeros((kv_len + 1) * kvd, np.uint16)
            kc[: kv_len * kvd] = k.cpu().numpy().view(np.uint16).reshape(-1)
            vc[: kv_len * kvd] = v.cpu().numpy().view(np.uint16).reshape(-1)
            host["layers"][l]["k_cache"] = kc
            host["layers"][l]["v_cache"] = vc
    if keep_host:
        host["x"] = x.cpu().numpy()
        host["cfg"] = cfg
        host["kv_len"] = kv_len
    logits = torch.empty(vocab, device=dev, dtype=torch.float32)
    hidden_out = torch.empty(hidden, device=dev, dtype=torch.float32)
    torch.cuda.synchronize()
    return SynthModel(model=model, x=x, logits=logits, hidden_out=hidden_out, cfg=cfg, kv_len=kv_len, host=host,
                      keep=[ones])
