"""Writes small PolarEngine checkpoints for the loader tests.

The layers are quantized with the oracle's quantizer and stored in the
on-disk layouts the reference's loader reads (loader.py:300-445): split
tensors (int8 codes, nibble codes, Q5-packed codes with ``packed_q5``,
``.ct`` instead of ``.ct_scaled``), a bias, plain fp32 tensors, two shards
with an index, and a separate ``hlwq-q5`` checkpoint. Returns what was
written so the tests can compare."""

from __future__ import annotations

import json
import os
from typing import Dict

import numpy as np
import torch
from safetensors.torch import save_file

import polar_oracle as O

BS = 128


def _layer(seed: int, out_f: int, in_f: int, bits: int) -> Dict[str, np.ndarray]:
    w = O.seeded_normal((out_f, in_f), 0.02, seed).astype(np.float32)
    q = O.quantize_tensor(w, bits)
    q["weight"] = w
    return q


def write_split_checkpoint(root: str) -> Dict[str, dict]:
    """polar_engine_v4 checkpoint in two shards; returns {layer: info}."""
    layers = {
        # name: (seed, out_f, in_f, bits, storage)
        "model.layers.0.self_attn.q_proj": (1, 64, 256, 5, "q5"),
        "model.layers.0.self_attn.k_proj": (2, 32, 256, 5, "int8_ct"),
        "model.layers.0.self_attn.v_proj": (3, 32, 256, 5, "int8"),
        "model.layers.0.self_attn.o_proj": (4, 48, 200, 6, "int8_pattern"),
        "model.layers.0.mlp.gate_proj": (5, 96, 256, 3, "nibble"),
        "model.layers.0.mlp.up_proj": (6, 96, 256, 3, "nibble"),
        "model.layers.0.mlp.down_proj": (7, 40, 384, 4, "nibble_bias"),
    }
    shard_a: Dict[str, torch.Tensor] = {}
    shard_b: Dict[str, torch.Tensor] = {}
    meta_layers: Dict[str, dict] = {}
    info: Dict[str, dict] = {}
    for i, (name, (seed, out_f, in_f, bits, kind)) in enumerate(layers.items()):
        q = _layer(seed, out_f, in_f, bits)
        kp = q["codes"].shape[1]
        dst = shard_a if i % 2 == 0 else shard_b
        meta = {"in_features": in_f, "out_features": out_f, "in_f_padded": kp,
                "n_blocks": kp // BS, "block_size": BS}
        if kind != "int8_pattern":
            meta["bits"] = bits
        if kind == "q5":
            dst[name + ".codes"] = torch.from_numpy(O.pack_q5(q["codes"]))
            meta["packed_q5"] = True
        elif kind.startswith("nibble"):
            dst[name + ".codes"] = torch.from_numpy(O.pack_nibble(q["codes"]))
        else:
            dst[name + ".codes"] = torch.from_numpy(q["codes"])
        dst[name + ".norms"] = torch.from_numpy(q["norms"])
        if kind == "int8_ct":
            dst[name + ".ct"] = torch.from_numpy(O.get_centroids(bits).astype(np.float32))
        else:
            dst[name + ".ct_scaled"] = torch.from_numpy(q["ct_scaled"])
        if kind == "nibble_bias":
            b = O.seeded_normal((out_f,), 0.1, seed + 100)
            dst[name + ".bias"] = torch.from_numpy(b)
            q["bias"] = b
        meta_layers[name] = meta
        info[name] = dict(q, bits=bits, kind=kind, in_f=in_f, out_f=out_f)
    shard_b["model.norm.weight"] = torch.from_numpy(np.linspace(0.5, 1.5, 256).astype(np.float32))
    shard_a["lm_head"] = torch.from_numpy(O.seeded_normal((16, 256), 0.02, 99).astype(np.float32))
    save_file(shard_a, os.path.join(root, "model-00001-of-00002.safetensors"))
    save_file(shard_b, os.path.join(root, "model-00002-of-00002.safetensors"))
    index = {"metadata": {}, "weight_map": {}}
    for k in shard_a:
        index["weight_map"][k] = "model-00001-of-00002.safetensors"
    for k in shard_b:
        index["weight_map"][k] = "model-00002-of-00002.safetensors"
    with open(os.path.join(root, "model.safetensors.index.json"), "w") as f:
        json.dump(index, f)
    cfg = {"format": "polar_engine_v4", "base_model": "synthetic", "block_size": BS,
           "bit_assignment": {"q_proj": 5, "k_proj": 5, "v_proj": 5, "o_proj": 6,
                              "gate_proj": 3, "up_proj": 3, "down_proj": 4},
           "layers": meta_layers}
    with open(os.path.join(root, "polar_config.json"), "w") as f:
        json.dump(cfg, f)
    with open(os.path.join(root, "config.json"), "w") as f:
        json.dump({"model_type": "synthetic", "hidden_size": 256}, f)
    return info


def write_hlwq_checkpoint(root: str) -> Dict[str, dict]:
    """hlwq-q5 checkpoint, one shard, no index; K not a multiple of 8 codes
    per matrix is avoided by the block size, total_codes = out_f * Kp."""
    info: Dict[str, dict] = {}
    tensors: Dict[str, torch.Tensor] = {}
    for name, (seed, out_f, in_f) in {"model.layers.0.mlp.up_proj": (11, 24, 384),
                                      "model.layers.0.self_attn.q_proj": (12, 40, 250)}.items():
        q = _layer(seed, out_f, in_f, 5)
        kp = q["codes"].shape[1]
        flat = q["codes"].reshape(-1)
        tensors[name + ".weight__packed"] = torch.from_numpy(O.pack_q5_hlwq(flat))
        tensors[name + ".weight__norms"] = torch.from_numpy(q["norms"])
        tensors[name + ".weight__meta"] = torch.tensor([out_f, kp // BS, BS, flat.size, in_f],
                                                       dtype=torch.int64)
        info[name] = dict(q, bits=5, in_f=in_f, out_f=out_f)
    save_file(tensors, os.path.join(root, "model.safetensors"))
    with open(os.path.join(root, "polar_config.json"), "w") as f:
        json.dump({"format": "hlwq-q5", "block_size": BS, "layers": {}}, f)
    return info
