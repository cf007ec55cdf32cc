"""Write golden input/output vectors of the reference's KV-cache quantizer.

Run in the build container only (the reference tree is absent on the GPU box):

    python tests/golden/make_golden_kv.py /path/to/reference

It loads ``polarengine_vllm/kv_cache/config.py`` and ``cache.py`` by path
(no package ``__init__``, no Triton), runs their CPU functions and saves plain
arrays to ``golden_kv.npz`` beside this script:

* ``get_centroids(b)`` for b = 2, 3, 4 -- the KV codebook (finite +-4 ends,
  float32 round trips each iteration), which no closed form pins bit-exactly;
* ``BitPacker.pack`` on a seeded code array for b = 2, 3, 4;
* ``PolarKVQuantizer(D, b, "cpu").quantize`` (packed codes, bf16 norms) and
  ``dequantize`` (bf16 output) on a seeded input, D = 64 and 128.
"""

from __future__ import annotations

import importlib.util
import os
import sys
import types

import numpy as np
import torch


def _load(modname: str, path: str):
    spec = importlib.util.spec_from_file_location(modname, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[modname] = mod
    spec.loader.exec_module(mod)
    return mod


def main(ref_root: str) -> None:
    kv_dir = os.path.join(ref_root, "polarengine_vllm", "kv_cache")
    for name, path in (("polarengine_vllm", os.path.join(ref_root, "polarengine_vllm")),
                       ("polarengine_vllm.kv_cache", kv_dir)):
        shell = types.ModuleType(name)
        shell.__path__ = [path]
        sys.modules[name] = shell
    _load("polarengine_vllm.kv_cache.config", os.path.join(kv_dir, "config.py"))
    cache = _load("polarengine_vllm.kv_cache.cache", os.path.join(kv_dir, "cache.py"))

    out = {}
    for b in (2, 3, 4):
        out[f"kv_centroids_b{b}"] = cache.get_centroids(b).numpy().astype(np.float32)
    g = torch.Generator().manual_seed(1234)
    codes = torch.randint(0, 16, (4, 128), generator=g, dtype=torch.int64)
    out["kv_pack_codes"] = codes.numpy().astype(np.int8)
    for b in (2, 3, 4):
        c = codes % (1 << b)
        out[f"kv_pack_b{b}"] = cache.BitPacker.pack(c, b).numpy()
    for d in (64, 128):
        x = (torch.randn(24, d, generator=torch.Generator().manual_seed(d)) * 0.7).to(torch.bfloat16)
        out[f"kv_x_d{d}"] = x.view(torch.int16).numpy().view(np.uint16)
        for b in (2, 3, 4):
            qz = cache.PolarKVQuantizer(head_dim=d, nbits=b, device="cpu")
            packed, norms = qz.quantize(x)
            deq = qz.dequantize(packed, norms, tuple(x.shape))
            out[f"kv_packed_d{d}_b{b}"] = packed.numpy()
            out[f"kv_norms_d{d}_b{b}"] = norms.view(torch.int16).numpy().view(np.uint16)
            out[f"kv_deq_d{d}_b{b}"] = deq.view(torch.int16).numpy().view(np.uint16)
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_kv.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out)} arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
