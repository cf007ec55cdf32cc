"""Write golden input/output vectors from the reference's own CPU functions.

Run in the build container only (the reference tree is absent on the GPU box):

    python tests/golden/make_golden.py /path/to/reference

It loads individual reference source files by path (utils.py, packing.py,
kernels/fwht.py, quantizer.py, weight_converter.py) without executing the
package ``__init__`` (which pulls in the HF integration), calls the CPU
functions whose exact float32/byte output no closed form pins, and saves
inputs and outputs as ``golden.npz`` (plain arrays, no pickles) beside this
script. The vectors pin the oracle in ``oracle/polar_oracle.py``:

* ``utils.get_centroids(b)`` for b = 2..8 (100-iteration Lloyd-Max);
* ``kernels.fwht.build_hadamard(128)`` and ``fwht_matmul`` on a seeded input;
* ``PolarQuantizer.quantize_tensor`` codes/norms/ct_scaled at b = 2..6 on a
  seeded fp16 weight with a padded K;
* ``packing.pack_codes_half_block``, ``pack_codes_q5``, ``pack_codes_q5_hlwq``
  byte outputs;
* ``weight_converter._dequant_weight`` (bf16 result) on the Q4 codes.
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
    pkg_dir = os.path.join(ref_root, "polarengine_vllm")
    # Namespace shells so that ``from polarengine_vllm.x import y`` inside the
    # loaded files resolves to the files loaded here, not to the package
    # __init__ (which imports transformers/hub code unrelated to this path).
    pkg = types.ModuleType("polarengine_vllm")
    pkg.__path__ = [pkg_dir]
    sys.modules["polarengine_vllm"] = pkg
    kpkg = types.ModuleType("polarengine_vllm.kernels")
    kpkg.__path__ = [os.path.join(pkg_dir, "kernels")]
    sys.modules["polarengine_vllm.kernels"] = kpkg

    utils = _load("polarengine_vllm.utils", os.path.join(pkg_dir, "utils.py"))
    packing = _load("polarengine_vllm.packing", os.path.join(pkg_dir, "packing.py"))
    fwht = _load("polarengine_vllm.kernels.fwht", os.path.join(pkg_dir, "kernels", "fwht.py"))
    quantizer = _load("polarengine_vllm.quantizer", os.path.join(pkg_dir, "quantizer.py"))
    wconv = _load("polarengine_vllm.weight_converter",
                  os.path.join(pkg_dir, "weight_converter.py"))

    out = {}
    for b in range(2, 9):
        out[f"centroids_b{b}"] = utils.get_centroids(b).numpy().astype(np.float32)

    out["hadamard128"] = fwht.build_hadamard(128).numpy().astype(np.float32)
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(4, 384, generator=g, dtype=torch.float32)
    out["fwht_in"] = x.numpy()
    out["fwht_out"] = fwht.fwht_matmul(x, 128).numpy()

    g = torch.Generator().manual_seed(2024)
    w = (torch.randn(32, 200, generator=g, dtype=torch.float32) * 0.02).half()
    out["quant_w"] = w.numpy()
    q = quantizer.PolarQuantizer(block_size=128)
    for b in range(2, 7):
        r = q.quantize_tensor(w, b)
        out[f"quant_codes_b{b}"] = r["codes"].numpy()
        out[f"quant_norms_b{b}"] = r["norms"].numpy()
        out[f"quant_ct_scaled_b{b}"] = r["ct_scaled"].numpy()

    g = torch.Generator().manual_seed(7)
    c16 = torch.randint(0, 16, (4, 256), generator=g, dtype=torch.int8)
    c32 = torch.randint(0, 32, (4, 256), generator=g, dtype=torch.int8)
    c32_odd = torch.randint(0, 32, (3, 250), generator=g, dtype=torch.int8)
    out["pack_codes16"] = c16.numpy()
    out["pack_nibble"] = packing.pack_codes_half_block(c16, 128).numpy()
    out["pack_codes32"] = c32.numpy()
    out["pack_q5"] = packing.pack_codes_q5(c32, 128).numpy()
    out["pack_q5_hlwq"] = packing.pack_codes_q5_hlwq(c32).numpy()
    out["pack_codes32_odd"] = c32_odd.numpy()
    out["pack_q5_hlwq_odd"] = packing.pack_codes_q5_hlwq(c32_odd).numpy()

    # weight_converter._dequant_weight takes the raw centroids (it divides by
    # sqrt(bs) itself) and returns bf16; keep the fp32 view of that bf16.
    r4 = q.quantize_tensor(w, 4)
    deq = wconv._dequant_weight(r4["codes"], r4["norms"], utils.get_centroids(4), 128)
    out["dequant_b4_bf16_as_f32"] = deq.float().numpy()

    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out)} arrays")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
