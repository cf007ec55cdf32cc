"""Offline PolarQuant quantizer (reference: polarengine_vllm/quantizer.py:178-257).

``PolarQuantizer.quantize_tensor`` turns a weight matrix into the
codes / fp16 norms / ct_scaled triple: pad K to the block, per-block L2 norm
(clamped at 1e-10), unit blocks rotated by H and scaled by sqrt(bs), code =
first index of the nearest centroid. A weight on the GPU (block size 128) is
quantized by the HIP kernel ``pe_quantize`` in one pass (``pack=True`` also
writes the half-block nibbles for bits <= 4); a CPU weight takes the torch
expressions below (offline checkpoint tooling).
(``quantize_model`` of the reference downloads a model and is not provided.)
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import torch
import torch.nn.functional as F

from polarengine_vllm.utils import DEFAULT_BIT_ASSIGNMENT, get_centroids


def _hadamard(n: int, device) -> torch.Tensor:
    i = torch.arange(n)
    x = i[:, None] & i[None, :]
    parity = torch.zeros_like(x)
    while bool(x.any()):
        parity ^= x & 1
        x = x >> 1
    return ((1 - 2 * parity).to(torch.float64) / math.sqrt(n)).to(torch.float32).to(device)


class PolarQuantizer:
    def __init__(self, block_size: int = 128, bit_assignment: Optional[Dict[str, int]] = None):
        if block_size < 1 or block_size & (block_size - 1):
            raise ValueError(f"block_size must be a positive power of 2, got {block_size}")
        self.block_size = block_size
        self.bit_assignment = bit_assignment or dict(DEFAULT_BIT_ASSIGNMENT)

    @torch.no_grad()
    def quantize_tensor(self, weight: torch.Tensor, bits: int,
                        pack: bool = False) -> Dict[str, torch.Tensor]:
        """codes int8 [N, Kp] (or nibbles uint8 [N, Kp/2] with ``pack`` on the
        GPU, bits <= 4), norms fp16 [N, nb], ct_scaled fp32 [2**bits]."""
        bs = self.block_size
        dev = weight.device
        if dev.type == "cuda" and bs == 128:
            return _quantize_gpu(weight, bits, pack)
        if pack:
            raise ValueError("pack=True needs a GPU weight (the pe_quantize kernel)")
        ct = get_centroids(bits).to(dev)
        H = _hadamard(bs, dev)
        out_f, in_f = weight.shape
        kp = (in_f + bs - 1) // bs * bs
        nb = kp // bs
        w = weight.detach().float()
        if kp != in_f:
            w = F.pad(w, (0, kp - in_f))
        blocks = w.view(out_f, nb, bs)
        norms = blocks.norm(dim=2).clamp(min=1e-10)
        unit = blocks / norms.unsqueeze(2)
        codes = torch.empty(out_f, nb, bs, dtype=torch.int8, device=dev)
        scale = math.sqrt(bs)
        # rows per chunk: keep the (rows, nb, bs, levels) distance tensor ~256 MB
        chunk = max(1, (1 << 26) // max(1, nb * bs * ct.numel()))
        for i in range(0, out_f, chunk):
            e = min(i + chunk, out_f)
            rot = (unit[i:e].reshape(-1, bs) @ H) * scale
            d = (rot.view(e - i, nb, bs).unsqueeze(-1) - ct.view(1, 1, 1, -1)).abs()
            codes[i:e] = d.argmin(dim=-1).to(torch.int8)
        return {"codes": codes.reshape(out_f, kp), "norms": norms.half(), "ct_scaled": ct / scale}


def _quantize_gpu(weight: torch.Tensor, bits: int, pack: bool) -> Dict[str, torch.Tensor]:
    from polarengine_vllm import _lib
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D, got shape {tuple(weight.shape)}")
    if pack and bits > 4:
        raise ValueError(f"nibble packing needs bits <= 4, got {bits}")
    dtypes = {torch.float16: _lib.PE_DTYPE_F16, torch.bfloat16: _lib.PE_DTYPE_BF16,
              torch.float32: _lib.PE_DTYPE_F32}
    w = weight if weight.dtype in dtypes else weight.float()
    if w.stride(1) != 1:
        w = w.contiguous()
    n, k = w.shape
    kp = (k + 127) // 128 * 128
    ct = get_centroids(bits).to(device=w.device, dtype=torch.float32).contiguous()
    codes = torch.empty(n, kp // 2 if pack else kp, device=w.device,
                        dtype=torch.uint8 if pack else torch.int8)
    norms = torch.empty(n, kp // 128, device=w.device, dtype=torch.float16)
    _lib.check(_lib.lib().pe_quantize(w.data_ptr(), dtypes[w.dtype], n, k, w.stride(0),
                                      ct.data_ptr(), ct.numel(), int(pack), codes.data_ptr(),
                                      norms.data_ptr(), _lib.stream_ptr(w.device)),
               "pe_quantize")
    # divided on the CPU, as the reference does (a GPU division by the scalar
    # can round differently)
    ct_scaled = (get_centroids(bits) / math.sqrt(128)).to(device=w.device, dtype=torch.float32)
    return {"codes": codes, "norms": norms, "ct_scaled": ct_scaled}
