"""Offline PolarQuant quantizer (reference: polarengine_vllm/quantizer.py:178-257).

``PolarQuantizer.quantize_tensor`` turns a weight matrix into the
codes / fp16 norms / ct_scaled triple: pad K to the block, per-block L2 norm
(clamped at 1e-10), unit blocks rotated by H and scaled by sqrt(bs), code =
first index of the nearest centroid. Torch ops on whatever device the weight
is on -- this is checkpoint tooling, not the inference path.
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
    def quantize_tensor(self, weight: torch.Tensor, bits: int) -> Dict[str, torch.Tensor]:
        bs = self.block_size
        dev = weight.device
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
