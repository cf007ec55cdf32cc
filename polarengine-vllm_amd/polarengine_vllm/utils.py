"""PolarEngine format utilities: Lloyd-Max codebook, bit rules, nibble packing.

Host-side (load-time / offline) helpers with the reference's names and
behaviour (polarengine_vllm/utils.py). The per-token compute lives in the HIP
library; nothing here runs on the inference hot path.
"""

from __future__ import annotations

from typing import Dict, Optional

import numpy as np
import torch

# ---------------------------------------------------------------------------
# Lloyd-Max codebook (reference: utils.py:21-105)
# ---------------------------------------------------------------------------


def compute_lloyd_max_centroids(n_levels: int, n_iter: int = 100) -> torch.Tensor:
    """MSE-optimal levels for N(0, 1) after ``n_iter`` Lloyd-Max iterations.

    Float64 iteration from uniform boundaries on [-4, 4] with infinite ends;
    centroid = conditional mean (pdf(a) - pdf(b)) / (cdf(b) - cdf(a)) where
    that probability exceeds 1e-10, midpoint otherwise; boundaries = centroid
    midpoints. The stored format depends on the exact iteration count (the
    reference stops at 100, before convergence for 4+ bits), so keep it.
    Returns float32.
    """
    from scipy.stats import norm

    edges = np.linspace(-4.0, 4.0, n_levels + 1)
    edges[0], edges[-1] = -np.inf, np.inf
    cents = np.zeros(n_levels)
    for _ in range(n_iter):
        lo, hi = edges[:-1], edges[1:]
        cents = np.empty(n_levels)
        for i in range(n_levels):
            p = norm.cdf(hi[i]) - norm.cdf(lo[i])
            cents[i] = (norm.pdf(lo[i]) - norm.pdf(hi[i])) / p if p > 1e-10 else (lo[i] + hi[i]) / 2
        edges = np.concatenate([[-np.inf], (cents[:-1] + cents[1:]) / 2, [np.inf]])
    return torch.tensor(cents, dtype=torch.float32)


_centroids_cache: Dict[int, torch.Tensor] = {}


def get_centroids(bits: int) -> torch.Tensor:
    """Cached Lloyd-Max centroids for ``bits`` in [2, 8] (float32, CPU)."""
    if bits < 2 or bits > 8:
        raise ValueError(f"bits must be in [2, 8], got {bits}")
    if bits not in _centroids_cache:
        _centroids_cache[bits] = compute_lloyd_max_centroids(1 << bits)
    return _centroids_cache[bits]


# ---------------------------------------------------------------------------
# Mixed-bit assignment (reference: utils.py:112-204)
# ---------------------------------------------------------------------------

DEFAULT_BIT_ASSIGNMENT: Dict[str, int] = {
    "embed": 5,
    "lm_head": 6,
    "q_proj": 5,
    "k_proj": 5,
    "v_proj": 5,
    "o_proj": 6,
    "out_proj": 6,
    "gate_up_proj": 3,
    "gate_proj": 3,
    "up_proj": 3,
    "down_proj": 4,
    "in_proj": 5,
}

_SKIP_LOWER = ("norm", "layernorm", "rmsnorm", "a_log", "dt_bias", "dt_proj", "conv1d")
_SKIP_EXACT = (".D", "A_log")  # case-sensitive: ".d" would hit "down_proj"


def get_bits_for_layer(name: str, param: torch.Tensor,
                       assignment: Optional[Dict[str, int]] = None) -> int:
    """Bit width for a named parameter; 16 means "keep in fp16".

    Same rules and order as the reference: small / 1-D tensors, norm and
    Mamba buffers, biases and MoE routers stay fp16; otherwise the longest
    matching key of ``assignment`` wins; unknown names default to 5 bits.
    """
    table = DEFAULT_BIT_ASSIGNMENT if assignment is None else assignment
    if param.ndim < 2 or param.numel() < 256:
        return 16
    low = name.lower()
    if any(k in low for k in _SKIP_LOWER) or any(k in name for k in _SKIP_EXACT):
        return 16
    if "bias" in name and param.ndim == 1:
        return 16
    if name.endswith(".gate.weight") or "router" in name:
        return 16
    for key in sorted(table, key=len, reverse=True):
        if key in name:
            return table[key]
    return 5


# ---------------------------------------------------------------------------
# Nibble packing, half-block order (reference: utils.py:211-286)
# ---------------------------------------------------------------------------


def pack_codes_half_block(codes: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """``byte[i] = code[block_size // 2 + i] << 4 | code[i]`` per block.

    Works on any leading shape. Device tensors go through the HIP packer.
    """
    from polarengine_vllm.packing import pack_codes_half_block as _p
    return _p(codes, block_size)


def unpack_codes_half_block(packed: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """Inverse of :func:`pack_codes_half_block`."""
    from polarengine_vllm.packing import unpack_codes_half_block as _u
    return _u(packed, block_size)
