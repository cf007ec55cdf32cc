"""Split-K GEMV names (reference: kernels/polar_gemv_splitk.py).

The reference splits K over workgroups to fill NVIDIA SMs and reduces in a
second pass. The gfx950 kernel streams whole rows per wave with a persistent
grid and needs no split, so these names compute the same function through
the same entry points as :mod:`polar_gemv`.
"""

from __future__ import annotations

import torch

from polarengine_vllm.kernels.polar_gemv import polar_gemv, polar_gemv_packed


def polar_gemv_splitk(codes: torch.Tensor, x_transformed: torch.Tensor, norms: torch.Tensor,
                      ct_scaled: torch.Tensor, out_f: int, in_f_padded: int, n_blocks: int,
                      block_size: int = 128, split_k: int | None = None,
                      use_atomic: bool = False) -> torch.Tensor:
    return polar_gemv(codes, x_transformed, norms, ct_scaled, out_f, in_f_padded, n_blocks,
                      block_size)


def polar_gemv_packed_splitk(packed_codes: torch.Tensor, x_transformed: torch.Tensor,
                             norms: torch.Tensor, ct_scaled: torch.Tensor, out_f: int,
                             in_f_half: int, n_blocks: int, block_size: int = 128,
                             split_k: int | None = None, use_atomic: bool = False) -> torch.Tensor:
    return polar_gemv_packed(packed_codes, x_transformed, norms, ct_scaled, out_f, in_f_half,
                             n_blocks, block_size)
