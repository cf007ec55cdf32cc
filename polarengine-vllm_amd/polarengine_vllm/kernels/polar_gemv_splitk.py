"""Split-K GEMV names (reference: kernels/polar_gemv_splitk.py).

The reference splits K over workgroups to fill NVIDIA SMs: ``split_k``
picks the number of K slices (``_choose_split_k``, :399-418, when None) and
``use_atomic`` chooses between a two-pass reduction and ``tl.atomic_add``
into a zeroed output (:421-569). Both are schedule knobs: every choice
computes the same function, y[n] = sum over blocks of norm * <ct[codes],
x_tf>. On gfx950 the GEMV behind these names (``pe_polar_gemv[_packed]``)
already spreads each row's K over a wave and fills the 256 CUs with a
persistent row grid, so it has no K split to configure: the knobs are
validated and have no other effect, and the result is deterministic (the
reference's atomic variant is not).
"""

from __future__ import annotations

from typing import Optional

import torch

from polarengine_vllm.kernels.polar_gemv import polar_gemv, polar_gemv_packed


def _check_knobs(split_k: Optional[int], use_atomic: bool) -> None:
    if split_k is not None and int(split_k) < 1:
        raise ValueError(f"split_k must be None or >= 1, got {split_k}")
    if not isinstance(use_atomic, bool):
        raise TypeError("use_atomic must be a bool")


def polar_gemv_splitk(codes: torch.Tensor, x_transformed: torch.Tensor, norms: torch.Tensor,
                      ct_scaled: torch.Tensor, out_f: int, in_f_padded: int, n_blocks: int,
                      block_size: int = 128, split_k: Optional[int] = None,
                      use_atomic: bool = False) -> torch.Tensor:
    """int8 codes: float32 [out_f] (reference :421-494); split_k / use_atomic
    are accepted for the reference's signature and change nothing here."""
    _check_knobs(split_k, use_atomic)
    return polar_gemv(codes, x_transformed, norms, ct_scaled, out_f, in_f_padded, n_blocks,
                      block_size)


def polar_gemv_packed_splitk(packed_codes: torch.Tensor, x_transformed: torch.Tensor,
                             norms: torch.Tensor, ct_scaled: torch.Tensor, out_f: int,
                             in_f_half: int, n_blocks: int, block_size: int = 128,
                             split_k: Optional[int] = None, use_atomic: bool = False
                             ) -> torch.Tensor:
    """Nibble codes: float32 [out_f] (reference :497-569); knobs as above."""
    _check_knobs(split_k, use_atomic)
    return polar_gemv_packed(packed_codes, x_transformed, norms, ct_scaled, out_f, in_f_half,
                             n_blocks, block_size)
