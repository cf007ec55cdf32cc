"""Batched matmul and dispatch (reference: kernels/polar_gemm.py).

``polar_matmul`` keeps the reference's signature and returns float32:
M = 1 runs the decode GEMV, M > 1 the MFMA GEMM, both through
``pe_polar_matmul``.
"""

from __future__ import annotations

from typing import Optional

import torch

from polarengine_vllm import _lib


def _matmul(codes: torch.Tensor, packed: bool, x_tf: torch.Tensor, norms: torch.Tensor,
            ct_scaled: torch.Tensor, out_f: int, in_f_padded: int) -> torch.Tensor:
    dev = _lib.require_device(codes, x_tf, norms, ct_scaled)
    x = x_tf.reshape(-1, in_f_padded).to(torch.float32).contiguous()
    m = x.shape[0]
    out = torch.empty(m, out_f, dtype=torch.float32, device=dev)
    nrm = norms.reshape(-1).to(torch.float16).contiguous()
    ct = ct_scaled.to(torch.float32).contiguous()
    L = _lib.lib()
    ws_bytes = L.pe_polar_matmul_workspace_size(m, in_f_padded)
    ws = _lib.workspace(dev, ws_bytes)
    _lib.check(L.pe_polar_matmul(codes.contiguous().data_ptr(), int(packed), x.data_ptr(), m,
                                 nrm.data_ptr(), ct.data_ptr(), ct.numel(), out.data_ptr(), out_f,
                                 in_f_padded, _lib.ptr(ws), ws_bytes, _lib.stream_ptr(dev)),
               "pe_polar_matmul")
    return out


def polar_gemm(codes: torch.Tensor, x_transformed: torch.Tensor, norms: torch.Tensor,
               ct_scaled: torch.Tensor, out_f: int, in_f_padded: int, n_blocks: int,
               block_size: int = 128) -> torch.Tensor:
    """int8 codes, x_tf float32 [M, in_f_padded] -> float32 [M, out_f]."""
    return _matmul(codes, False, x_transformed, norms, ct_scaled, out_f, in_f_padded)


def polar_gemm_packed(packed_codes: torch.Tensor, x_transformed: torch.Tensor,
                      norms: torch.Tensor, ct_scaled: torch.Tensor, out_f: int, in_f_half: int,
                      n_blocks: int, block_size: int = 128) -> torch.Tensor:
    """Nibble codes, x_tf float32 [M, 2 * in_f_half] -> float32 [M, out_f]."""
    return _matmul(packed_codes, True, x_transformed, norms, ct_scaled, out_f, n_blocks * block_size)


def polar_matmul(codes: Optional[torch.Tensor], x_transformed: torch.Tensor,
                 norms: torch.Tensor, ct_scaled: torch.Tensor, out_f: int, in_f_padded: int,
                 n_blocks: int, block_size: int = 128, packed: bool = False,
                 packed_codes: Optional[torch.Tensor] = None,
                 in_f_half: Optional[int] = None) -> torch.Tensor:
    """GEMV for one vector, GEMM for a batch; output shape follows the input
    (``[out_f]`` for a 1-D x, ``[M, out_f]`` for 2-D), float32."""
    use_packed = packed and packed_codes is not None and in_f_half is not None
    c = packed_codes if use_packed else codes
    if c is None:
        raise ValueError("codes (or packed_codes with packed=True) required")
    y = _matmul(c, use_packed, x_transformed, norms, ct_scaled, out_f, in_f_padded)
    return y.reshape(-1) if x_transformed.dim() == 1 else y
