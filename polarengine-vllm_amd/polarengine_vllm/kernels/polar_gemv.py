"""Decode GEMV entry points (reference: kernels/polar_gemv.py).

Same names and arguments as the reference's Triton wrappers; the work is done
by the gfx950 kernels behind ``pe_polar_gemv`` / ``pe_polar_gemv_packed``.
Output is float32 ``[out_f]`` as in the reference.
"""

from __future__ import annotations

import torch

from polarengine_vllm import _lib

HAS_TRITON = False  # kept for API parity: no Triton anywhere in this package


def _norms_f16(norms: torch.Tensor) -> torch.Tensor:
    # the runtime format stores fp16 norms; accept fp32 like the Triton
    # wrappers did and convert (load-time cost, not per call, when cached)
    n = norms.reshape(-1)
    return n if n.dtype == torch.float16 else n.to(torch.float16)


def polar_gemv(codes: torch.Tensor, x_transformed: torch.Tensor, norms: torch.Tensor,
               ct_scaled: torch.Tensor, out_f: int, in_f_padded: int, n_blocks: int,
               block_size: int = 128) -> torch.Tensor:
    """int8 codes [out_f, in_f_padded] . x_tf (float32 [in_f_padded]) -> float32 [out_f]."""
    dev = _lib.require_device(codes, x_transformed, norms, ct_scaled)
    out = torch.empty(out_f, dtype=torch.float32, device=dev)
    x = x_transformed.reshape(-1).to(torch.float32).contiguous()
    nrm = _norms_f16(norms).contiguous()
    ct = ct_scaled.to(torch.float32).contiguous()
    _lib.check(_lib.lib().pe_polar_gemv(
        codes.contiguous().data_ptr(), x.data_ptr(), nrm.data_ptr(), ct.data_ptr(), ct.numel(),
        out.data_ptr(), out_f, in_f_padded, n_blocks, block_size, _lib.stream_ptr(dev)),
        "pe_polar_gemv")
    return out


def polar_gemv_packed(packed_codes: torch.Tensor, x_transformed: torch.Tensor,
                      norms: torch.Tensor, ct_scaled: torch.Tensor, out_f: int, in_f_half: int,
                      n_blocks: int, block_size: int = 128) -> torch.Tensor:
    """Nibble codes uint8 [out_f, in_f_half] . x_tf -> float32 [out_f]."""
    dev = _lib.require_device(packed_codes, x_transformed, norms, ct_scaled)
    out = torch.empty(out_f, dtype=torch.float32, device=dev)
    x = x_transformed.reshape(-1).to(torch.float32).contiguous()
    nrm = _norms_f16(norms).contiguous()
    ct = ct_scaled.to(torch.float32).contiguous()
    _lib.check(_lib.lib().pe_polar_gemv_packed(
        packed_codes.contiguous().data_ptr(), x.data_ptr(), nrm.data_ptr(), ct.data_ptr(),
        ct.numel(), out.data_ptr(), out_f, in_f_half, n_blocks, block_size, _lib.stream_ptr(dev)),
        "pe_polar_gemv_packed")
    return out


def pack_codes_int4(codes: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """Half-block nibble pack (same mapping as packing.pack_codes_half_block)."""
    from polarengine_vllm.packing import pack_codes_half_block
    return pack_codes_half_block(codes, block_size)
