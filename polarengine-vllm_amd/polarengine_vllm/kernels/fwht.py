"""Blockwise Walsh-Hadamard transform (reference: kernels/fwht.py).

``fwht_matmul`` keeps the reference's name and contract (each contiguous
``block_size`` block of the last dimension multiplied by the normalised
Hadamard matrix) but runs the gfx950 butterfly kernel ``pe_fwht128`` instead
of an fp32 GEMM against H. GPU tensors only; block_size 128.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
from torch.autograd.graph import increment_version

from polarengine_vllm import _lib

_hadamard_cache: dict = {}


def build_hadamard(n: int, device: torch.device = None) -> torch.Tensor:
    """Normalised Sylvester Hadamard matrix (power-of-two ``n``), cached.

    Reference: kernels/fwht.py:28-70 (recursive [[h, h], [h, -h]] / sqrt 2).
    Host-side constant for callers that want H itself; the kernels never use it.
    """
    assert n >= 1 and (n & (n - 1)) == 0, f"n must be a power of 2, got {n}"
    key = (n, str(device) if device is not None else "cpu")
    if key not in _hadamard_cache:
        if n == 1:
            h = torch.tensor([[1.0]])
        else:
            s = build_hadamard(n // 2)
            h = torch.cat([torch.cat([s, s], 1), torch.cat([s, -s], 1)], 0) / math.sqrt(2)
        _hadamard_cache[key] = h if device is None else h.to(device)
    return _hadamard_cache[key]


def fwht_matmul(x: torch.Tensor, block_size: int = 128, out: Optional[torch.Tensor] = None
                ) -> torch.Tensor:
    """FWHT of every contiguous ``block_size`` block of the last dim.

    Output has x's shape; dtype float32 for float32 input, else x's dtype.
    ``out`` may alias ``x`` for float32 (in-place, like the CUDA ``fwht_``).
    """
    in_features = x.shape[-1]
    assert in_features % block_size == 0, (
        f"in_features ({in_features}) must be divisible by block_size ({block_size})")
    if block_size != 128:
        raise ValueError("the gfx950 FWHT kernel implements block_size 128")
    dev = _lib.require_device(x)
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"unsupported dtype {x.dtype}")
    xc = x.contiguous()
    rows = xc.numel() // in_features if in_features else 0
    caller_out = out is not None
    if out is None:
        out = torch.empty_like(xc)
    layout = {torch.float32: _lib.PE_XTF_F32, torch.float16: _lib.PE_XTF_F16,
              torch.bfloat16: _lib.PE_XTF_BF16}.get(out.dtype)
    if layout is None:
        raise TypeError(f"unsupported output dtype {out.dtype}")
    dt = {torch.float16: _lib.PE_DTYPE_F16, torch.bfloat16: _lib.PE_DTYPE_BF16,
          torch.float32: _lib.PE_DTYPE_F32}[xc.dtype]
    _lib.check(_lib.lib().pe_fwht128(xc.data_ptr(), dt, rows, in_features, in_features,
                                     out.data_ptr(), layout, _lib.stream_ptr(dev)), "pe_fwht128")
    if caller_out:
        # the kernel wrote the caller's tensor through a raw pointer: record
        # the write so that version-keyed caches (FWHTCache) see it
        increment_version(out)
    return out.view(x.shape)


def fwht_pairs(x: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """FWHT into the kernels' pair-f16 layout: int32 view [rows, K/2] where
    word ``(b, i)`` holds halves (x_tf[128 b + i], x_tf[128 b + 64 + i])."""
    k = x.shape[-1]
    assert k % block_size == 0 and block_size == 128
    dev = _lib.require_device(x)
    xc = x.contiguous()
    rows = xc.numel() // k
    dt = {torch.float16: _lib.PE_DTYPE_F16, torch.bfloat16: _lib.PE_DTYPE_BF16,
          torch.float32: _lib.PE_DTYPE_F32}[xc.dtype]
    out = torch.empty(rows, k // 2, dtype=torch.int32, device=dev)
    _lib.check(_lib.lib().pe_fwht128(xc.data_ptr(), dt, rows, k, k, out.data_ptr(),
                                     _lib.PE_XTF_PAIR_F16, _lib.stream_ptr(dev)), "pe_fwht128")
    return out


class FWHTCache:
    """Single-entry cache of an FWHT result, shared by Q/K/V projections.

    Same interface as the reference (kernels/fwht.py:115-153): ``get``
    returns the cached transform when ``x`` is the tensor that was ``put``,
    ``clear`` empties it. The entry keeps a reference to ``x`` and records
    its version counter and geometry, so a different tensor that later
    reuses the same storage address, or an in-place update of ``x`` through
    torch, misses instead of returning a stale transform.

    A write that bypasses torch (a kernel handed ``x.data_ptr()``) does not
    bump the version. This package's own wrappers record such writes into
    caller tensors (``increment_version``); for anything else the cache must
    be scoped: ``install_fwht_cache_hooks`` (linear_method) clears it at the
    start of every forward of a module that owns PolarQuant linears, so an
    entry only ever serves sibling projections inside one parent forward.
    """

    def __init__(self):
        self._x: Optional[torch.Tensor] = None
        self._key = None
        self._result: Optional[torch.Tensor] = None

    @staticmethod
    def _make_key(x: torch.Tensor, in_f: int):
        return (x.data_ptr(), in_f, tuple(x.shape), tuple(x.stride()), x.dtype, x._version)

    def get(self, x: torch.Tensor, in_f: int) -> Optional[torch.Tensor]:
        if self._x is not None and self._key == self._make_key(x, in_f):
            return self._result
        return None

    def put(self, x: torch.Tensor, in_f: int, result: torch.Tensor) -> None:
        self._x = x
        self._key = self._make_key(x, in_f)
        self._result = result

    def clear(self) -> None:
        self._x = None
        self._key = None
        self._result = None


# Process-wide cache used by the linear method, so separate q/k/v (or
# gate/up) modules reading the same hidden state share one transform.
GLOBAL_FWHT_CACHE = FWHTCache()
