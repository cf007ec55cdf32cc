"""Blockwise Walsh-Hadamard transform (reference: kernels/fwht.py).

``fwht_matmul`` keeps the reference's name and contract (each contiguous
``block_size`` block of the last dimension multiplied by the normalised
Hadamard matrix) but runs the gfx950 butterfly kernel ``pe_fwht128`` instead
of an fp32 GEMM against H; block_size 128. ``fwht_butterfly`` transforms the
whole last dimension (any power of two up to 32768) with ``pe_fwht_pow2``.
GPU tensors only.
"""

from __future__ import annotations

import math
import weakref
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


def fwht_butterfly(x: torch.Tensor) -> torch.Tensor:
    """Normalised Walsh-Hadamard transform over the whole last dimension.

    Reference: kernels/fwht.py:160-190 (``fwht_butterfly``): stages
    h = 1, 2, 4, ..., n/2 pair (a, b) -> (a + b, a - b), then divide by
    sqrt(n); the last dimension must be a power of two (AssertionError
    otherwise). Runs ``pe_fwht_pow2`` (n <= 32768): fp32 arithmetic, one
    rounding to x's dtype. Unlike the reference, which butterflies in x's own
    precision and leaves x overwritten with the unnormalised stages, x is not
    modified. GPU tensors only.
    """
    n = x.shape[-1]
    assert n >= 1 and (n & (n - 1)) == 0, f"last dim must be power of 2, got {n}"
    dev = _lib.require_device(x)
    dt = {torch.float16: _lib.PE_DTYPE_F16, torch.bfloat16: _lib.PE_DTYPE_BF16,
          torch.float32: _lib.PE_DTYPE_F32}.get(x.dtype)
    if dt is None:
        raise TypeError(f"unsupported dtype {x.dtype}")
    xc = x.contiguous()
    out = torch.empty_like(xc)
    rows = xc.numel() // n
    if rows:
        _lib.check(_lib.lib().pe_fwht_pow2(xc.data_ptr(), dt, rows, n, n, out.data_ptr(), dt,
                                           _lib.stream_ptr(dev)), "pe_fwht_pow2")
    return out.view(x.shape)


class FWHTCache:
    """Single-entry cache of an FWHT result, shared by Q/K/V projections.

    Same interface as the reference (kernels/fwht.py:115-153): ``get``
    returns the cached transform when ``x`` is the tensor that was ``put``,
    ``clear`` empties it.

    The entry is keyed on the tensor object itself (held weakly: the entry,
    and with it the transform, is dropped as soon as ``x`` is freed), its
    geometry and, for tensors that track versions, its version counter, so an
    in-place update of ``x`` through torch misses instead of returning a stale
    transform.

    Inference tensors (``torch.inference_mode()``, which vLLM runs every
    forward under) track no version. For them the cache holds an entry only
    inside a *scope*: ``install_fwht_cache_hooks`` (linear_method) opens one
    around every forward of a module that owns PolarQuant linears and clears
    the cache on entry and exit, so an entry only ever serves sibling
    projections inside one parent forward. Outside a scope an inference
    tensor is never cached (each projection transforms its own input), since
    a hidden-state tensor that is updated in place between layers would
    otherwise be served the previous layer's transform.

    A write that bypasses torch (a kernel handed ``x.data_ptr()``) does not
    bump the version either. This package's own wrappers record such writes
    into caller tensors (``increment_version``); anything else must use the
    scope hooks.
    """

    def __init__(self):
        self._ref = None
        self._key = None
        self._result: Optional[torch.Tensor] = None
        self._scope = 0

    @staticmethod
    def _make_key(x: torch.Tensor, in_f: int):
        ver = None if x.is_inference() else x._version
        return (x.data_ptr(), in_f, tuple(x.shape), tuple(x.stride()), x.dtype, ver)

    def _cacheable(self, x: torch.Tensor) -> bool:
        return self._scope > 0 or not x.is_inference()

    def get(self, x: torch.Tensor, in_f: int) -> Optional[torch.Tensor]:
        if self._ref is None or self._ref() is not x or not self._cacheable(x):
            return None
        if self._key != self._make_key(x, in_f):
            return None
        return self._result

    def put(self, x: torch.Tensor, in_f: int, result: torch.Tensor) -> None:
        if not self._cacheable(x):
            self.clear()
            return
        self.clear()
        self._ref = weakref.ref(x, self._on_free)
        self._key = self._make_key(x, in_f)
        self._result = result

    def _on_free(self, ref) -> None:
        if self._ref is ref:
            self.clear()

    def clear(self) -> None:
        self._ref = None
        self._key = None
        self._result = None

    def enter_scope(self) -> None:
        """Start a parent module's forward: empty, and serve inference tensors."""
        self.clear()
        self._scope += 1

    def exit_scope(self) -> None:
        """End a parent module's forward: empty, and drop the transform."""
        self.clear()
        self._scope = max(0, self._scope - 1)


# Process-wide cache used by the linear method, so separate q/k/v (or
# gate/up) modules reading the same hidden state share one transform.
GLOBAL_FWHT_CACHE = FWHTCache()
