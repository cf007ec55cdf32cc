"""PolarQuant KV-cache compression (reference: kv_cache/cache.py).

* ``get_centroids(nbits)`` -- the KV codebook (Lloyd-Max for N(0,1) with the
  finite +-4 interval ends and float32 round trips of the reference's loop,
  cache.py:27-54; not the weight codebook of utils.get_centroids);
* ``BitPacker`` -- the KV byte layouts (MSB first; 4-bit keeps the even code
  in the high nibble), torch expressions for host-side tooling;
* ``PolarKVQuantizer`` -- quantize / dequantize on the GPU through the HIP
  kernels ``pe_kv_quantize`` / ``pe_kv_dequantize`` (one pass each: norm,
  Hadamard, nearest centroid, pack; unpack, lookup, Hadamard, scale);
* ``PolarKVLayer`` / ``PolarKVCache`` -- the cache manager: the newest
  ``residual_length`` tokens stay in bf16, older ones are compressed.

What differs from the reference, on purpose: the quantized history is kept in
place in preallocated buffers that grow geometrically (the reference
concatenates the whole history on every update, cache.py:304-306) and only
the newly compressed tokens are expanded again on the next read: the layer
keeps the bf16 expansion of its compressed history and appends to it.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch
from torch.autograd.graph import increment_version

from .config import PolarKVConfig

_CT_CACHE: Dict[int, torch.Tensor] = {}


def get_centroids(nbits: int) -> torch.Tensor:
    """KV Lloyd-Max levels, float32, cached (reference: cache.py:27-54)."""
    if nbits in _CT_CACHE:
        return _CT_CACHE[nbits]
    from scipy.stats import norm as sp_norm
    n = 1 << nbits
    bnd = torch.linspace(-4.0, 4.0, n + 1)
    ct = torch.zeros(n)
    for _ in range(100):
        for i in range(n):
            a, b = float(bnd[i]), float(bnd[i + 1])
            pa, pb = sp_norm.cdf(a), sp_norm.cdf(b)
            ct[i] = (a + b) / 2 if pb - pa < 1e-12 else (sp_norm.pdf(a) - sp_norm.pdf(b)) / (pb - pa)
        for i in range(1, n):
            bnd[i] = (ct[i - 1] + ct[i]) / 2
    _CT_CACHE[nbits] = ct
    return ct


def build_hadamard(n: int, device: str = "cpu") -> torch.Tensor:
    """Orthonormal Sylvester-Hadamard matrix, float32 (reference: cache.py:65-88)."""
    if n < 1 or n & (n - 1):
        raise ValueError(f"n must be a power of 2, got {n}")
    i = torch.arange(n)
    x = i[:, None] & i[None, :]
    parity = torch.zeros_like(x)
    while bool(x.any()):
        parity ^= x & 1
        x = x >> 1
    return ((1 - 2 * parity).to(torch.float64) / math.sqrt(n)).to(torch.float32).to(device)


class BitPacker:
    """KV code byte layouts (reference: cache.py:95-173)."""

    @staticmethod
    def pack(codes: torch.Tensor, nbits: int) -> torch.Tensor:
        c = codes.long()
        n = c.shape[0]
        if nbits == 2:
            g = c.reshape(n, -1, 4)
            out = (g[..., 0] << 6) | (g[..., 1] << 4) | (g[..., 2] << 2) | g[..., 3]
        elif nbits == 3:
            g = c.reshape(n, -1, 8)
            b0 = (g[..., 0] << 5) | (g[..., 1] << 2) | (g[..., 2] >> 1)
            b1 = ((g[..., 2] & 1) << 7) | (g[..., 3] << 4) | (g[..., 4] << 1) | (g[..., 5] >> 2)
            b2 = ((g[..., 5] & 3) << 6) | (g[..., 6] << 3) | g[..., 7]
            out = torch.stack([b0, b1, b2], dim=-1).reshape(n, -1)
        elif nbits == 4:
            out = (c[:, 0::2] << 4) | c[:, 1::2]
        else:
            return codes.to(torch.uint8)
        return out.to(torch.uint8)

    @staticmethod
    def unpack(packed: torch.Tensor, nbits: int, D: int) -> torch.Tensor:
        p = packed.long()
        n = p.shape[0]
        if nbits == 2:
            return torch.stack([(p >> 6) & 3, (p >> 4) & 3, (p >> 2) & 3, p & 3], -1).reshape(n, D)
        if nbits == 3:
            g = p.reshape(n, -1, 3)
            b0, b1, b2 = g[..., 0], g[..., 1], g[..., 2]
            return torch.stack([(b0 >> 5) & 7, (b0 >> 2) & 7, ((b0 & 3) << 1) | ((b1 >> 7) & 1),
                                (b1 >> 4) & 7, (b1 >> 1) & 7, ((b1 & 1) << 2) | ((b2 >> 6) & 3),
                                (b2 >> 3) & 7, b2 & 7], -1).reshape(n, D)
        if nbits == 4:
            return torch.stack([(p >> 4) & 0xF, p & 0xF], -1).reshape(n, D)
        return p

    @staticmethod
    def packed_size(D: int, nbits: int) -> int:
        return D * nbits // 8 if nbits in (2, 3, 4) else D


_KV_DTYPES = {torch.bfloat16: 1, torch.float16: 0, torch.float32: 2}


class PolarKVQuantizer:
    """Quantize / dequantize K or V vectors of ``head_dim`` (64, 128 or 256)
    on the GPU (reference: cache.py:180-256)."""

    def __init__(self, head_dim: int, nbits: int = 3, device: str = "cuda") -> None:
        if head_dim not in (64, 128, 256):
            raise ValueError(f"head_dim must be 64, 128 or 256 for the gfx950 kernels, got {head_dim}")
        if nbits not in (2, 3, 4):
            raise ValueError(f"nbits must be 2, 3 or 4, got {nbits}")
        self.head_dim = head_dim
        self.nbits = nbits
        self.device = torch.device(device)
        self.scale = math.sqrt(head_dim)
        self.centroids = get_centroids(nbits).to(self.device)
        self.H = build_hadamard(head_dim, str(self.device))

    def quantize(self, tensor: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """(..., head_dim) -> packed uint8 [N, head_dim*nbits/8], norms bf16 [N]."""
        from polarengine_vllm import _lib
        dev = _lib.require_device(tensor)
        flat = tensor.reshape(-1, self.head_dim)
        if flat.dtype not in _KV_DTYPES:
            flat = flat.float()
        if flat.stride(1) != 1:
            flat = flat.contiguous()
        n = flat.shape[0]
        packed = torch.empty(n, BitPacker.packed_size(self.head_dim, self.nbits),
                             dtype=torch.uint8, device=dev)
        norms = torch.empty(n, dtype=torch.bfloat16, device=dev)
        _lib.check(_lib.lib().pe_kv_quantize(flat.data_ptr(), _KV_DTYPES[flat.dtype], n,
                                             self.head_dim, flat.stride(0), self.centroids.data_ptr(),
                                             self.nbits, packed.data_ptr(), norms.data_ptr(),
                                             _lib.stream_ptr(dev)), "pe_kv_quantize")
        return packed, norms

    def dequantize(self, packed: torch.Tensor, norms: torch.Tensor,
                   shape: Tuple[int, ...], out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """packed + bf16 norms -> bf16 tensor of ``shape`` (into ``out`` if given:
        a [N, head_dim] view with 16-byte aligned rows)."""
        from polarengine_vllm import _lib
        dev = _lib.require_device(packed)
        n = packed.shape[0]
        caller_out = out is not None
        if out is None:
            out = torch.empty(n, self.head_dim, dtype=torch.bfloat16, device=dev)
        nb = norms.contiguous().to(torch.bfloat16)
        _lib.check(_lib.lib().pe_kv_dequantize(packed.contiguous().data_ptr(), nb.data_ptr(), n,
                                               self.head_dim, self.centroids.data_ptr(), self.nbits,
                                               out.data_ptr(), out.stride(0), _lib.stream_ptr(dev)),
                   "pe_kv_dequantize")
        if caller_out:
            increment_version(out)  # written through a raw pointer
        return out.reshape(shape)


class PolarKVLayer:
    """One layer's K (or V) cache: bf16 residual of the newest tokens plus the
    compressed history (reference: cache.py:263-350).

    ``update(new)`` appends ``new`` [B, H, S_new, D]; tokens beyond
    ``residual_length`` are compressed; the return value is the whole history
    [B, H, S, D] in bf16 (expanded history followed by the residual).

    By default only the codes, norms and residual persist and the history is
    expanded per call, as the reference does. ``keep_expanded=True`` keeps a
    bf16 copy of the expanded history as a read cache (each token expanded
    once), at the cost of more memory than an uncompressed cache;
    ``memory_bytes`` then counts it."""

    def __init__(self, quantizer: PolarKVQuantizer, residual_length: int = 128,
                 keep_expanded: bool = False) -> None:
        self.quantizer = quantizer
        self.residual_length = residual_length
        self.keep_expanded = keep_expanded
        self.reset()

    def reset(self) -> None:
        self._packed: Optional[torch.Tensor] = None  # [B*H, cap, RB]
        self._norms: Optional[torch.Tensor] = None   # [B*H, cap]
        self._expanded: Optional[torch.Tensor] = None  # [B*H, cap, D] bf16
        self._q_count = 0
        self.residual: Optional[torch.Tensor] = None
        self._B = self._H = self._D = None
        self._can_quantize = True

    def _grow(self, need: int) -> None:
        bh, d = self._B * self._H, self._D
        cap = 0 if self._packed is None else self._packed.shape[1]
        if need <= cap:
            return
        new_cap = max(need, 2 * cap, 64)
        dev = self.residual.device
        rb = BitPacker.packed_size(d, self.quantizer.nbits)
        packed = torch.empty(bh, new_cap, rb, dtype=torch.uint8, device=dev)
        norms = torch.empty(bh, new_cap, dtype=torch.bfloat16, device=dev)
        expanded = None
        if self.keep_expanded:
            expanded = torch.empty(bh, new_cap, d, dtype=torch.bfloat16, device=dev)
        if cap:
            packed[:, :self._q_count] = self._packed[:, :self._q_count]
            norms[:, :self._q_count] = self._norms[:, :self._q_count]
            if expanded is not None:
                expanded[:, :self._q_count] = self._expanded[:, :self._q_count]
        self._packed, self._norms, self._expanded = packed, norms, expanded

    def update(self, new_tensor: torch.Tensor) -> torch.Tensor:
        if self._B is None:
            self._B, self._H, self._D = new_tensor.shape[0], new_tensor.shape[1], new_tensor.shape[3]
            self._can_quantize = self._D == self.quantizer.head_dim and not (self._D & (self._D - 1))
        new_tensor = new_tensor.to(torch.bfloat16)
        self.residual = new_tensor if self.residual is None else torch.cat([self.residual, new_tensor], 2)
        if self._can_quantize and self.residual.shape[2] > self.residual_length:
            n_q = self.residual.shape[2] - self.residual_length
            old = self.residual[:, :, :n_q, :]
            self.residual = self.residual[:, :, n_q:, :].contiguous()
            bh = self._B * self._H
            packed, norms = self.quantizer.quantize(old.reshape(bh * n_q, self._D))
            self._grow(self._q_count + n_q)
            s0, s1 = self._q_count, self._q_count + n_q
            self._packed[:, s0:s1] = packed.view(bh, n_q, -1)
            self._norms[:, s0:s1] = norms.view(bh, n_q)
            if self._expanded is not None:
                # read cache: expand only the newly compressed tokens into it
                dst = self._expanded[:, s0:s1]
                if dst.is_contiguous():
                    self.quantizer.dequantize(packed, norms, (bh * n_q, self._D),
                                              out=dst.view(bh * n_q, self._D))
                else:
                    dst.copy_(self.quantizer.dequantize(packed, norms, (bh, n_q, self._D)))
            self._q_count = s1
        if self._q_count:
            q = self._q_count
            if self._expanded is not None:
                hist = self._expanded[:, :q]
            else:  # transient expansion of the whole compressed history
                bh = self._B * self._H
                hist = self.quantizer.dequantize(self._packed[:, :q].reshape(bh * q, -1),
                                                 self._norms[:, :q].reshape(bh * q),
                                                 (bh * q, self._D))
            hist = hist.reshape(self._B, self._H, q, self._D)
            return torch.cat([hist, self.residual], dim=2)
        return self.residual

    def compressed(self) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """The packed codes [B*H*S_q, RB] and bf16 norms [B*H*S_q] in the
        reference's order (head-major, then token)."""
        if not self._q_count:
            return None, None
        return (self._packed[:, :self._q_count].reshape(-1, self._packed.shape[2]),
                self._norms[:, :self._q_count].reshape(-1))

    def get_seq_length(self) -> int:
        return self._q_count + (self.residual.shape[2] if self.residual is not None else 0)

    def memory_bytes(self) -> int:
        """Bytes of the compressed history (codes + norms) and the residual,
        as the reference counts them, plus the expanded read cache's
        allocation when ``keep_expanded`` holds one."""
        total = 0
        if self._q_count:
            bh = self._B * self._H
            total += bh * self._q_count * self._packed.shape[2] + bh * self._q_count * 2
        if self.residual is not None:
            total += self.residual.numel() * 2
        if self._expanded is not None:
            total += self._expanded.numel() * 2
        return total


class PolarKVCache:
    """K and V caches of all layers (reference: cache.py:357-462)."""

    def __init__(self, config: PolarKVConfig, device: Optional[str] = None,
                 keep_expanded: bool = False) -> None:
        self.config = config
        device = device or ("cuda" if torch.cuda.is_available() else "cpu")
        self.quantizer = PolarKVQuantizer(config.head_dim, config.nbits, device)
        self.k_layers = []
        self.v_layers = []
        for i in range(config.num_layers):
            skip = i in config.skip_layers
            mk = lambda: PolarKVLayer(self.quantizer, config.residual_length, keep_expanded)
            self.k_layers.append(None if skip else mk())
            self.v_layers.append(None if skip else mk())
        self._seen_tokens = 0

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor,
               layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[2]
        k, v = self.k_layers[layer_idx], self.v_layers[layer_idx]
        if k is None:  # skipped layer: the caller keeps its own K/V
            return key_states, value_states
        return k.update(key_states), v.update(value_states)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        k = self.k_layers[layer_idx]
        return 0 if k is None else k.get_seq_length()

    def memory_bytes(self) -> int:
        return sum(k.memory_bytes() + v.memory_bytes()
                   for k, v in zip(self.k_layers, self.v_layers) if k is not None)

    def memory_mb(self) -> float:
        return self.memory_bytes() / (1024 * 1024)

    def reset(self) -> None:
        for k, v in zip(self.k_layers, self.v_layers):
            if k is not None:
                k.reset()
                v.reset()
        self._seen_tokens = 0

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    def stats(self) -> dict:
        fp16 = (self.config.num_layers * 2 * self.config.num_kv_heads * self.config.head_dim
                * self.get_seq_length() * 2)
        actual = self.memory_bytes()
        return {"seq_length": self.get_seq_length(), "memory_mb": self.memory_mb(),
                "fp16_memory_mb": fp16 / (1024 * 1024),
                "compression_ratio": fp16 / max(actual, 1), "seen_tokens": self._seen_tokens}
