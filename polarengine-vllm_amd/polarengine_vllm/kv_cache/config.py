"""Configuration of the PolarQuant KV cache (reference: kv_cache/config.py)."""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List


@dataclass
class PolarKVConfig:
    """nbits 2..4; the newest ``residual_length`` tokens stay in bf16; head_dim
    a power of 2 (the gfx950 kernels take 64, 128 and 256); ``skip_layers``
    keep uncompressed K/V (reference: kv_cache/config.py:10-96)."""

    nbits: int = 3
    residual_length: int = 128
    head_dim: int = 128
    num_kv_heads: int = 8
    num_layers: int = 32
    enabled: bool = True
    skip_layers: List[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        if self.nbits not in (2, 3, 4):
            raise AssertionError(f"KV codes are 2, 3 or 4 bits wide (nbits={self.nbits})")
        if self.head_dim <= 0:
            raise AssertionError(f"head_dim has to be at least 1 (head_dim={self.head_dim})")
        if self.head_dim & (self.head_dim - 1):
            raise ValueError(f"the KV rotation is a Hadamard transform over the whole head, so "
                             f"head_dim must be a power of 2 (head_dim={self.head_dim})")

    @property
    def compression_ratio(self) -> float:
        """Theoretical ratio against fp16 (norms not counted)."""
        return 16.0 / self.nbits

    @property
    def n_levels(self) -> int:
        return 1 << self.nbits

    def bytes_per_token(self, fp16: bool = False) -> float:
        """Bytes of K and V per token per layer: codes plus one bf16 norm per
        vector (or plain fp16)."""
        if fp16:
            return self.num_kv_heads * self.head_dim * 2 * 2
        return self.num_kv_heads * (self.head_dim * self.nbits / 8 + 2) * 2

    def max_context(self, budget_gb: float) -> int:
        """Tokens that fit a KV budget of ``budget_gb`` GiB over all layers."""
        return int(budget_gb * 1024 ** 3 / (self.bytes_per_token() * self.num_layers))

    @classmethod
    def for_gemma4_31b(cls, nbits: int = 3) -> "PolarKVConfig":
        return cls(nbits=nbits, head_dim=256, num_kv_heads=16, num_layers=60)

    # model shapes of the presets: (head_dim, num_kv_heads, num_layers)
    _LLAMA3 = {"8b": (128, 8, 32), "70b": (128, 8, 80)}
    _QWEN35 = {"9b": (128, 8, 48), "27b": (128, 4, 48)}

    @classmethod
    def for_llama3(cls, nbits: int = 3, size: str = "8b") -> "PolarKVConfig":
        d, h, n = cls._LLAMA3[size]
        return cls(nbits=nbits, head_dim=d, num_kv_heads=h, num_layers=n)

    @classmethod
    def for_qwen35(cls, nbits: int = 3, size: str = "9b") -> "PolarKVConfig":
        d, h, n = cls._QWEN35[size]
        return cls(nbits=nbits, head_dim=d, num_kv_heads=h, num_layers=n)
