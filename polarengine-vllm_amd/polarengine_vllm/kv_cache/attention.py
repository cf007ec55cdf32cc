"""KV-cache hooks for attention (reference: kv_cache/attention.py).

``PolarKVAttentionWrapper`` exposes a PolarKVCache through the transformers
``Cache.update`` interface and wraps a vLLM-style attention forward so that
new K/V are compressed and the attention reads the expanded history.
``patch_model_attention`` tags a model's attention modules with their layer
index and the cache."""

from __future__ import annotations

from typing import Any, Callable, Optional, Tuple

import torch

from .cache import PolarKVCache
from .config import PolarKVConfig


class PolarKVAttentionWrapper:
    def __init__(self, cache: PolarKVCache) -> None:
        self.cache = cache
        self.config = cache.config

    # transformers Cache interface
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: Optional[dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.cache.update(key_states, value_states, layer_idx)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.cache.get_seq_length(layer_idx)

    def get_max_cache_shape(self) -> None:
        return None

    @property
    def seen_tokens(self) -> int:
        return self.cache.seen_tokens

    @property
    def is_initialized(self) -> bool:
        return self.cache.seen_tokens > 0

    def wrap_attention_forward(self, original_forward: Callable[..., torch.Tensor],
                               layer_idx: int) -> Callable[..., torch.Tensor]:
        """A forward that compresses the new K/V ([tokens, heads, D] as vLLM
        passes them, or [B, H, S, D]) and calls ``original_forward`` with the
        whole history in the same layout."""
        cache = self.cache

        def wrapped_forward(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                            kv_cache: Any, attn_metadata: Any, **kwargs: Any) -> torch.Tensor:
            flat = key.dim() == 3
            k4 = key.unsqueeze(0).transpose(1, 2) if flat else key
            v4 = value.unsqueeze(0).transpose(1, 2) if flat else value
            full_k, full_v = cache.update(k4, v4, layer_idx)
            if flat:
                full_k = full_k.squeeze(0).transpose(0, 1)
                full_v = full_v.squeeze(0).transpose(0, 1)
            return original_forward(query, full_k, full_v, kv_cache, attn_metadata, **kwargs)

        return wrapped_forward


def patch_model_attention(model: torch.nn.Module, config: PolarKVConfig) -> PolarKVCache:
    """Tag the attention modules (names containing self_attn / attention /
    attn that own a q_proj or qkv_proj) with ``_polar_kv_layer_idx`` and
    ``_polar_kv_cache``, in module order, up to ``config.num_layers``."""
    cache = PolarKVCache(config)
    idx = 0
    for name, module in model.named_modules():
        if any(p in name for p in ("self_attn", "attention", "attn")) and (
                hasattr(module, "q_proj") or hasattr(module, "qkv_proj")):
            if idx < config.num_layers:
                module._polar_kv_layer_idx = idx
                module._polar_kv_cache = cache
                idx += 1
    return cache
