"""KV-cache hooks for attention (reference: kv_cache/attention.py).

``PolarKVAttentionWrapper`` exposes a PolarKVCache through the transformers
``Cache.update`` interface and wraps a vLLM-style attention forward so that
new K/V are compressed and the attention reads the expanded history.
``patch_model_attention`` wraps a model's attention backends (or tags its
attention blocks) with the cache."""

from __future__ import annotations

import inspect
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


def _backend_forward(module: torch.nn.Module) -> bool:
    """True for an attention backend: its forward takes (query, key, value,
    kv_cache, attn_metadata), the call the wrapper intercepts."""
    fwd = getattr(module, "forward", None)
    try:
        names = list(inspect.signature(fwd).parameters)[:5]
    except (TypeError, ValueError):
        return False
    return names == ["query", "key", "value", "kv_cache", "attn_metadata"]


def patch_model_attention(model: torch.nn.Module, config: PolarKVConfig) -> PolarKVCache:
    """Give a model a PolarKVCache and return it.

    Attention backends (modules whose forward takes query, key, value,
    kv_cache, attn_metadata: vLLM's per-layer attention) get that forward
    replaced by ``wrap_attention_forward``, so their new K/V are compressed
    and the whole history is what they attend to; they are numbered in
    module order, up to ``config.num_layers``. A model without such backends
    (transformers attention blocks, which take the cache through
    ``past_key_values``, where ``PolarKVAttentionWrapper`` itself serves)
    has its attention blocks, the modules owning a q_proj or qkv_proj, tagged
    with ``_polar_kv_layer_idx`` / ``_polar_kv_cache`` in the same order, as
    the reference's hook does (kv_cache/attention.py:128-155). Patching a
    model again re-points every backend at the new cache (its original
    forward is kept, so wrappers never stack)."""
    cache = PolarKVCache(config)
    wrapper = PolarKVAttentionWrapper(cache)
    backends = [m for m in model.modules() if _backend_forward(m)]
    targets = backends or [m for m in model.modules()
                           if hasattr(m, "q_proj") or hasattr(m, "qkv_proj")]
    for idx, module in enumerate(targets[:config.num_layers]):
        if backends:
            # a backend patched before is re-pointed at the new cache: its
            # original forward is wrapped again, never the earlier wrapper
            orig = getattr(module, "_polar_kv_orig_forward", None) or module.forward
            module._polar_kv_orig_forward = orig
            module.forward = wrapper.wrap_attention_forward(orig, idx)
        module._polar_kv_layer_idx = idx
        module._polar_kv_cache = cache
    return cache
