"""PolarQuant KV-cache compression (reference: polarengine_vllm/kv_cache).

Q2/Q3/Q4 K/V compression with the Hadamard rotation and the KV Lloyd-Max
codebook; quantize and dequantize run as single HIP kernels on the GPU.

    from polarengine_vllm.kv_cache import PolarKVConfig, PolarKVCache
    cache = PolarKVCache(PolarKVConfig(nbits=3, head_dim=128, num_layers=32))
    k_all, v_all = cache.update(k_new, v_new, layer_idx)
"""

from .attention import PolarKVAttentionWrapper, patch_model_attention
from .cache import BitPacker, PolarKVCache, PolarKVLayer, PolarKVQuantizer, get_centroids
from .config import PolarKVConfig

__all__ = ["PolarKVConfig", "PolarKVCache", "PolarKVQuantizer", "PolarKVLayer",
           "PolarKVAttentionWrapper", "patch_model_attention", "BitPacker", "get_centroids"]
