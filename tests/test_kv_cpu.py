"""CPU tests of the KV-cache path: the oracle against the reference's golden
vectors (tests/golden/golden_kv.npz), the bit orders by hand-computed bytes,
the product's host-side pieces (codebook, BitPacker, config) and the absence
of a CPU compute path (reference: kv_cache/cache.py, config.py)."""

import numpy as np
import pytest
import torch

import polar_oracle as O
from polarengine_vllm.kv_cache import BitPacker, PolarKVConfig, PolarKVQuantizer, get_centroids


@pytest.fixture(scope="module")
def gkv():
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_kv.npz"))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_oracle_centroids_and_pack_match_golden(gkv, bits):
    assert np.array_equal(O.kv_centroids(bits), gkv[f"kv_centroids_b{bits}"])
    codes = gkv["kv_pack_codes"].astype(np.int64) % (1 << bits)
    assert np.array_equal(O.kv_pack(codes, bits), gkv[f"kv_pack_b{bits}"])
    assert np.array_equal(O.kv_unpack(gkv[f"kv_pack_b{bits}"], bits, 128), codes)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_oracle_quantize_dequantize_match_golden(gkv, d, bits):
    x = O.bf16_bits_to_f32(gkv[f"kv_x_d{d}"])
    packed, norms = O.kv_quantize(x, bits)
    assert np.array_equal(packed, gkv[f"kv_packed_d{d}_b{bits}"])
    assert np.array_equal(norms, gkv[f"kv_norms_d{d}_b{bits}"])
    deq = O.kv_dequantize(gkv[f"kv_packed_d{d}_b{bits}"], gkv[f"kv_norms_d{d}_b{bits}"], bits, d)
    assert np.array_equal(deq, gkv[f"kv_deq_d{d}_b{bits}"])


def test_pack_bit_orders_hand_computed():
    # 2 bits, MSB first: 01 10 11 00
    assert O.kv_pack(np.array([[1, 2, 3, 0]]), 2)[0, 0] == 0x6C
    # 3 bits, 8 codes 1..7,0 -> 001 010 011 100 101 110 111 000
    assert list(O.kv_pack(np.array([[1, 2, 3, 4, 5, 6, 7, 0]]), 3)[0]) == [0x29, 0xCB, 0xB8]
    # 4 bits: the even-indexed code in the HIGH nibble (weights do the reverse)
    assert O.kv_pack(np.array([[1, 2]]), 4)[0, 0] == 0x12
    assert O.pack_nibble(np.r_[np.full(64, 1), np.full(64, 2)][None])[0, 0] == 0x21


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_product_host_pieces(gkv, bits):
    assert np.array_equal(get_centroids(bits).numpy(), gkv[f"kv_centroids_b{bits}"])
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (5, 256))
    p = BitPacker.pack(torch.from_numpy(codes), bits)
    assert np.array_equal(p.numpy(), O.kv_pack(codes, bits))
    assert np.array_equal(BitPacker.unpack(p, bits, 256).numpy(), codes)
    assert BitPacker.packed_size(128, bits) == 128 * bits // 8


def test_config():
    c = PolarKVConfig(nbits=3, head_dim=128, num_kv_heads=8, num_layers=32)
    assert c.n_levels == 8 and c.compression_ratio == pytest.approx(16 / 3)
    assert c.bytes_per_token() == pytest.approx(8 * (128 * 3 / 8 + 2) * 2)
    assert c.bytes_per_token(fp16=True) == 8 * 128 * 4
    assert c.max_context(1.0) == int(1024 ** 3 / (c.bytes_per_token() * 32))
    assert PolarKVConfig.for_gemma4_31b().head_dim == 256
    with pytest.raises(AssertionError, match="nbits"):
        PolarKVConfig(nbits=5)
    with pytest.raises(ValueError, match="power of 2"):
        PolarKVConfig(head_dim=96)


def test_no_cpu_compute_path():
    q = PolarKVQuantizer(128, 3, device="cpu")
    with pytest.raises(RuntimeError, match="GPU only"):
        q.quantize(torch.zeros(4, 128))
    with pytest.raises(ValueError, match="head_dim"):
        PolarKVQuantizer(96, 3, device="cpu")


def test_presets_and_patch_model_attention():
    from polarengine_vllm.kv_cache import patch_model_attention
    assert PolarKVConfig.for_llama3(size="70b").num_layers == 80
    assert PolarKVConfig.for_qwen35(2, "27b").num_kv_heads == 4

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = torch.nn.Identity()

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = Attn()
            self.mlp = torch.nn.Identity()

    model = torch.nn.Module()
    model.layers = torch.nn.ModuleList([Block() for _ in range(3)])
    cfg = PolarKVConfig(num_layers=2)
    cache = patch_model_attention(model, cfg)
    assert [getattr(b.self_attn, "_polar_kv_layer_idx", None) for b in model.layers] == [0, 1, None]
    assert model.layers[0].self_attn._polar_kv_cache is cache

    # vLLM-style attention backends: their forward is wrapped (not called here:
    # the cache's kernels need a GPU)
    class Backend(torch.nn.Module):
        def forward(self, query, key, value, kv_cache, attn_metadata, **kw):
            return query

    class VBlock(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.qkv_proj = torch.nn.Identity()
            self.attn = Backend()

    vmodel = torch.nn.ModuleList([VBlock() for _ in range(3)])
    vcache = patch_model_attention(vmodel, PolarKVConfig(num_layers=3))
    for i, blk in enumerate(vmodel):
        assert blk.attn._polar_kv_layer_idx == i and blk.attn._polar_kv_cache is vcache
        assert blk.attn.forward.__name__ == "wrapped_forward"
        assert not hasattr(blk, "_polar_kv_layer_idx")  # the backends were found, not the blocks
