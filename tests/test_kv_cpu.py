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
    # patching again re-points the backends at the new cache: the original
    # forward is wrapped once more, never the earlier wrapper
    orig = [blk.attn._polar_kv_orig_forward for blk in vmodel]
    vcache2 = patch_model_attention(vmodel, PolarKVConfig(num_layers=3))
    for i, blk in enumerate(vmodel):
        assert blk.attn._polar_kv_cache is vcache2
        assert blk.attn._polar_kv_orig_forward is orig[i]
        inner = blk.attn.forward.__closure__
        cells = [c.cell_contents for c in inner]
        assert orig[i] in cells and not any(getattr(c, "__name__", "") == "wrapped_forward"
                                            for c in cells if callable(c))


def _count_codes(r, ct):
    mid = ((ct[:-1] + ct[1:]) * np.float32(0.5)).astype(np.float32)
    return (r[:, None] > mid[None, :]).sum(1)


def _cell_codes(r, ct):
    """The quantize kernel's count by cell (pe_kv.hip, kv_cells_setup and
    the loop after it), restated on float32 numpy: power-of-two cells of
    width w over [-32 w, 32 w) with every midpoint in [-31 w, 31 w] and at
    most one per cell; code = midpoints below r's cell + (r > the cell's
    midpoint), on t = r / w."""
    mid = ((ct[:-1] + ct[1:]) * np.float32(0.5)).astype(np.float32)
    amax = np.float32(np.abs(mid).max())
    _, e = np.frexp(amax / np.float32(31))
    w = np.float32(np.ldexp(1.0, int(e)))
    if np.float32(31) * w < amax:
        w = np.float32(w * 2)
    assert w <= np.diff(mid).min()  # the table path applies to these codebooks
    inv_w = np.float32(1) / w
    lo = np.zeros(64, np.int64)
    tm = np.full(64, np.inf, np.float32)
    for c in range(64):
        b = np.float32((c - 32) * w)
        lo[c] = 0 if c == 0 else int((mid < b).sum())
        for m in mid:
            if m >= b and (c == 63 or m < b + w):
                tm[c] = np.float32(m * inv_w)
    t = (r * inv_w).astype(np.float32)
    with np.errstate(invalid="ignore"):
        cl = np.fmin(np.fmax(t, np.float32(-32)), np.float32(31))  # fmax: NaN -> -32
        cell = np.floor(cl).astype(np.int64) + 32
        return lo[cell] + (t > tm[cell])


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_kv_cell_count_equals_midpoint_count(bits):
    """Pins the quantize kernel's one-compare code against the count of
    midpoints below r on the values where an off-by-one would show: every
    midpoint and its float neighbours, every cell boundary and its
    neighbours, 0, +-inf, NaN, tiny and huge values, and random normals."""
    ct = get_centroids(bits).numpy().astype(np.float32)
    mid = ((ct[:-1] + ct[1:]) * np.float32(0.5)).astype(np.float32)
    amax = np.float32(np.abs(mid).max())
    _, e = np.frexp(amax / np.float32(31))
    w = np.float32(np.ldexp(1.0, int(e)))
    if np.float32(31) * w < amax:
        w = np.float32(w * 2)
    bounds = (np.arange(-33, 34) * w).astype(np.float32)
    pts = np.concatenate([mid, bounds, np.array([0, -0.0, 1e-30, -1e-30, 1e30, -1e30], np.float32)])
    near = np.concatenate([np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(-np.inf))])
    rng = np.random.default_rng(bits)
    r = np.concatenate([pts, near, rng.standard_normal(200000).astype(np.float32) * 1.5,
                        np.array([np.inf, -np.inf], np.float32)]).astype(np.float32)
    np.testing.assert_array_equal(_cell_codes(r, ct), _count_codes(r, ct))
    # NaN: code 0, as the count gives
    assert _cell_codes(np.array([np.nan], np.float32), ct)[0] == 0 == _count_codes(np.array([np.nan], np.float32), ct)[0]
