"""CPU tests of the product's host logic: codebook, bit rules, packing
formats (CPU path), quantizer, config and the FWHT cache. Mirrors the
reference suites tests/test_utils.py, test_packing.py, test_config.py and
the cache part of test_fwht.py."""

import math

import numpy as np
import pytest
import torch

import polar_oracle as O
from polarengine_vllm import packing, utils
from polarengine_vllm.config import PolarQuantConfig
from polarengine_vllm.kernels.fwht import FWHTCache, build_hadamard
from polarengine_vllm.quantizer import PolarQuantizer


# ---- codebook ---------------------------------------------------------------

@pytest.mark.parametrize("bits", range(2, 9))
def test_centroids_bit_exact_vs_reference(golden, bits):
    assert np.array_equal(utils.get_centroids(bits).numpy(), golden[f"centroids_b{bits}"])


def test_centroid_cache_and_range():
    assert utils.get_centroids(4).data_ptr() == utils.get_centroids(4).data_ptr()
    with pytest.raises(ValueError, match="bits must be in"):
        utils.get_centroids(1)
    with pytest.raises(ValueError, match="bits must be in"):
        utils.get_centroids(9)


def test_convergence_200_vs_300():
    a = utils.compute_lloyd_max_centroids(16, n_iter=200)
    b = utils.compute_lloyd_max_centroids(16, n_iter=300)
    assert torch.allclose(a, b, atol=0.01)


# ---- bit rules (reference tests/test_utils.py:98-201) -------------------------

def test_bit_rules():
    g = utils.get_bits_for_layer
    v, w = torch.randn(4096), torch.randn(4096, 4096)
    assert g("model.layers.0.input_layernorm.weight", v) == 16
    assert g("model.layers.0.self_attn.q_proj.bias", v) == 16
    assert g("model.layers.0.conv1d.weight", torch.randn(128, 128)) == 16
    assert g("model.layers.0.block_sparse_moe.router.weight", torch.randn(64, 4096)) == 16
    assert g("model.layers.0.block_sparse_moe.gate.weight", torch.randn(8, 4096)) == 16
    for name, bits in [("q_proj", 5), ("k_proj", 5), ("v_proj", 5), ("o_proj", 6),
                       ("gate_proj", 3), ("up_proj", 3), ("down_proj", 4)]:
        assert g(f"model.layers.0.x.{name}.weight", w) == bits
    assert g("model.layers.0.mlp.gate_up_proj.weight", torch.randn(24576, 4096)) == 3
    assert g("model.embed_tokens.weight", torch.randn(1000, 4096)) == 5
    assert g("lm_head.weight", torch.randn(1000, 4096)) == 6
    assert g("model.layers.0.self_attn.q_proj.weight", torch.randn(8, 8)) == 16
    assert g("some_scalar", torch.tensor(1.0)) == 16
    assert g("model.layers.0.self_attn.q_proj.weight", w, {"q_proj": 3}) == 3
    assert g("model.layers.0.some_unknown_proj.weight", w) == 5
    assert g("model.layers.0.dt_bias", torch.randn(128, 128)) == 16
    assert g("model.layers.0.mamba.D", torch.randn(128, 128)) == 16


# ---- packing, CPU path -------------------------------------------------------

def test_nibble_pack_matches_oracle_and_kats(golden):
    c = torch.from_numpy(golden["pack_codes16"])
    assert np.array_equal(packing.pack_codes_half_block(c).numpy(), golden["pack_nibble"])
    codes = torch.zeros(128, 512, dtype=torch.int8)
    codes.view(128, -1, 128)[:, :, :64] = 3
    codes.view(128, -1, 128)[:, :, 64:] = 12
    assert (packing.pack_codes_half_block(codes) == 0xC3).all()
    rng = np.random.default_rng(0)
    r = torch.from_numpy(rng.integers(0, 16, (64, 1024)).astype(np.int8))
    assert np.array_equal(packing.pack_codes_half_block(r).numpy(), O.pack_nibble(r.numpy()))
    assert packing.verify_packing_roundtrip(r)
    for bs in (32, 64, 128, 256):
        rr = r[:, : bs * 4]
        assert torch.equal(packing.unpack_codes_half_block(packing.pack_codes_half_block(rr, bs), bs), rr)
    with pytest.raises(AssertionError):
        packing.pack_codes_half_block(torch.full((1, 128), 16, dtype=torch.int8))


def test_q5_and_hlwq_match_golden(golden):
    c = torch.from_numpy(golden["pack_codes32"])
    assert np.array_equal(packing.pack_codes_q5(c).numpy(), golden["pack_q5"])
    assert torch.equal(packing.unpack_codes_q5(packing.pack_codes_q5(c)), c)
    assert np.array_equal(packing.pack_codes_q5_hlwq(c).numpy(), golden["pack_q5_hlwq"])
    odd = torch.from_numpy(golden["pack_codes32_odd"])
    assert np.array_equal(packing.pack_codes_q5_hlwq(odd).numpy(), golden["pack_q5_hlwq_odd"])
    assert torch.equal(packing.unpack_codes_q5_hlwq(packing.pack_codes_q5_hlwq(odd), odd.shape[1]), odd)
    assert packing.verify_packing_roundtrip_q5(c)


def test_pack_model_codes():
    class Fake(torch.nn.Module):
        def __init__(self, n, k, bits):
            super().__init__()
            self.bits = bits
            self.register_buffer("codes", torch.randint(0, 16, (n, k), dtype=torch.int8))

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.a, self.b, self.c = Fake(64, 256, 3), Fake(32, 256, 4), Fake(32, 256, 5)

    m = Model()
    st = packing.pack_model_codes(m)
    assert st["layers_packed"] == 2 and st["saved_gb"] > 0
    assert m.a._codes_packed and m.b._codes_packed and not getattr(m.c, "_codes_packed", False)


# ---- quantizer ----------------------------------------------------------------

@pytest.mark.parametrize("bits", range(2, 7))
def test_quantizer_matches_reference_golden(golden, bits):
    q = PolarQuantizer(128).quantize_tensor(torch.from_numpy(golden["quant_w"]), bits)
    assert np.array_equal(q["codes"].numpy(), golden[f"quant_codes_b{bits}"])
    assert np.array_equal(q["norms"].numpy(), golden[f"quant_norms_b{bits}"])
    assert np.array_equal(q["ct_scaled"].numpy(), golden[f"quant_ct_scaled_b{bits}"])


def test_hadamard_builder_matches_golden(golden):
    assert np.array_equal(build_hadamard(128).numpy(), golden["hadamard128"])
    with pytest.raises(AssertionError):
        build_hadamard(3)


# ---- config (reference tests/test_config.py) ----------------------------------

def test_config_parse_and_resolve(sample_polar_config):
    c = PolarQuantConfig.from_config(sample_polar_config)
    assert c.block_size == 128 and len(c.layers_meta) == 5
    assert c._resolve_bits("model.layers.0.self_attn.q_proj") == 5
    assert c._resolve_bits("model.layers.0.self_attn.o_proj") == 6
    assert c._resolve_bits("model.layers.5.self_attn.q_proj") == 5
    assert c._resolve_bits("model.layers.5.mlp.down_proj") == 4
    assert c._resolve_bits("model.layers.0.some_unknown_layer") is None
    c2 = PolarQuantConfig.from_config({"bit_assignment": {"proj": 3, "gate_proj": 4,
                                                          "mlp.gate_proj": 5}})
    assert c2._resolve_bits("model.layers.0.mlp.gate_proj") == 5
    d = PolarQuantConfig.from_config({})
    assert d.block_size == 128 and d.bit_assignment == {} and d.layers_meta == {}
    assert PolarQuantConfig.get_name() == "polarengine"
    assert PolarQuantConfig.get_config_filenames() == ["polar_config.json"]
    assert torch.float16 in PolarQuantConfig.get_supported_act_dtypes()
    assert PolarQuantConfig.get_min_capability() == 70
    assert "128-wide blocks" in repr(c) and "[3, 4, 5, 6]" in repr(c)


def test_get_quant_method(sample_polar_config):
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    c = PolarQuantConfig.from_config(sample_polar_config)
    m = c.get_quant_method(torch.nn.Linear(128, 128), "model.layers.0.self_attn.q_proj")
    assert isinstance(m, PolarQuantLinearMethod) and m.bits == 5 and m.block_size == 128
    empty = PolarQuantConfig.from_config({"bit_assignment": {}, "layers": {}})
    assert empty.get_quant_method(torch.nn.Linear(128, 128), "model.layers.99.x") is None


def test_create_weights_layout():
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    layer = torch.nn.Module()
    PolarQuantLinearMethod(128, 3).create_weights(layer, 200, [64, 32], 200, 96, torch.float16)
    assert layer.codes.shape == (96, 256) and layer.codes.dtype == torch.int8
    assert layer.norms.shape == (96, 2) and layer.norms.dtype == torch.float16
    assert layer.ct_scaled.dtype == torch.float32
    np.testing.assert_array_equal(layer.ct_scaled.numpy(),
                                  (utils.get_centroids(3) / math.sqrt(128)).numpy())
    assert layer.codes.output_dim == 0 and layer.codes.input_dim == 1


# ---- FWHT cache (reference tests/test_fwht.py:115-180) ------------------------

def test_fwht_cache_semantics():
    cache = FWHTCache()
    x, y = torch.randn(32, 128), torch.randn(32, 128)
    r = torch.randn(32, 128)
    assert cache.get(x, 128) is None
    cache.put(x, 128, r)
    assert cache.get(x, 128) is r
    assert cache.get(x, 64) is None
    assert cache.get(y, 128) is None
    cache.put(y, 128, r)
    assert cache.get(x, 128) is None and cache.get(y, 128) is r
    y.add_(1.0)  # in-place update must invalidate
    assert cache.get(y, 128) is None
    cache.put(x, 128, r)
    cache.clear()
    assert cache.get(x, 128) is None


def test_fwht_cache_inference_tensors_need_a_scope():
    """Inference tensors (vLLM runs every forward under inference_mode) have
    no version counter: put/get must not touch it, and outside a scope the
    cache never serves them (a hidden state updated in place between layers
    would otherwise get the previous layer's transform)."""
    cache = FWHTCache()
    r = torch.randn(4, 128)
    with torch.inference_mode():
        x = torch.randn(4, 128)
        cache.put(x, 128, r)          # must not raise
        assert cache.get(x, 128) is None
        cache.enter_scope()
        cache.put(x, 128, r)
        assert cache.get(x, 128) is r
        cache.exit_scope()            # the scope's end drops the transform
        assert cache.get(x, 128) is None


def test_fwht_cache_entry_dies_with_its_tensor():
    """The cache holds x weakly: once x is freed the entry and its transform
    go, and a new tensor at the same address misses."""
    import gc
    import weakref
    cache = FWHTCache()
    x, r = torch.randn(8, 128), torch.randn(8, 128)
    cache.put(x, 128, r)
    rref = weakref.ref(r)
    del r, x
    gc.collect()
    assert cache._result is None and rref() is None
    y = torch.randn(8, 128)
    assert cache.get(y, 128) is None


def test_fwht_cache_scope_hooks_share_inside_one_forward():
    """install_fwht_cache_hooks: siblings inside one parent forward share the
    transform under inference_mode; the parent's forward end releases it."""
    from polarengine_vllm.linear_method import PolarQuantLinearMethod, install_fwht_cache_hooks
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE
    method = PolarQuantLinearMethod(128, 4)
    seen = []

    class Proj(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.quant_method = method

        def forward(self, t):
            hit = GLOBAL_FWHT_CACHE.get(t, 128)
            if hit is None:
                GLOBAL_FWHT_CACHE.put(t, 128, t * 2)
            seen.append(hit is not None)
            return t

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q, self.k, self.v = Proj(), Proj(), Proj()

        def forward(self, t):
            return self.q(t) + self.k(t) + self.v(t)

    blk = Block()
    assert install_fwht_cache_hooks(blk) == 1
    assert install_fwht_cache_hooks(blk) == 0  # idempotent
    with torch.inference_mode():
        h = torch.randn(2, 128)
        blk(h)
        assert seen == [False, True, True]
        assert GLOBAL_FWHT_CACHE.get(h, 128) is None and GLOBAL_FWHT_CACHE._result is None
        h.add_(1.0)   # in place, untracked: the next forward starts empty anyway
        blk(h)
        assert seen[3:] == [False, True, True]


def test_workspace_growth_keeps_old_buffers():
    """A workspace that grows keeps every earlier buffer alive: a graph
    captured earlier still writes through their raw pointers."""
    from polarengine_vllm import _lib
    dev = torch.device("cpu")
    key = _lib._ws_key(dev)
    _lib._WS_CACHE.pop(key, None)
    _lib._WS_RETIRED.pop(key, None)
    a = _lib.workspace(dev, 100)
    assert a.numel() >= 100 and int(a.sum()) == 0
    assert _lib.workspace(dev, 50) is a
    b = _lib.workspace(dev, a.numel() + 1)
    assert b is not a and b.numel() >= 2 * a.numel()
    assert _lib._WS_RETIRED[key] == [a]
    c = _lib.workspace(dev, b.numel() + 1)
    assert _lib._WS_RETIRED[key] == [a, b] and c.numel() >= 2 * b.numel()
    _lib._WS_CACHE.pop(key, None)
    _lib._WS_RETIRED.pop(key, None)


def test_fwht_butterfly_is_gpu_only_and_checks_length():
    """fwht_butterfly (reference kernels/fwht.py:160-190) asserts a
    power-of-two last dimension and has no CPU path."""
    from polarengine_vllm.kernels.fwht import fwht_butterfly
    with pytest.raises(AssertionError):
        fwht_butterfly(torch.randn(2, 96))
    with pytest.raises(RuntimeError, match="GPU only"):
        fwht_butterfly(torch.randn(2, 64))


def test_fwht_clear_hook_as_forward_pre_hook():
    """create_fwht_clear_hook (reference linear_method.py:265-288): a forward
    pre-hook that empties the method's cache before the module runs."""
    from polarengine_vllm.linear_method import PolarQuantLinearMethod, create_fwht_clear_hook
    method = PolarQuantLinearMethod(128, 4)
    x, r = torch.randn(4, 128), torch.randn(4, 128)
    method._fwht_cache.put(x, 128, r)
    seen = []

    class Block(torch.nn.Module):
        def forward(self, t):
            seen.append(method._fwht_cache.get(x, 128))
            return t

    blk = Block()
    blk.register_forward_pre_hook(create_fwht_clear_hook(method))
    blk(x)
    assert seen == [None]  # cleared before the forward ran
    method._fwht_cache.clear()


def test_custom_ops_registered_with_fake_shapes():
    """The linear and MoE forwards are torch custom ops whose fake
    implementations give the output's shape and dtype without running a
    kernel (what torch.compile traces)."""
    import polarengine_vllm.linear_method  # noqa: F401  (registers the ops)
    import polarengine_vllm.moe_method  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(3, 5, 256, dtype=torch.bfloat16)
        codes = torch.empty(96, 128, dtype=torch.uint8)
        y = torch.ops.polarengine.linear_apply(x, codes, torch.empty(96, 2, dtype=torch.float16),
                                               torch.empty(16), None, 4, 3, 256, 256, 96, [])
        assert y.shape == (3, 5, 96) and y.dtype == torch.bfloat16
        y32 = torch.ops.polarengine.linear_apply(x.float(), codes, torch.empty(96, 2), torch.empty(16),
                                                 None, 4, 3, 256, 256, 96, [])
        assert y32.dtype == torch.float16
        xm = torch.empty(7, 256, dtype=torch.float16)
        w = [torch.empty(1)] * 6
        out = torch.ops.polarengine.moe_routed(xm, torch.empty(7, 8), None, *w, [2, 1, 0, 0, 0],
                                               [3, 1, 4, 1, 8, 256, 128])
        assert out.shape == xm.shape and out.dtype == xm.dtype
        out = torch.ops.polarengine.moe_given(xm, torch.empty(7, 2), torch.empty(7, 2, dtype=torch.int32),
                                              *w, [3, 1, 4, 1, 8, 256, 128])
        assert out.shape == xm.shape
