"""CPU tests of the checkpoint loader (reference: polarengine_vllm/loader.py):
config and weight-map parsing, every stored code layout, bit resolution,
packed detection, TP sharding and the merged-shard weight loader. The
checkpoints are written by tests/ckpt_fixture.py from the oracle quantizer."""

import json
import logging
import os

import numpy as np
import pytest
import torch

import polar_oracle as O
from ckpt_fixture import write_hlwq_checkpoint, write_split_checkpoint
from polarengine_vllm import loader as LD
from polarengine_vllm.linear_method import PolarQuantLinearMethod


@pytest.fixture(scope="module")
def split_ckpt(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("split"))
    return root, write_split_checkpoint(root)


@pytest.fixture(scope="module")
def hlwq_ckpt(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("hlwq"))
    return root, write_hlwq_checkpoint(root)


def test_load_polar_config(split_ckpt, tmp_path, caplog):
    root, _ = split_ckpt
    cfg = LD.load_polar_config(root)
    assert cfg["format"] == "polar_engine_v4" and cfg["block_size"] == 128
    with pytest.raises(FileNotFoundError, match="no polar_config.json"):
        LD.load_polar_config(str(tmp_path))
    (tmp_path / "polar_config.json").write_text(json.dumps({"format": "mystery"}))
    with caplog.at_level(logging.WARNING):
        assert LD.load_polar_config(str(tmp_path))["format"] == "mystery"
    assert "not one this loader knows" in caplog.text


def test_weight_map_index_and_scan(split_ckpt, hlwq_ckpt, tmp_path):
    root, info = split_ckpt
    wm = LD.get_weight_map(root)
    assert wm["model.layers.0.self_attn.q_proj.codes"] == "model-00001-of-00002.safetensors"
    assert wm["model.layers.0.self_attn.k_proj.codes"] == "model-00002-of-00002.safetensors"
    assert len(wm) == sum(4 if i["kind"] == "nibble_bias" else 3 for i in info.values()) + 2
    hroot, _ = hlwq_ckpt
    wm2 = LD.get_weight_map(hroot)  # no index: scanned
    assert set(wm2.values()) == {"model.safetensors"}
    with pytest.raises(FileNotFoundError, match="safetensors shard"):
        LD.get_weight_map(str(tmp_path))


def test_layer_weights_every_stored_layout(split_ckpt):
    root, info = split_ckpt
    cfg = LD.load_polar_config(root)
    with LD.PolarWeightLoader(root, cfg, device="cpu") as ld:
        for name, q in info.items():
            w = ld.load_layer_weights(name)
            if q["kind"].startswith("nibble"):
                # stored nibbles come back as stored (unpacked later on the GPU)
                assert w["codes"].dtype == torch.uint8
                assert np.array_equal(O.unpack_nibble(w["codes"].numpy()), q["codes"])
            else:
                # int8 and Q5 (unpacked at load) -> int8 [N, Kp]
                assert w["codes"].dtype == torch.int8
                assert np.array_equal(w["codes"].numpy(), q["codes"]), name
            assert np.array_equal(w["norms"].numpy().view(np.uint16), q["norms"].view(np.uint16))
            # .ct is scaled by 1/sqrt(128) at load; .ct_scaled is used as stored
            np.testing.assert_allclose(w["ct_scaled"].numpy(), q["ct_scaled"], rtol=1e-6)
            if q["kind"] == "nibble_bias":
                assert np.array_equal(w["bias"].numpy().view(np.uint16), q["bias"].view(np.uint16))
            else:
                assert "bias" not in w
        # plain tensors: "<name>.weight" missing -> bare name
        assert tuple(ld.load_layer_weights("lm_head")["weight"].shape) == (16, 256)
        with pytest.raises(KeyError, match="has no weight"):
            ld.load_layer_weights("model.layers.9.nothing")
        with pytest.raises(KeyError, match="no tensor named"):
            ld.load_tensor("model.layers.0.absent.codes")


def test_missing_centroids_raise(split_ckpt, tmp_path):
    root, info = split_ckpt
    cfg = LD.load_polar_config(root)
    ld = LD.PolarWeightLoader(root, cfg, device="cpu")
    name = "model.layers.0.self_attn.v_proj"
    ld.weight_map = {k: v for k, v in ld.weight_map.items() if not k.startswith(name + ".ct")}
    with pytest.raises(KeyError, match="stores no codebook"):
        ld.load_layer_weights(name)


def test_hlwq_format(hlwq_ckpt):
    root, info = hlwq_ckpt
    cfg = LD.load_polar_config(root)
    ld = LD.PolarWeightLoader(root, cfg, device="cpu")
    for name, q in info.items():
        assert ld.is_quantized_layer(name)  # by its .weight__packed tensor
        w = ld.load_layer_weights(name)
        assert np.array_equal(w["codes"].numpy(), q["codes"])
        assert w["norms"].dtype == torch.float16
        np.testing.assert_allclose(w["ct_scaled"].numpy(), O.ct_scaled(5), rtol=1e-6)
        assert int(w["_hlwq_in_f"][0]) == q["in_f"]
    ld.weight_map = {k: v for k, v in ld.weight_map.items() if not k.endswith("__packed")}
    ld._quantized_layers.add("model.layers.0.mlp.up_proj")
    with pytest.raises(KeyError, match="lacks"):
        ld.load_layer_weights("model.layers.0.mlp.up_proj")


def test_bits_packed_and_names(split_ckpt):
    root, info = split_ckpt
    cfg = LD.load_polar_config(root)
    ld = LD.PolarWeightLoader(root, cfg, device="cpu")
    for name, q in info.items():
        assert ld.get_layer_bits(name) == q["bits"], name
        assert ld.is_quantized_layer(name)
        assert ld.is_packed(name) == (q["kind"] in ("q5", "nibble", "nibble_bias")), name
    assert not ld.is_quantized_layer("lm_head")
    # longest matching pattern wins; unmatched -> 5
    ld.polar_config = dict(cfg, layers={}, bit_assignment={"proj": 2, "gate_proj": 3, "mlp.gate_proj": 4})
    assert ld.get_layer_bits("model.layers.3.mlp.gate_proj") == 4
    assert ld.get_layer_bits("model.layers.3.self_attn.q_proj") == 2
    assert ld.get_layer_bits("model.layers.3.mixer") == 5
    assert LD.PolarWeightLoader(root, cfg, device="cpu").get_all_layer_names() == sorted(info)


def test_load_polar_model_state_dict(split_ckpt):
    root, info = split_ckpt
    sd, hf, cfg = LD.load_polar_model(root, device="cpu")
    assert hf["model_type"] == "synthetic" and cfg["format"] == "polar_engine_v4"
    assert sd["model.norm.weight"].dtype == torch.float16      # plain float -> dtype
    assert sd["lm_head"].dtype == torch.float16
    q = "model.layers.0.self_attn.v_proj"
    assert sd[q + ".codes"].dtype == torch.int8               # components keep their dtypes
    assert sd[q + ".ct_scaled"].dtype == torch.float32
    assert sd[q + ".norms"].dtype == torch.float16


def test_tp_shard_helpers():
    c = torch.arange(8 * 6, dtype=torch.int8).reshape(8, 6)
    assert torch.equal(LD.shard_codes_for_tp(c, 1, 2), c[4:])
    assert LD.shard_codes_for_tp(c, 1, 2, dim=1) is c
    assert LD.shard_codes_for_tp(c, 0, 1) is c
    n = torch.ones(8, 3, dtype=torch.float16)
    assert LD.shard_norms_for_tp(n, 3, 4, 3).shape == (2, 3)
    with pytest.raises(ValueError, match="do not split evenly"):
        LD.shard_codes_for_tp(c, 0, 3)
    with pytest.raises(ValueError, match="do not split evenly"):
        LD.shard_norms_for_tp(n, 0, 3, 3)


def test_merged_weight_loader_qkv_and_gate_up(split_ckpt):
    """Shards of a merged QKV / gate_up layer land at their partition rows."""
    root, info = split_ckpt
    cfg = LD.load_polar_config(root)
    ld = LD.PolarWeightLoader(root, cfg, device="cpu")
    names = ["model.layers.0.self_attn.q_proj", "model.layers.0.self_attn.k_proj",
             "model.layers.0.self_attn.v_proj"]
    sizes = [info[n]["out_f"] for n in names]
    meth = PolarQuantLinearMethod(bits=5)
    layer = torch.nn.Module()
    meth.create_weights(layer, 256, sizes, 256, sum(sizes), torch.float16)
    load = LD.merged_weight_loader(sizes)
    for sid, n in zip("qkv", names):
        w = ld.load_layer_weights(n)
        load(layer.codes, w["codes"], sid)
        load(layer.norms, w["norms"], sid)
    want = np.concatenate([info[n]["codes"] for n in names])
    assert np.array_equal(layer.codes.numpy(), want)
    assert np.array_equal(layer.norms.numpy().view(np.uint16),
                          np.concatenate([info[n]["norms"] for n in names]).view(np.uint16))
    # gate/up stored as nibbles: the buffer takes the stored row width
    g, u = "model.layers.0.mlp.gate_proj", "model.layers.0.mlp.up_proj"
    layer2 = torch.nn.Module()
    PolarQuantLinearMethod(bits=3).create_weights(layer2, 256, [96, 96], 256, 192, torch.float16)
    load2 = LD.merged_weight_loader([96, 96])
    for sid, n in ((0, g), (1, u)):
        load2(layer2.codes, ld.load_layer_weights(n)["codes"], sid)
    assert layer2.codes.dtype == torch.uint8 and tuple(layer2.codes.shape) == (192, 128)
    assert np.array_equal(O.unpack_nibble(layer2.codes.numpy()),
                          np.concatenate([info[g]["codes"], info[u]["codes"]]))
    # whole-tensor load and bad shard ids
    layer3 = torch.nn.Module()
    PolarQuantLinearMethod(bits=5).create_weights(layer3, 256, [32], 256, 32, torch.float16)
    load3 = LD.merged_weight_loader([32])
    load3(layer3.codes, torch.from_numpy(info[names[2]]["codes"]))
    assert np.array_equal(layer3.codes.numpy(), info[names[2]]["codes"])
    with pytest.raises(ValueError, match="outside"):
        load3(layer3.codes, torch.from_numpy(info[names[2]]["codes"]), 3)
    with pytest.raises(ValueError, match="unknown shard id"):
        load3(layer3.codes, torch.from_numpy(info[names[2]]["codes"]), "z")
    with pytest.raises(ValueError, match="partition expects"):
        load(layer.codes, torch.from_numpy(info[names[0]]["codes"]), "k")


def test_load_weights_into_layer_checks_shapes(split_ckpt):
    root, info = split_ckpt
    cfg = LD.load_polar_config(root)
    ld = LD.PolarWeightLoader(root, cfg, device="cpu")
    n = "model.layers.0.mlp.down_proj"
    w = ld.load_layer_weights(n)
    layer = torch.nn.Module()
    PolarQuantLinearMethod(bits=4).create_weights(layer, 384, [40], 384, 40, torch.float16)
    LD.load_weights_into_layer(layer, w)  # no method: buffers only
    assert layer.packed and tuple(layer.codes_packed.shape) == (40, 192)
    assert not hasattr(layer, "codes")
    assert layer.bias.dtype == torch.float16
    bad = torch.nn.Module()
    PolarQuantLinearMethod(bits=4).create_weights(bad, 256, [40], 256, 40, torch.float16)
    with pytest.raises(ValueError, match="norms shape"):
        LD.load_weights_into_layer(bad, w)
    bad2 = torch.nn.Module()
    PolarQuantLinearMethod(bits=5).create_weights(bad2, 384, [40], 384, 40, torch.float16)
    with pytest.raises(ValueError, match="levels"):
        LD.load_weights_into_layer(bad2, w)
