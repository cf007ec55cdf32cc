"""GPU tests of the checkpoint loader: the HIP unpack kernels against the
oracle (bit-exact), and checkpoint -> loader -> PolarQuantLinearMethod ->
forward against the oracle's linear on the same quantized weights."""

import numpy as np
import pytest
import torch

import polar_oracle as O
from ckpt_fixture import write_hlwq_checkpoint, write_split_checkpoint

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _say(msg):
    print(f"[case] {msg}", flush=True)


def check_close(got, want, what, tol=1e-2, cos_tol=0.9999):
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    w = np.asarray(want, dtype=np.float64).reshape(-1)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - w).max() / max(np.abs(w).max(), 1e-30)
    cos = float(g @ w / (np.linalg.norm(g) * np.linalg.norm(w) + 1e-300))
    assert err <= tol, f"{what}: normwise err {err:.3e}"
    assert cos >= cos_tol, f"{what}: cosine {cos:.7f}"


@pytest.fixture(scope="module")
def split_ckpt(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("split_gpu"))
    return root, write_split_checkpoint(root)


@pytest.fixture(scope="module")
def hlwq_ckpt(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("hlwq_gpu"))
    return root, write_hlwq_checkpoint(root)


@pytest.mark.parametrize("groups,total", [(1, 8), (7, 53), (1000, 8000), (4097, 32771)])
def test_unpack_q5_hlwq_kernel_bit_exact(groups, total):
    from polarengine_vllm.packing import unpack_codes_q5_hlwq
    _say(f"hlwq unpack groups={groups} total={total}")
    rng = np.random.default_rng(groups)
    packed = rng.integers(0, 256, groups * 5, dtype=np.uint8)
    got = unpack_codes_q5_hlwq(torch.from_numpy(packed).to(DEV), total=total)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), O.unpack_q5_hlwq(packed, total=total))


def test_unpack_q5_hlwq_rejects_bad_sizes():
    from polarengine_vllm import _lib
    L = _lib.lib()
    buf = torch.zeros(64, dtype=torch.uint8, device=DEV)
    out = torch.zeros(128, dtype=torch.int8, device=DEV)
    st = _lib.stream_ptr(torch.device(DEV))
    assert L.pe_unpack_q5_hlwq(buf.data_ptr(), 12, out.data_ptr(), 8, st) == _lib.PE_ERR_DIMS
    assert L.pe_unpack_q5_hlwq(buf.data_ptr(), 10, out.data_ptr(), 17, st) == _lib.PE_ERR_DIMS
    assert L.pe_unpack_q5_hlwq(None, 10, out.data_ptr(), 8, st) == _lib.PE_ERR_NULL


def test_gpu_loader_matches_cpu_loader(split_ckpt, hlwq_ckpt):
    """Q5 and HLWQ codes unpacked by the HIP kernels equal the stored codes."""
    from polarengine_vllm import loader as LD
    for root, info in (split_ckpt, hlwq_ckpt):
        cfg = LD.load_polar_config(root)
        with LD.PolarWeightLoader(root, cfg, device=DEV) as ld:
            for name, q in info.items():
                _say(f"gpu loader {name}")
                w = ld.load_layer_weights(name)
                assert w["codes"].device.type == "cuda"
                c = w["codes"].cpu().numpy()
                if q.get("kind", "").startswith("nibble"):
                    c = O.unpack_nibble(c)
                assert np.array_equal(c.astype(np.int8), q["codes"]), name


def _linear_from_checkpoint(ld, names, sizes, bits):
    from polarengine_vllm import loader as LD
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    in_f = ld.polar_config["layers"].get(names[0], {}).get("in_features")
    meth = PolarQuantLinearMethod(bits=bits)
    layer = torch.nn.Module()
    meth.create_weights(layer, in_f, sizes, in_f, sum(sizes), torch.float16)
    layer.to(DEV)
    if len(names) == 1:
        LD.load_weights_into_layer(layer, ld.load_layer_weights(names[0]), meth)
    else:
        load = LD.merged_weight_loader(sizes)
        ws = [ld.load_layer_weights(n) for n in names]
        for i, w in enumerate(ws):
            load(layer.codes, w["codes"], i)
            load(layer.norms, w["norms"], i)
        merged = {"codes": layer.codes, "norms": layer.norms, "ct_scaled": ws[0]["ct_scaled"]}
        LD.load_weights_into_layer(layer, merged, meth)
    return meth, layer


@pytest.mark.parametrize("m", [1, 3, 40])
def test_checkpoint_to_forward(split_ckpt, m):
    """Every stored layout, loaded and run through the plugin's apply()."""
    from polarengine_vllm import loader as LD
    root, info = split_ckpt
    cfg = LD.load_polar_config(root)
    with LD.PolarWeightLoader(root, cfg, device=DEV) as ld:
        for name, q in info.items():
            _say(f"checkpoint forward {name} m={m}")
            meth, layer = _linear_from_checkpoint(ld, [name], [q["out_f"]], q["bits"])
            x = O.seeded_normal((m, q["in_f"]), 1.0, 7 + m)
            bias = q.get("bias")
            b = torch.from_numpy(bias).to(DEV) if bias is not None else None
            y = meth.apply(layer, torch.from_numpy(x).to(DEV), b)
            torch.cuda.synchronize()
            want = O.linear_apply(x, q["codes"], q["norms"], q["ct_scaled"], q["in_f"], bias)
            check_close(y.float().cpu().numpy(), want, f"{name} m={m}")
            # the quantized layer approximates the original weight
            dense = x.astype(np.float32) @ q["weight"].T
            if bias is not None:
                dense = dense + bias.astype(np.float32)
            cos = float((want.reshape(-1) @ dense.reshape(-1)) /
                        (np.linalg.norm(want) * np.linalg.norm(dense)))
            assert cos > 0.97, f"{name}: quantized vs dense cosine {cos}"


@pytest.mark.parametrize("m", [1, 17])
def test_merged_qkv_checkpoint_forward(split_ckpt, m):
    from polarengine_vllm import loader as LD
    root, info = split_ckpt
    cfg = LD.load_polar_config(root)
    names = ["model.layers.0.self_attn.q_proj", "model.layers.0.self_attn.k_proj",
             "model.layers.0.self_attn.v_proj"]
    sizes = [info[n]["out_f"] for n in names]
    with LD.PolarWeightLoader(root, cfg, device=DEV) as ld:
        _say(f"merged qkv m={m}")
        meth, layer = _linear_from_checkpoint(ld, names, sizes, 5)
        x = O.seeded_normal((m, 256), 1.0, 40 + m)
        y = meth.apply(layer, torch.from_numpy(x).to(DEV))
        torch.cuda.synchronize()
    want = np.concatenate([O.linear_apply(x, info[n]["codes"], info[n]["norms"],
                                          info[n]["ct_scaled"], 256) for n in names], axis=1)
    check_close(y.float().cpu().numpy(), want, f"merged qkv m={m}")
