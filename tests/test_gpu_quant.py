"""GPU quantizer (pe_quantize) against the oracle's quantize_tensor and the
reference's golden codes (quantizer.py:206-257).

Codes are integers but come from an argmin over fp32 distances: the kernel's
butterfly transform and the reference's fp32 matmul round differently, so a
code may differ where the rotated value sits within fp32 rounding of the
midpoint between two centroids. The tests accept exactly those cases (and
count them); every other code, and every fp16 norm, must be equal."""

import math

import numpy as np
import pytest
import torch

import polar_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TIE_TOL = 1e-5  # |d_a - d_b| of a tolerated flip, relative to the centroid scale


def _say(msg):
    print(f"[case] {msg}", flush=True)


def rotated(w: np.ndarray) -> np.ndarray:
    """float64 statement of the rotated unit blocks (r in quantizer.py:235-241)."""
    w = np.asarray(w, dtype=np.float64)
    n, k = w.shape
    kp = (k + 127) // 128 * 128
    w = np.pad(w, ((0, 0), (0, kp - k))).reshape(n, kp // 128, 128)
    nrm = np.maximum(np.sqrt((w ** 2).sum(-1)), 1e-10)
    return ((w / nrm[..., None]) @ (O.hadamard(128).astype(np.float64) * math.sqrt(128))).reshape(n, kp)


def check_codes(got: np.ndarray, want: np.ndarray, w: np.ndarray, bits: int, what: str) -> int:
    got = np.asarray(got).astype(np.int64)
    want = np.asarray(want).astype(np.int64)
    assert got.shape == want.shape, what
    bad = np.argwhere(got != want)
    if len(bad):
        r = rotated(w)
        ct = O.get_centroids(bits).astype(np.float64)
        for i, j in bad:
            da = abs(r[i, j] - ct[got[i, j]])
            db = abs(r[i, j] - ct[want[i, j]])
            assert abs(da - db) <= TIE_TOL, (f"{what}: code ({i},{j}) {got[i, j]} vs {want[i, j]} "
                                             f"is not a near-tie (|d| {da:.3e} vs {db:.3e})")
    assert len(bad) <= max(2, got.size // 10000), f"{what}: {len(bad)} near-tie flips"
    return len(bad)


def check_norms(got: np.ndarray, want: np.ndarray, what: str) -> None:
    g = np.asarray(got).view(np.uint16).astype(np.int64)
    w = np.asarray(want).view(np.uint16).astype(np.int64)
    diff = np.abs(g - w)
    assert diff.max() <= 1, f"{what}: fp16 norm off by {diff.max()} ulp"
    assert (diff != 0).mean() <= 1e-3, f"{what}: {(diff != 0).sum()} norms off by 1 ulp"


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6])
def test_quantizer_matches_reference_golden(golden, bits):
    from polarengine_vllm.quantizer import PolarQuantizer
    _say(f"quantize golden bits={bits}")
    w = golden["quant_w"]
    q = PolarQuantizer(128).quantize_tensor(torch.from_numpy(w).to(DEV), bits)
    torch.cuda.synchronize()
    check_codes(q["codes"].cpu().numpy(), golden[f"quant_codes_b{bits}"], w.astype(np.float32),
                bits, f"golden b{bits}")
    check_norms(q["norms"].cpu().numpy(), golden[f"quant_norms_b{bits}"], f"golden b{bits}")
    assert np.array_equal(q["ct_scaled"].cpu().numpy(), golden[f"quant_ct_scaled_b{bits}"])


@pytest.mark.parametrize("n,k,bits,dt", [(64, 4096, 4, torch.float16), (333, 1000, 3, torch.float32),
                                         (128, 384, 5, torch.bfloat16), (96, 2048, 6, torch.float16),
                                         (17, 130, 2, torch.float32), (512, 1408, 8, torch.float16)])
def test_quantizer_matches_oracle(n, k, bits, dt):
    from polarengine_vllm.quantizer import PolarQuantizer
    _say(f"quantize n={n} k={k} bits={bits} dt={dt}")
    w16 = O.seeded_normal((n, k), 0.02, n + k + bits)
    wt = torch.from_numpy(w16.astype(np.float32)).to(dt)
    w = wt.float().numpy()  # the values the kernel sees
    q = PolarQuantizer(128).quantize_tensor(wt.to(DEV), bits)
    torch.cuda.synchronize()
    want = O.quantize_tensor(w, bits)
    flips = check_codes(q["codes"].cpu().numpy(), want["codes"], w, bits, f"{n}x{k} b{bits}")
    check_norms(q["norms"].cpu().numpy(), want["norms"], f"{n}x{k} b{bits}")
    np.testing.assert_array_equal(q["ct_scaled"].cpu().numpy(), want["ct_scaled"])
    print(f"near-tie flips: {flips}")


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quantizer_packed_output(bits):
    """pack=True writes exactly the nibbles of the int8 codes."""
    from polarengine_vllm.quantizer import PolarQuantizer
    _say(f"quantize packed bits={bits}")
    w = torch.from_numpy(O.seeded_normal((200, 1536), 0.02, 5 + bits)).to(DEV)
    qz = PolarQuantizer(128)
    q = qz.quantize_tensor(w, bits)
    qp = qz.quantize_tensor(w, bits, pack=True)
    torch.cuda.synchronize()
    assert qp["codes"].dtype == torch.uint8 and tuple(qp["codes"].shape) == (200, 768)
    assert np.array_equal(qp["codes"].cpu().numpy(), O.pack_nibble(q["codes"].cpu().numpy()))
    assert torch.equal(qp["norms"], q["norms"])


def test_quantizer_roundtrip_quality_and_plugin():
    """Quantize on the GPU, run the plugin's linear, compare with the dense
    product (the format's approximation) and with the oracle (the kernels)."""
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    from polarengine_vllm.quantizer import PolarQuantizer
    _say("quantize -> linear")
    w = O.seeded_normal((768, 2048), 0.02, 77).astype(np.float32)
    q = PolarQuantizer(128).quantize_tensor(torch.from_numpy(w).to(DEV), 4)
    deq = O.dequant_weight(q["codes"].cpu().numpy(), q["norms"].cpu().numpy(),
                           q["ct_scaled"].cpu().numpy())
    cos = float((deq * w).sum() / (np.linalg.norm(deq) * np.linalg.norm(w)))
    assert cos > 0.99, f"Q4 reconstruction cosine {cos}"
    meth = PolarQuantLinearMethod(bits=4)
    layer = torch.nn.Module()
    meth.create_weights(layer, 2048, [768], 2048, 768, torch.float16)
    layer.to(DEV)
    layer.codes.copy_(q["codes"])
    layer.norms.copy_(q["norms"])
    meth.process_weights_after_loading(layer)
    x = O.seeded_normal((5, 2048), 1.0, 78)
    y = meth.apply(layer, torch.from_numpy(x).to(DEV)).float().cpu().numpy()
    want = O.linear_apply(x, q["codes"].cpu().numpy(), q["norms"].cpu().numpy(),
                          q["ct_scaled"].cpu().numpy(), 2048)
    err = np.abs(y - want).max() / np.abs(want).max()
    assert err <= 1e-2, err


def test_quantize_rejects_bad_arguments():
    from polarengine_vllm import _lib
    L = _lib.lib()
    w = torch.zeros(4, 256, device=DEV, dtype=torch.float16)
    ct = torch.zeros(32, device=DEV)
    c = torch.zeros(4, 256, dtype=torch.int8, device=DEV)
    nr = torch.zeros(4, 2, dtype=torch.float16, device=DEV)
    st = _lib.stream_ptr(torch.device(DEV))
    assert L.pe_quantize(w.data_ptr(), 0, 4, 256, 256, ct.data_ptr(), 32, 1, c.data_ptr(),
                         nr.data_ptr(), st) == _lib.PE_ERR_BITS  # nibbles need <= 16 levels
    assert L.pe_quantize(w.data_ptr(), 0, 4, 256, 100, ct.data_ptr(), 32, 0, c.data_ptr(),
                         nr.data_ptr(), st) == _lib.PE_ERR_DIMS  # ldw < K
    assert L.pe_quantize(w.data_ptr(), 7, 4, 256, 256, ct.data_ptr(), 32, 0, c.data_ptr(),
                         nr.data_ptr(), st) == _lib.PE_ERR_DTYPE
    assert L.pe_quantize(None, 0, 4, 256, 256, ct.data_ptr(), 32, 0, c.data_ptr(),
                         nr.data_ptr(), st) == _lib.PE_ERR_NULL
