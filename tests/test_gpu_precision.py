"""Precision margins of every kernel route at BASELINE's shapes.

The kernels compute in fp16 operands on the matrix cores with fp32 sums: the
transformed activation x_tf and the codebook values are rounded to fp16 (the
prefill GEMM also rounds ct * norm to fp16), while the reference's GEMV and
GEMM keep them in fp32 (polarengine_vllm/linear_method.py:184-221,
kernels/polar_gemv.py:48-94, kernels/polar_gemm.py:81-171). This test measures
what that costs against the unrounded fp32 oracle (no 16-bit cast of y), per
shape and route, through PolarQuantLinearMethod.apply on weights from the GPU
quantizer (N(0, 0.02), the configs' weights), for fp16 and bf16 activations,
both N(0, 1) and with outlier channels (8 channels x 64, as in LLM residual
streams). It asserts a margin to the north-star tolerance (normwise error
<= 1e-2, cosine >= 0.9999), not only the tolerance itself:

* fp16 out: normwise error <= 2.5e-3 (4x margin). The output rounding alone
  contributes up to 2^-11 of max|y| (4.9e-4);
* bf16 out: normwise error <= 5e-3 (2x margin). The bf16 output rounding
  alone contributes up to 2^-9 of max|y| (2e-3);
* cosine >= 0.99999 (10x margin on 1 - cos).

Routes: M = 1..16 the decode GEMV with the transform fused (M = 1 at K =
12288 and M = 16 through the K split over workgroups), M = 512 and 2048 the
prefill GEMM after the shared FWHT kernel; bf16 input at M > 32 also takes
the shared transform."""

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import DEV, say

pytestmark = pytest.mark.gpu

FP16_MAX_ERR = 2.5e-3
BF16_MAX_ERR = 5e-3
MIN_COS = 0.99999

# (label, n_out, k_in, bits, M values)
SHAPES = [
    ("C1 q5 4096x4096", 4096, 4096, 5, [1]),
    ("C2 gate/up q3 12288x4096", 12288, 4096, 3, [1, 4, 16]),
    ("C2 down q4 4096x12288", 4096, 12288, 4, [1, 4, 16]),
    ("C4 o q6 4096x4096", 4096, 4096, 6, [1, 512]),
    ("C3 q4 12288x4096", 12288, 4096, 4, [2048]),
    ("C3 q3 4096x12288", 4096, 12288, 3, [512]),
]
CASES = [(lab, n, k, b, m) for lab, n, k, b, ms in SHAPES for m in ms]
# rows compared at large M: every 128-row m-tile, both ends
SAMPLE_ROWS = 24


class _Layer(torch.nn.Module):
    def __init__(self, in_f, out_f, bits, seed):
        super().__init__()
        from polarengine_vllm.linear_method import PolarQuantLinearMethod
        from polarengine_vllm.quantizer import PolarQuantizer
        self.quant_method = PolarQuantLinearMethod(128, bits)
        self.quant_method.create_weights(self, in_f, [out_f], in_f, out_f, torch.float16)
        self.to(DEV)
        w = torch.from_numpy(O.seeded_normal((out_f, in_f), 0.02, seed)).to(DEV)
        q = PolarQuantizer(128).quantize_tensor(w, bits)
        self.codes.copy_(q["codes"])
        self.norms.copy_(q["norms"])
        self.o_codes = q["codes"].cpu().numpy()
        self.o_norms = q["norms"].cpu().numpy()
        self.o_ct = q["ct_scaled"].cpu().numpy()
        self.quant_method.process_weights_after_loading(self)


_LAYERS = {}


def _layer(n, k, bits):
    key = (n, k, bits)
    if key not in _LAYERS:
        _LAYERS[key] = _Layer(k, n, bits, seed=1200 + bits + n // 1024 + k // 1024)
    return _LAYERS[key]


def _activations(m, k, kind, seed):
    x = O.seeded_normal((m, k), 1.0, seed).astype(np.float32)
    if kind == "outlier":
        ch = np.random.default_rng(seed).choice(k, 8, replace=False)
        x[:, ch] *= 64.0
    return x


def _rows(m):
    if m <= SAMPLE_ROWS:
        return np.arange(m)
    rng = np.random.default_rng(m)
    rows = {0, m - 1}
    for t0 in range(0, m, 128):
        rows.add(int(rng.integers(t0, min(m, t0 + 128))))
    return np.array(sorted(rows))


@pytest.fixture(scope="module", autouse=True)
def _free_layers():
    yield
    _LAYERS.clear()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("kind", ["normal", "outlier"])
@pytest.mark.parametrize("label,n,k,bits,m", CASES)
def test_precision_margin(label, n, k, bits, m, kind, dtype):
    say(f"precision {label} m={m} {kind} {dtype}")
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE
    GLOBAL_FWHT_CACHE.clear()
    layer = _layer(n, k, bits)
    tdt = getattr(torch, dtype)
    x32 = _activations(m, k, kind, seed=1300 + m + bits)
    xd = torch.from_numpy(x32).to(tdt).to(DEV)
    y = layer.quant_method.apply(layer, xd)
    torch.cuda.synchronize()
    assert y.dtype == tdt and y.shape == (m, n)
    rows = _rows(m)
    xin = xd.float().cpu().numpy()[rows]  # the exact 16-bit input the kernels saw
    want = O.hadamard_domain_matmul(layer.o_codes, layer.o_norms, layer.o_ct,
                                    O.fwht_blocks(xin)).astype(np.float64)
    got = y[torch.from_numpy(rows).to(DEV)].float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    err = float(np.abs(got - want).max() / np.abs(want).max())
    cos = float((got * want).sum() / (np.linalg.norm(got) * np.linalg.norm(want)))
    rms_err = float(np.sqrt(((got - want) ** 2).mean()) / np.sqrt((want ** 2).mean()))
    limit = FP16_MAX_ERR if dtype == "float16" else BF16_MAX_ERR
    # distance from the correctly rounded 16-bit result, in units of its last place
    if dtype == "float16":
        w16 = want.astype(np.float16)
        ulp = np.spacing(np.abs(w16)).astype(np.float64)
    else:
        w16 = O.bf16_bits_to_f32(O.f32_to_bf16_bits(want.astype(np.float32)))
        e = np.floor(np.log2(np.maximum(np.abs(w16), 2.0 ** -126)))
        ulp = np.exp2(e - 7)
    dist = np.abs(got - w16.astype(np.float64)) / ulp
    say(f"  normwise {err:.3e} (margin {1e-2 / err:.1f}x)  rms-rel {rms_err:.3e}  "
        f"1-cos {1 - cos:.2e}  exact {np.mean(dist == 0):.2f}  "
        f"ulp p50/p99 {np.percentile(dist, 50):.0f}/{np.percentile(dist, 99):.0f}  rows {len(rows)}")
    assert err <= limit, f"{label} m={m} {kind} {dtype}: normwise {err:.3e} > {limit}"
    assert cos >= MIN_COS, f"{label} m={m} {kind} {dtype}: cosine {cos:.8f}"
