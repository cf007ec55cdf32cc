"""GPU parity at BASELINE's configs: the mixed-bit decoder layer (C4), the
decode MLP shapes at M = 4 / 16 (C2), and the prefill shapes at M = 256,
2048 and 8192 (C3), each against the CPU oracle on identical inputs.

C4 follows the reference fixture's decoder layer (tests/conftest.py:60-131)
and PolarQuantLinearMethod.apply (linear_method.py:184-221): Q/K/V are Q5
(32 query heads, 8 KV heads, head_dim 128) sharing one FWHT of the normed
hidden state, O is Q6, gate/up Q3 and down Q4 at hidden 4096 /
intermediate 12288; weights N(0, 0.02) fp16, quantized by the GPU quantizer;
RMSNorm weights fp16. Attention between Q/K/V and O is a plain causal GQA
softmax in float32 (no RoPE); the test covers the linears, each compared with
the oracle on the exact fp16 input the layer gave it.
"""

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import DEV, check_close, dev_tiled, linear_call, rand_layer, say, to_dev

pytestmark = pytest.mark.gpu

HID, INTER, NQ, NKV, HD = 4096, 12288, 32, 8, 128
C4_SPECS = [("q_proj", HID, NQ * HD, 5), ("k_proj", HID, NKV * HD, 5), ("v_proj", HID, NKV * HD, 5),
            ("o_proj", NQ * HD, HID, 6), ("gate_proj", HID, INTER, 3), ("up_proj", HID, INTER, 3),
            ("down_proj", INTER, HID, 4)]


# the checkpoint's polar_config.json for this layer (the reference fixture's
# bit assignment, tests/conftest.py:60-131): methods come from
# PolarQuantConfig.get_quant_method, as vLLM builds them
C4_POLAR_CONFIG = {
    "format": "polar_engine_v4", "quantization": "polarengine", "block_size": 128,
    "bit_assignment": {"q_proj": 5, "k_proj": 5, "v_proj": 5, "o_proj": 6, "gate_proj": 3,
                       "up_proj": 3, "down_proj": 4, "embed": 5, "lm_head": 6},
    "layers": {},
}


class PolarLinear(torch.nn.Module):
    """A vLLM-style linear module: forward = quant_method.apply(self, x), the
    method resolved from the polar config by the module's prefix."""

    def __init__(self, in_f, out_f, bits, seed, prefix):
        super().__init__()
        from polarengine_vllm.config import PolarQuantConfig
        from polarengine_vllm.linear_method import PolarQuantLinearMethod
        from polarengine_vllm.quantizer import PolarQuantizer
        cfg = PolarQuantConfig.from_config(C4_POLAR_CONFIG)
        self.quant_method = cfg.get_quant_method(self, prefix)
        assert isinstance(self.quant_method, PolarQuantLinearMethod)
        assert self.quant_method.bits == bits, (prefix, self.quant_method.bits, bits)
        self.quant_method.create_weights(self, in_f, [out_f], in_f, out_f, torch.float16)
        self.to(DEV)
        w = torch.from_numpy(O.seeded_normal((out_f, in_f), 0.02, seed)).to(DEV)
        q = PolarQuantizer(128).quantize_tensor(w, bits)
        self.codes.copy_(q["codes"])
        self.norms.copy_(q["norms"])
        # oracle copies of what was loaded
        self.o_codes = q["codes"].cpu().numpy()
        self.o_norms = q["norms"].cpu().numpy()
        self.o_ct = q["ct_scaled"].cpu().numpy()
        self.quant_method.process_weights_after_loading(self)
        self.seen = []  # the inputs this module was called with (device)

    def forward(self, x):
        self.seen.append(x)
        return self.quant_method.apply(self, x)


class Attn(torch.nn.Module):
    def __init__(self, seed):
        super().__init__()
        mods = {n: PolarLinear(i, o, b, seed + k, f"model.layers.0.self_attn.{n}")
                for k, (n, i, o, b) in enumerate(C4_SPECS[:4])}
        for n, m in mods.items():
            setattr(self, n, m)

    def forward(self, x):
        q, k, v = self.q_proj(x), self.k_proj(x), self.v_proj(x)
        m = x.shape[0]
        qh = q.float().view(m, NQ, HD).transpose(0, 1).contiguous()
        kh = k.float().view(m, NKV, HD).transpose(0, 1).repeat_interleave(NQ // NKV, 0).contiguous()
        vh = v.float().view(m, NKV, HD).transpose(0, 1).repeat_interleave(NQ // NKV, 0).contiguous()
        s = torch.matmul(qh, kh.transpose(1, 2).contiguous()) / HD ** 0.5
        causal = torch.triu(torch.ones(m, m, dtype=torch.bool, device=x.device), 1)
        p = torch.softmax(s.masked_fill(causal, float("-inf")), -1)
        a = torch.matmul(p, vh).transpose(0, 1).reshape(m, NQ * HD).half()
        return self.o_proj(a)


class Mlp(torch.nn.Module):
    def __init__(self, seed):
        super().__init__()
        for k, (n, i, o, b) in enumerate(C4_SPECS[4:]):
            setattr(self, n, PolarLinear(i, o, b, seed + 4 + k, f"model.layers.0.mlp.{n}"))

    def forward(self, x):
        g, u = self.gate_proj(x), self.up_proj(x)
        act = (torch.nn.functional.silu(g.float()) * u.float()).half()
        return self.down_proj(act)


def rmsnorm(h, w):
    hf = h.float()
    return (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()).half()


class DecoderLayer(torch.nn.Module):
    def __init__(self, seed=900):
        super().__init__()
        self.self_attn = Attn(seed)
        self.mlp = Mlp(seed)
        self.ln1 = torch.from_numpy(1.0 + O.seeded_normal((HID,), 0.1, seed - 1)).to(DEV)
        self.ln2 = torch.from_numpy(1.0 + O.seeded_normal((HID,), 0.1, seed - 2)).to(DEV)

    def forward(self, h):
        h2 = h + self.self_attn(rmsnorm(h, self.ln1))
        return h2 + self.mlp(rmsnorm(h2, self.ln2))


@pytest.fixture(scope="module")
def c4_layer():
    from polarengine_vllm.linear_method import install_fwht_cache_hooks
    say("building the C4 decoder layer (GPU quantizer)")
    layer = DecoderLayer()
    assert install_fwht_cache_hooks(layer) == 2  # the attention and MLP blocks
    torch.cuda.synchronize()
    return layer


@pytest.mark.parametrize("m", [1, 16, 512])
def test_decoder_layer_c4(c4_layer, m, monkeypatch):
    import polarengine_vllm.linear_method as lm
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE
    say(f"C4 decoder layer m={m}")
    calls = []
    real = lm.fwht_pairs

    def counting(x, *a, **k):
        calls.append(x.shape)
        return real(x, *a, **k)

    monkeypatch.setattr(lm, "fwht_pairs", counting)
    mods = [getattr(c4_layer.self_attn, n) for n, *_ in C4_SPECS[:4]] + \
           [getattr(c4_layer.mlp, n) for n, *_ in C4_SPECS[4:]]
    for mod in mods:
        mod.seen.clear()
    GLOBAL_FWHT_CACHE.clear()
    h = torch.from_numpy(O.seeded_normal((m, HID), 1.0, 950 + m)).to(DEV)
    out = c4_layer(h)
    torch.cuda.synchronize()
    assert out.shape == (m, HID) and out.dtype == torch.float16 and torch.isfinite(out).all()
    if m <= 32:
        assert calls == []  # the transform is fused into every decode GEMV
    else:
        # one transform for Q/K/V, one for O, one for gate/up, one for down
        assert len(calls) == 4, calls
    for (name, in_f, out_f, bits), mod in zip(C4_SPECS, mods):
        assert len(mod.seen) == 1
        x = mod.seen[0]
        y = mod.quant_method.apply(mod, x)  # same input again (cache cleared below)
        want = O.linear_apply(x.cpu().numpy(), mod.o_codes, mod.o_norms, mod.o_ct, in_f)
        check_close(y.float().cpu().numpy(), want.astype(np.float32), f"C4 m={m} {name} q{bits}")
        GLOBAL_FWHT_CACHE.clear()
    # Q, K and V read the same normed hidden state
    q_in = c4_layer.self_attn.q_proj.seen[0]
    assert c4_layer.self_attn.k_proj.seen[0] is q_in and c4_layer.self_attn.v_proj.seen[0] is q_in


@pytest.mark.parametrize("m", [1, 64, 512])
def test_decoder_layer_c4_inference_mode(c4_layer, m, monkeypatch):
    """The C4 layer under torch.inference_mode() (how vLLM runs every
    forward): inference tensors carry no version counter, the FWHT cache
    still shares one transform per input inside each hooked block, and the
    output equals the same forward outside inference mode bit for bit."""
    import polarengine_vllm.linear_method as lm
    say(f"C4 decoder layer under inference_mode m={m}")
    calls = []
    real = lm.fwht_pairs

    def counting(x, *a, **k):
        calls.append(x.shape)
        return real(x, *a, **k)

    monkeypatch.setattr(lm, "fwht_pairs", counting)
    h = torch.from_numpy(O.seeded_normal((m, HID), 1.0, 990 + m)).to(DEV)
    want = c4_layer(h)
    n_plain = len(calls)
    with torch.inference_mode():
        hi = h.clone()
        got = c4_layer(hi)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert len(calls) - n_plain == (0 if m <= 32 else 4)
    for mod in c4_layer.modules():
        if hasattr(mod, "seen"):
            mod.seen.clear()


# ---------------------------------------------------------------------------
# C2: decode MLP shapes at M = 4 and 16 (tiled runtime layout, with bias)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m", [4, 16])
@pytest.mark.parametrize("n,k,bits", [(12288, 4096, 3), (4096, 12288, 4), (12288, 4096, 4),
                                      (4096, 12288, 3)])
def test_c2_decode_mlp_shapes(m, n, k, bits):
    say(f"C2 decode m={m} n={n} k={k} q{bits}")
    rng = np.random.default_rng(m + n + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 960 + m)
    bias = O.seeded_normal((n,), 0.1, 961)
    dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
    from polarengine_vllm import _lib
    fmt = _lib.PE_PACK_NIBBLE | _lib.PE_LAYOUT_TILE16
    y = linear_call(to_dev(x), dcodes, dnorms, ct, bits, fmt, n, to_dev(bias))
    want = O.linear_apply(x, codes, norms, ct, k, bias)
    check_close(y.float().cpu().numpy(), want.astype(np.float32), f"C2 m={m} {n}x{k} q{bits}")


# ---------------------------------------------------------------------------
# C3: prefill shapes; whole outputs against the dense dequantize-then-matmul
# route (one fp32 sgemm), M = 8192 included
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k,bits", [(256, 4096, 12288, 3), (256, 12288, 4096, 4),
                                        (2048, 12288, 4096, 4), (2048, 4096, 12288, 3),
                                        (8192, 4096, 12288, 3), (8192, 12288, 4096, 4)])
def test_c3_prefill_whole_output(m, n, k, bits):
    from polarengine_vllm import _lib
    say(f"C3 prefill m={m} n={n} k={k} q{bits}")
    rng = np.random.default_rng(m + n + k + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 970 + bits)
    bias = O.seeded_normal((n,), 0.1, 971)
    dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
    fmt = _lib.PE_PACK_NIBBLE | _lib.PE_LAYOUT_TILE16
    y = linear_call(to_dev(x), dcodes, dnorms, ct, bits, fmt, n, to_dev(bias))
    w = O.dequant_weight(codes, norms, ct)
    rows = np.arange(m)  # every row, M = 8192 included
    want = O.dequant_matmul(x[rows], w, bias)
    got = y[torch.from_numpy(rows).to(DEV)].float().cpu().numpy()
    check_close(got, want.astype(np.float32), f"C3 m={m} {n}x{k} q{bits} ({len(rows)} rows)")
    # per m-tile as well: a wrong tile cannot hide behind the global maxima
    for t0 in range(0, len(rows), 128):
        sl = slice(t0, t0 + 128)
        check_close(got[sl], want[sl].astype(np.float32), f"C3 m={m} rows {rows[t0]}..")
    assert torch.isfinite(y).all()
