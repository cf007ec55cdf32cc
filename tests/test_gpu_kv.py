"""GPU tests of the KV-cache path: pe_kv_quantize / pe_kv_dequantize against
the reference's golden vectors and the oracle (kv_cache/cache.py:180-256),
and the cache manager / attention hook built on them (cache.py:263-462,
attention.py).

Codes come from an argmin over fp32 distances, and the kernel's butterfly
transform rounds differently from the reference's fp32 matmul, so a code may
differ where the rotated value lies within fp32 rounding of the midpoint of
two centroids; the tests accept exactly those flips and count them. Norms are
bf16 and may differ by one bf16 ulp where the fp32 norm sits on a rounding
boundary (rare, counted). Expanded values are bf16 and may differ by one bf16
ulp (plus 1e-6 of the vector's norm for values near zero)."""

import math
import os

import numpy as np
import pytest
import torch

import polar_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TIE_TOL = 1e-5
DTS = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def gkv():
    return np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_kv.npz"))


def _rot64(x: np.ndarray) -> np.ndarray:
    """float64 statement of the rotated unit vectors (cache.py:216-219)."""
    x = np.asarray(x, dtype=np.float64)
    d = x.shape[1]
    nrm = np.maximum(np.sqrt((x ** 2).sum(1, keepdims=True)), 1e-10)
    return (x / nrm) @ (O.hadamard(d).astype(np.float64) * math.sqrt(d))


def check_kv_codes(got_packed, want_packed, x, bits, what) -> int:
    d = x.shape[1]
    g = O.kv_unpack(np.asarray(got_packed), bits, d)
    w = O.kv_unpack(np.asarray(want_packed), bits, d)
    bad = np.argwhere(g != w)
    if len(bad):
        r = _rot64(x)
        ct = O.kv_centroids(bits).astype(np.float64)
        for i, j in bad:
            da, db = abs(r[i, j] - ct[g[i, j]]), abs(r[i, j] - ct[w[i, j]])
            assert abs(da - db) <= TIE_TOL, (f"{what}: code ({i},{j}) {g[i, j]} vs {w[i, j]} "
                                             f"is not a near-tie ({da:.3e} vs {db:.3e})")
    assert len(bad) <= max(2, g.size // 10000), f"{what}: {len(bad)} near-tie flips"
    return len(bad)


def check_bf16_norms(got, want, what):
    diff = np.abs(np.asarray(got).view(np.uint16).astype(np.int64) -
                  np.asarray(want).view(np.uint16).astype(np.int64))
    assert diff.max() <= 1, f"{what}: bf16 norm off by {diff.max()} ulp"
    assert (diff != 0).mean() <= 1e-2, f"{what}: {(diff != 0).sum()} norms off by 1 ulp"


def check_bf16_values(got_bits, want_bits, norms_bits, what):
    g = O.bf16_bits_to_f32(np.asarray(got_bits).view(np.uint16)).astype(np.float64)
    w = O.bf16_bits_to_f32(np.asarray(want_bits).view(np.uint16)).astype(np.float64)
    nrm = O.bf16_bits_to_f32(np.asarray(norms_bits).view(np.uint16)).astype(np.float64)[:, None]
    big = np.maximum(np.abs(g), np.abs(w))
    ulp = np.exp2(np.floor(np.log2(np.maximum(big, 1e-38))) - 7)
    tol = np.maximum(ulp, 1e-6 * nrm)
    bad = np.abs(g - w) > tol
    assert not bad.any(), f"{what}: {bad.sum()} values beyond 1 bf16 ulp (max |d| {np.abs(g - w).max():.3e})"
    assert (g != w).mean() <= 0.05, f"{what}: {(g != w).sum()} values differ by 1 ulp"


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_kv_kernels_match_reference_golden(gkv, d, bits):
    from polarengine_vllm.kv_cache import PolarKVQuantizer
    _say(f"kv golden d={d} bits={bits}")
    xb = gkv[f"kv_x_d{d}"]
    x = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16).to(DEV)
    qz = PolarKVQuantizer(d, bits, DEV)
    packed, norms = qz.quantize(x)
    deq = qz.dequantize(torch.from_numpy(gkv[f"kv_packed_d{d}_b{bits}"]).to(DEV),
                        torch.from_numpy(gkv[f"kv_norms_d{d}_b{bits}"].view(np.int16)).view(torch.bfloat16).to(DEV),
                        (xb.shape[0], d))
    torch.cuda.synchronize()
    xf = O.bf16_bits_to_f32(xb)
    check_kv_codes(packed.cpu().numpy(), gkv[f"kv_packed_d{d}_b{bits}"], xf, bits, f"golden d{d} b{bits}")
    check_bf16_norms(_bits(norms), gkv[f"kv_norms_d{d}_b{bits}"], f"golden d{d} b{bits}")
    check_bf16_values(_bits(deq), gkv[f"kv_deq_d{d}_b{bits}"], gkv[f"kv_norms_d{d}_b{bits}"],
                      f"golden deq d{d} b{bits}")


# D = 128 from bf16 / fp16 takes the matrix-core transform (counts that are
# not multiples of the 32-vector wave step included); fp32 and D = 64 / 256
# the butterfly kernel
CASES = [(1, 128, 3, "bf16"), (37, 64, 2, "f16"), (1000, 128, 4, "f32"), (513, 256, 3, "bf16"),
         (4096, 128, 2, "bf16"), (77, 256, 4, "f16"), (300, 64, 4, "f32"), (2049, 256, 2, "f32"),
         (999, 128, 3, "f16"), (130, 128, 4, "bf16"), (33, 128, 2, "f16")]


@pytest.mark.parametrize("n,d,bits,dt", CASES)
def test_kv_kernels_match_oracle(n, d, bits, dt):
    from polarengine_vllm.kv_cache import PolarKVQuantizer
    _say(f"kv oracle n={n} d={d} bits={bits} dt={dt}")
    xt = torch.from_numpy(O.seeded_normal((n, d), 0.9, n + d + bits)).to(DTS[dt])
    x = xt.float().numpy()
    qz = PolarKVQuantizer(d, bits, DEV)
    packed, norms = qz.quantize(xt.to(DEV))
    torch.cuda.synchronize()
    wp, wn = O.kv_quantize(x, bits)
    flips = check_kv_codes(packed.cpu().numpy(), wp, x, bits, f"n{n} d{d} b{bits} {dt}")
    check_bf16_norms(_bits(norms), wn, f"n{n} d{d} b{bits} {dt}")
    deq = qz.dequantize(packed, norms, (n, d))
    torch.cuda.synchronize()
    want = O.kv_dequantize(packed.cpu().numpy(), _bits(norms), bits, d)
    check_bf16_values(_bits(deq), want, _bits(norms), f"deq n{n} d{d} b{bits}")
    # the format's approximation: cosine of the expansion with the input
    g = O.bf16_bits_to_f32(_bits(deq)).astype(np.float64)
    cos = (g * x).sum(1) / (np.linalg.norm(g, axis=1) * np.linalg.norm(x, axis=1))
    assert cos.mean() > {2: 0.92, 3: 0.97, 4: 0.99}[bits], cos.mean()
    print(f"near-tie flips: {flips}; mean cosine {cos.mean():.5f}")


def test_kv_strided_rows():
    """Input rows with ldx > D, output rows with ldo > D (a slice of a wider
    buffer): the kernels honour both strides and leave the gap untouched."""
    from polarengine_vllm import _lib
    from polarengine_vllm.kv_cache import PolarKVQuantizer
    _say("kv strided")
    n, d, bits = 200, 128, 3
    wide = torch.from_numpy(O.seeded_normal((n, 3 * d), 1.0, 9)).to(torch.bfloat16).to(DEV)
    xv = wide[:, d:2 * d]
    qz = PolarKVQuantizer(d, bits, DEV)
    packed, norms = qz.quantize(xv)
    pc, nc = qz.quantize(xv.contiguous())
    out = torch.full((n, d + 24), 7.0, dtype=torch.bfloat16, device=DEV)
    qz.dequantize(packed, norms, (n, d), out=out[:, :d])
    ref = qz.dequantize(pc, nc, (n, d))
    torch.cuda.synchronize()
    assert torch.equal(packed, pc) and torch.equal(norms, nc)
    assert torch.equal(out[:, :d], ref)
    assert bool((out[:, d:] == 7.0).all())
    L = _lib.lib()
    st = _lib.stream_ptr(torch.device(DEV))
    assert L.pe_kv_dequantize(packed.data_ptr(), norms.data_ptr(), n, d, qz.centroids.data_ptr(), bits,
                              out.data_ptr(), d + 3, st) == _lib.PE_ERR_ALIGN


def test_kv_rejects_bad_arguments():
    from polarengine_vllm import _lib
    L = _lib.lib()
    st = _lib.stream_ptr(torch.device(DEV))
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device=DEV)
    ct = torch.zeros(16, device=DEV)
    p = torch.zeros(4, 64, dtype=torch.uint8, device=DEV)
    nr = torch.zeros(4, dtype=torch.bfloat16, device=DEV)
    o = torch.zeros(4, 128, dtype=torch.bfloat16, device=DEV)
    args = (ct.data_ptr(),)
    assert L.pe_kv_quantize(x.data_ptr(), 1, 4, 96, 128, *args, 3, p.data_ptr(), nr.data_ptr(), st) == _lib.PE_ERR_DIMS
    assert L.pe_kv_quantize(x.data_ptr(), 1, 4, 128, 64, *args, 3, p.data_ptr(), nr.data_ptr(), st) == _lib.PE_ERR_DIMS
    assert L.pe_kv_quantize(x.data_ptr(), 1, 4, 128, 128, *args, 5, p.data_ptr(), nr.data_ptr(), st) == _lib.PE_ERR_BITS
    assert L.pe_kv_quantize(x.data_ptr(), 9, 4, 128, 128, *args, 3, p.data_ptr(), nr.data_ptr(), st) == _lib.PE_ERR_DTYPE
    assert L.pe_kv_quantize(None, 1, 4, 128, 128, *args, 3, p.data_ptr(), nr.data_ptr(), st) == _lib.PE_ERR_NULL
    assert L.pe_kv_dequantize(p.data_ptr(), nr.data_ptr(), 4, 128, *args, 1, o.data_ptr(), 128, st) == _lib.PE_ERR_BITS
    assert L.pe_kv_dequantize(p.data_ptr(), nr.data_ptr(), 4, 128, *args, 3, None, 128, st) == _lib.PE_ERR_NULL
    assert L.pe_kv_quantize(x.data_ptr(), 1, 0, 128, 128, *args, 3, p.data_ptr(), nr.data_ptr(), st) == _lib.PE_OK


def _expected_history(tokens: np.ndarray, residual: int, bits: int) -> tuple:
    """tokens [B, H, S, D] float32 (bf16 values) -> (packed, norms) of the
    compressed prefix in head-major token order, by the oracle."""
    b, h, s, d = tokens.shape
    sq = max(0, s - residual)
    if not sq:
        return None, None
    return O.kv_quantize(tokens[:, :, :sq].reshape(-1, d), bits)


@pytest.mark.parametrize("keep", [False, True])
@pytest.mark.parametrize("b,h,d,bits,chunks", [(2, 3, 128, 3, [40, 1, 1, 1, 20, 1]),
                                               (1, 1, 64, 2, [10, 10, 10]),
                                               (1, 4, 256, 4, [5, 300, 1, 2])])
def test_kv_layer_update(b, h, d, bits, chunks, keep):
    """The history returned after every update: the residual tokens exactly,
    the compressed ones as the expansion of the oracle's codes; compressed()
    holds the oracle's codes and norms for every token so far, in token order
    per head (the order the reference's buffer has while it holds one chunk).
    keep: with the expanded read cache (counted by memory_bytes) or without
    (the history expanded per call)."""
    from polarengine_vllm.kv_cache import PolarKVLayer, PolarKVQuantizer
    R = 16
    qz = PolarKVQuantizer(d, bits, DEV)
    layer = PolarKVLayer(qz, residual_length=R, keep_expanded=keep)
    seen = np.zeros((b, h, 0, d), np.float32)
    for step, s_new in enumerate(chunks):
        _say(f"kv layer b={b} h={h} d={d} bits={bits} keep={keep} step={step} s_new={s_new}")
        new = torch.from_numpy(O.seeded_normal((b, h, s_new, d), 1.0, 100 * step + d)).to(torch.bfloat16)
        seen = np.concatenate([seen, new.float().numpy()], axis=2)
        full = layer.update(new.to(DEV))
        torch.cuda.synchronize()
        S = seen.shape[2]
        assert tuple(full.shape) == (b, h, S, d) and full.dtype == torch.bfloat16
        assert layer.get_seq_length() == S
        r0 = max(0, S - R)
        assert torch.equal(full[:, :, r0:].cpu(), torch.from_numpy(seen[:, :, r0:]).to(torch.bfloat16))
        wp, wn = _expected_history(seen, R, bits)
        gp, gn = layer.compressed()
        if wp is None:
            assert gp is None
            continue
        flat_x = seen[:, :, :r0].reshape(-1, d)
        check_kv_codes(gp.cpu().numpy(), wp, flat_x, bits, f"layer step {step}")
        check_bf16_norms(_bits(gn), wn, f"layer step {step}")
        hist = full[:, :, :r0].reshape(-1, d)
        want = O.kv_dequantize(gp.cpu().numpy(), _bits(gn), bits, d)
        check_bf16_values(_bits(hist), want, _bits(gn), f"layer history step {step}")
        cache_bytes = layer._expanded.numel() * 2 if keep else 0
        assert (layer._expanded is not None) == keep
        assert layer.memory_bytes() == (gp.numel() + gn.numel() * 2 + b * h * min(S, R) * d * 2
                                        + cache_bytes)


def test_kv_cache_and_attention_wrapper():
    from polarengine_vllm.kv_cache import PolarKVAttentionWrapper, PolarKVCache, PolarKVConfig
    _say("kv cache + wrapper")
    cfg = PolarKVConfig(nbits=3, residual_length=8, head_dim=128, num_kv_heads=2, num_layers=3,
                        skip_layers=[1])
    cache = PolarKVCache(cfg, device=DEV)
    wrap = PolarKVAttentionWrapper(cache)
    assert not wrap.is_initialized
    k = torch.from_numpy(O.seeded_normal((1, 2, 20, 128), 1.0, 1)).to(torch.bfloat16).to(DEV)
    v = torch.from_numpy(O.seeded_normal((1, 2, 20, 128), 1.0, 2)).to(torch.bfloat16).to(DEV)
    fk, fv = wrap.update(k, v, 0)
    sk, sv = wrap.update(k, v, 1)
    assert sk is k and sv is v  # skipped layer: the caller's own K/V
    assert wrap.seen_tokens == 20 and wrap.is_initialized and wrap.get_seq_length(0) == 20
    assert cache.get_seq_length(1) == 0
    assert torch.equal(fk[:, :, 12:], k[:, :, 12:]) and torch.equal(fv[:, :, 12:], v[:, :, 12:])
    st = cache.stats()
    assert st["seq_length"] == 20 and st["compression_ratio"] > 1.0
    want_mem = 2 * (2 * 12 * (48 + 2) + 2 * 8 * 128 * 2)
    assert cache.memory_bytes() == want_mem
    # vLLM layout: [tokens, heads, D]
    seen = {}

    def attn(q, key, value, kv_cache, meta, **kw):
        seen["k"], seen["v"] = key, value
        return q

    fwd = wrap.wrap_attention_forward(attn, 2)
    kt = torch.from_numpy(O.seeded_normal((11, 2, 128), 1.0, 3)).to(torch.bfloat16).to(DEV)
    vt = torch.from_numpy(O.seeded_normal((11, 2, 128), 1.0, 4)).to(torch.bfloat16).to(DEV)
    q = torch.zeros(11, 8, 128, device=DEV)
    assert fwd(q, kt, vt, None, None) is q
    torch.cuda.synchronize()
    assert tuple(seen["k"].shape) == (11, 2, 128)
    assert torch.equal(seen["k"][3:], kt[3:]) and torch.equal(seen["v"][3:], vt[3:])
    gp, gn = cache.k_layers[2].compressed()
    wp, wn = O.kv_quantize(kt[:3].transpose(0, 1).float().cpu().numpy().reshape(-1, 128), 3)
    check_kv_codes(gp.cpu().numpy(), wp, kt[:3].transpose(0, 1).float().cpu().numpy().reshape(-1, 128),
                   3, "wrapper")
    cache.reset()
    assert cache.seen_tokens == 0 and cache.get_seq_length(0) == 0 and cache.memory_bytes() == 0
