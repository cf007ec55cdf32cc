"""GPU parity at the plugin boundary: bf16 activations on every dispatch
route (the reference casts any float input, linear_method.py:186, and
advertises fp16 and bf16, config.py:108-110), grouped top-k MoE routing
(moe_method.py:74-89), workspace sizing on the M = 1 fallbacks, the FWHT
cache against writes outside torch, and the reference's split-K GEMV names.

bf16 results are compared with the oracle's fp32 route rounded to bf16
(oracle.linear_apply(out_dtype="bfloat16")) at the north-star tolerance."""

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import (DEV, bf16_dev, check_close, dev_codes, dev_tiled, linear_call,
                         rand_layer, say, to_dev)

pytestmark = pytest.mark.gpu


def _bits_to_f32(y_bf16):
    return y_bf16.float().cpu().numpy()


def _want_bf16(x32, codes, norms, ct, k, bias32=None):
    wb = O.linear_apply(x32, codes, norms, ct, k, bias32, out_dtype="bfloat16")
    return O.bf16_bits_to_f32(wb)


# every route of pe_linear_forward that a test-sized matrix reaches: decode
# M = 1 (tiled and row-major, fused FWHT), decode with the K split (M = 16),
# small-M matmul (M = 40), prefill with the K split (M = 300; M = 128 and
# M = 48 on the four-wave kernel's 64-row tiles), the four-wave prefill
# (M = 2048; with 384-column tiles at N = 12200, ragged), its 64-row tiles
# in one launch (M = 300, N = 10000), and the M = 1 fallback past the decode
# kernel (K = 53248). (The M = 1 GEMV on raw x is left only for row-major
# weights past 2 GiB.)
BF16_ROUTES = [(1, 12288, 4096, 4, True), (16, 12288, 4096, 4, True), (1, 4096, 4096, 5, False),
               (40, 768, 2048, 3, True), (300, 4100, 8192, 4, True),
               (2048, 4096, 4096, 6, True), (1, 4096, 53248, 4, True),
               (2048, 12200, 2048, 3, True), (300, 10000, 2048, 4, False),
               (128, 4096, 12288, 4, True), (48, 12288, 4096, 3, True)]


@pytest.mark.parametrize("m,n,k,bits,tiled", BF16_ROUTES)
def test_bf16_linear_every_route(m, n, k, bits, tiled):
    from polarengine_vllm import _lib
    say(f"bf16 linear m={m} n={n} k={k} q{bits} tiled={tiled}")
    rng = np.random.default_rng(m + n + k)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    xd, x32 = bf16_dev(O.seeded_normal((m, k), 1.0, 600 + m, np.float32))
    bd, b32 = bf16_dev(O.seeded_normal((n,), 0.1, 601, np.float32))
    if tiled:
        dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
        fmt = (_lib.PE_PACK_NIBBLE if nib else 0) | _lib.PE_LAYOUT_TILE16
    else:
        dcodes, nib = dev_codes(codes, bits)
        dnorms = to_dev(norms)
        fmt = _lib.PE_PACK_NIBBLE if nib else 0
    y = linear_call(xd, dcodes, dnorms, ct, bits, fmt, n, bd)
    assert y.dtype == torch.bfloat16
    # every 128-row m-tile is represented
    rows = np.arange(m) if m <= 512 else np.unique(np.r_[0:64, m - 64:m, 128:m:61])
    want = _want_bf16(x32[rows], codes, norms, ct, k, b32)
    check_close(_bits_to_f32(y)[rows], want, f"bf16 route m={m} {n}x{k}")


@pytest.mark.parametrize("m", [1, 4, 16, 512])
@pytest.mark.parametrize("n,k,bits", [(12288, 4096, 4), (4096, 12288, 3), (1024, 4096, 5)])
def test_bf16_through_apply(m, n, k, bits):
    """PolarQuantLinearMethod.apply with bf16 hidden states: bf16 result."""
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    say(f"bf16 apply m={m} {n}x{k} q{bits}")
    rng = np.random.default_rng(m * 3 + n + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    layer = torch.nn.Module()
    meth = PolarQuantLinearMethod(128, bits)
    meth.create_weights(layer, k, [n], k, n, torch.bfloat16)
    layer.to(DEV)
    layer.codes.copy_(to_dev(codes))
    layer.norms.copy_(to_dev(norms))
    meth.process_weights_after_loading(layer)
    xd, x32 = bf16_dev(O.seeded_normal((m, k), 1.0, 610 + m, np.float32))
    bd, b32 = bf16_dev(O.seeded_normal((n,), 0.05, 611, np.float32))
    y = meth.apply(layer, xd, bd)
    assert y.dtype == torch.bfloat16 and y.shape == (m, n)
    check_close(_bits_to_f32(y), _want_bf16(x32, codes, norms, ct, k, b32),
                f"bf16 apply m={m} {n}x{k} q{bits}")
    meth._fwht_cache.clear()


def test_bf16_xtf_entry_and_fp32_input():
    """pe_linear_forward_xtf with a bf16 result; fp32 activations through
    apply give the reference's fp16 result."""
    from polarengine_vllm import _lib
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE, fwht_pairs
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    say("bf16 xtf entry / fp32 input")
    rng = np.random.default_rng(620)
    m, n, k, bits = 24, 2048, 1024, 4
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x32 = O.seeded_normal((m, k), 1.0, 621, np.float32)
    xt = fwht_pairs(to_dev(x32))
    dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
    fmt = _lib.PE_PACK_NIBBLE | _lib.PE_LAYOUT_TILE16
    L = _lib.lib()
    wsb = L.pe_linear_xtf_workspace_size(m, k, n, bits, fmt)
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=DEV)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    cd = to_dev(ct)
    rc = L.pe_linear_forward_xtf(xt.data_ptr(), m, k, dcodes.data_ptr(), bits, fmt,
                                 dnorms.data_ptr(), cd.data_ptr(), None, 1 << bits, None,
                                 _lib.PE_DTYPE_BF16, y.data_ptr(), n, ws.data_ptr(), wsb,
                                 _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    _lib.check(rc, "pe_linear_forward_xtf")
    check_close(_bits_to_f32(y), _want_bf16(x32, codes, norms, ct, k), "bf16 xtf")
    # fp32 activations through the plugin: transformed from fp32, fp16 out
    layer = torch.nn.Module()
    meth = PolarQuantLinearMethod(128, bits)
    meth.create_weights(layer, k, [n], k, n, torch.float32)
    layer.to(DEV)
    layer.codes.copy_(to_dev(codes))
    layer.norms.copy_(to_dev(norms))
    meth.process_weights_after_loading(layer)
    for mm in (1, m):
        yf = meth.apply(layer, to_dev(x32[:mm]))
        assert yf.dtype == torch.float16
        check_close(yf.float().cpu().numpy(),
                    O.linear_apply(x32[:mm], codes, norms, ct, k).astype(np.float32), "fp32 in")
        GLOBAL_FWHT_CACHE.clear()


# t = 600: 2400 pairs, 150 rows per expert: the prefill regime (grouped GEMM,
# bf16 expert rows for the combine) and the bucketing launch
@pytest.mark.parametrize("t", [40, 600])
def test_bf16_moe_forward(t):
    say(f"bf16 moe t={t}")
    from test_gpu_kernels import _moe_layer
    rng = np.random.default_rng(630)
    meth, layer, (w13, w2) = _moe_layer(rng, 16, 512, 384, 3, 4)
    xd, x32 = bf16_dev(O.seeded_normal((t, 512), 1.0, 631, np.float32))
    logits = O.seeded_normal((t, 16), 1.0, 632, np.float32)
    y = meth.apply(layer, xd, to_dev(logits), 4, True)
    assert y.dtype == torch.bfloat16 and y.shape == (t, 512)
    w_ref, ids_ref = O.moe_route(logits, 4, True)
    want = O.moe_forward(x32, w_ref, ids_ref, w13, w2).astype(np.float32)
    check_close(_bits_to_f32(y), want, "bf16 moe")


# ---------------------------------------------------------------------------
# grouped top-k routing
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("t,e,g,tg,k,scoring,with_bias", [
    (128, 256, 8, 4, 8, "sigmoid", True),   # DeepSeek-V3 shape
    (128, 64, 8, 3, 6, "softmax", False),
    (33, 160, 20, 5, 6, "softmax", True),   # 8 experts per group, odd T
    (9, 32, 32, 32, 4, "sigmoid", False),   # one expert per group, all kept
    (7, 16, 1, 1, 2, "softmax", False),     # one group
])
def test_grouped_route_matches_oracle(t, e, g, tg, k, scoring, with_bias):
    from polarengine_vllm.moe_method import PolarQuantMoEMethod
    say(f"grouped route t={t} e={e} g={g} tg={tg} k={k} {scoring} bias={with_bias}")
    logits = O.seeded_normal((t, e), 1.0, 640 + e, np.float32)
    logits[0, :] = 0.125  # all equal: group and expert ties
    bias = O.seeded_normal((e,), 0.2, 641, np.float32) if with_bias else None
    w_ref, ids_ref = O.moe_route_grouped(logits, k, True, g, tg, scoring, bias)
    meth = PolarQuantMoEMethod(128, 3, 4)
    w, ids = meth.select_experts(to_dev(logits), k, True, scoring,
                                 None if bias is None else to_dev(bias), True, g, tg)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)


def test_grouped_route_rejects_bad_groups():
    from polarengine_vllm import _lib
    L = _lib.lib()
    lg = torch.zeros(4, 64, device=DEV)
    w = torch.empty(4, 8, device=DEV)
    ids = torch.empty(4, 8, dtype=torch.int32, device=DEV)
    st = _lib.stream_ptr(torch.device(DEV))
    for g, tg, k in ((7, 2, 8), (8, 9, 8), (8, 1, 9), (128, 2, 2), (0, 1, 1)):
        assert L.pe_moe_route_grouped(lg.data_ptr(), 4, 64, k, 1, 0, None, g, tg, w.data_ptr(),
                                      ids.data_ptr(), st) == _lib.PE_ERR_DIMS, (g, tg, k)


def test_moe_apply_grouped_topk():
    say("moe apply grouped top-k")
    from test_gpu_kernels import _moe_layer
    rng = np.random.default_rng(650)
    meth, layer, (w13, w2) = _moe_layer(rng, 32, 256, 256, 3, 4)
    x = O.seeded_normal((20, 256), 1.0, 651)
    logits = O.seeded_normal((20, 32), 1.0, 652, np.float32)
    bias = O.seeded_normal((32,), 0.3, 653, np.float32)
    y = meth.apply(layer, to_dev(x), to_dev(logits), 4, True, use_grouped_topk=True,
                   topk_group=2, num_expert_group=8, scoring_func="sigmoid",
                   e_score_correction_bias=to_dev(bias))
    w_ref, ids_ref = O.moe_route_grouped(logits, 4, True, 8, 2, "sigmoid", bias)
    want = O.moe_forward(x, w_ref, ids_ref, w13, w2).astype(np.float32)
    check_close(y.float().cpu().numpy(), want, "moe grouped")


# ---------------------------------------------------------------------------
# Workspace sizing on the M = 1 fallbacks
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("tiled", [True, False])
def test_m1_wide_k_fallback(tiled):
    """K = 53248 (a wide down projection): too many activation registers for
    the decode kernel at M = 1, and past the M = 1 GEMV's LDS budget: FWHT
    into the workspace, then the small-M matmul, with exactly the queried
    workspace."""
    from polarengine_vllm import _lib
    say(f"M=1 K=53248 fallback tiled={tiled}")
    rng = np.random.default_rng(660)
    n, k, bits = 1024, 53248, 4
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((1, k), 1.0, 661)
    bias = O.seeded_normal((n,), 0.1, 662)
    if tiled:
        dcodes, dnorms, _ = dev_tiled(codes, norms, bits)
        fmt = _lib.PE_PACK_NIBBLE | _lib.PE_LAYOUT_TILE16
    else:
        dcodes, _ = dev_codes(codes, bits)
        dnorms = to_dev(norms)
        fmt = _lib.PE_PACK_NIBBLE
    assert _lib.lib().pe_linear_workspace_size(1, k, n, bits, fmt) >= k * 2
    y = linear_call(to_dev(x), dcodes, dnorms, ct, bits, fmt, n, to_dev(bias))
    want = O.linear_apply(x, codes, norms, ct, k, bias)
    check_close(y.float().cpu().numpy(), want.astype(np.float32), f"M=1 K={k} tiled={tiled}")


def test_polar_matmul_m1_int8_wide_k():
    """Reference API at M = 1, int8 codes, K = 28672 (past the M = 1 GEMV's
    int8 budget): the repacked activation needs the queried workspace."""
    from polarengine_vllm.kernels.polar_gemm import polar_matmul
    say("polar_matmul M=1 int8 K=28672")
    rng = np.random.default_rng(670)
    n, k, bits = 512, 28672, 5
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x_tf = O.fwht_blocks(rng.standard_normal((1, k)).astype(np.float32))
    y = polar_matmul(to_dev(codes), to_dev(x_tf[0]), to_dev(norms), to_dev(ct), n, k, k // 128)
    assert y.shape == (n,)
    want = O.hadamard_domain_matmul(codes, norms, ct, x_tf)[0]
    check_close(y.cpu().numpy(), want, "polar_matmul M=1 K=28672")


# ---------------------------------------------------------------------------
# FWHT cache: writes that bypass torch
# ---------------------------------------------------------------------------

def _qkv_parent(k=512, bits=5, seed=680):
    from polarengine_vllm.linear_method import PolarQuantLinearMethod

    class Lin(torch.nn.Module):
        def __init__(self, n, s):
            super().__init__()
            self.quant_method = PolarQuantLinearMethod(128, bits)
            self.quant_method.create_weights(self, k, [n], k, n, torch.float16)
            self.to(DEV)
            rng = np.random.default_rng(s)
            self.o = rand_layer(rng, n, k, bits)
            self.codes.copy_(to_dev(self.o[0]))
            self.norms.copy_(to_dev(self.o[1]))
            self.quant_method.process_weights_after_loading(self)

        def forward(self, x):
            return self.quant_method.apply(self, x)

    class Parent(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.q, self.k, self.v = Lin(256, seed), Lin(128, seed + 1), Lin(128, seed + 2)

        def forward(self, x):
            return self.q(x), self.k(x), self.v(x)

    return Parent()


def _raw_overwrite(dst, src):
    """Write src's values into dst through a raw pointer (the library's FWHT
    applied twice is the identity up to fp16 rounding: a write torch does not
    see, so dst._version is unchanged)."""
    from polarengine_vllm import _lib
    L = _lib.lib()
    tmp = torch.empty(src.shape, dtype=torch.float32, device=DEV)
    st = _lib.stream_ptr(torch.device(DEV))
    m, k = src.shape
    _lib.check(L.pe_fwht128(src.data_ptr(), _lib.PE_DTYPE_F16, m, k, k, tmp.data_ptr(),
                            _lib.PE_XTF_F32, st), "fwht")
    _lib.check(L.pe_fwht128(tmp.data_ptr(), _lib.PE_DTYPE_F32, m, k, k, dst.data_ptr(),
                            _lib.PE_XTF_F16, st), "fwht")
    torch.cuda.synchronize()


def test_fwht_cache_scoped_by_hooks_against_raw_writes():
    """M = 64: above the decode range, where the transform is materialised
    and shared through the cache."""
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE
    from polarengine_vllm.linear_method import install_fwht_cache_hooks
    say("fwht cache hooks vs raw writes")
    parent = _qkv_parent()
    assert install_fwht_cache_hooks(parent) == 1
    assert install_fwht_cache_hooks(parent) == 0  # idempotent
    import polarengine_vllm.linear_method as LM
    x = to_dev(O.seeded_normal((64, 512), 1.0, 690))
    GLOBAL_FWHT_CACHE.clear()
    calls = []
    real = LM.fwht_pairs

    def counting(t, *a, **k):
        calls.append(t.shape)
        return real(t, *a, **k)

    LM.fwht_pairs = counting
    try:
        parent(x)
        with torch.inference_mode():  # inference tensors share inside the scope too
            parent(x.clone())
    finally:
        LM.fwht_pairs = real
    assert len(calls) == 2  # one transform per parent forward, shared by q/k/v
    assert GLOBAL_FWHT_CACHE.get(x, 512) is None  # released when the forward ended
    ver = x._version
    x2 = O.seeded_normal((64, 512), 1.0, 691)
    _raw_overwrite(x, to_dev(x2))
    assert x._version == ver  # torch did not see the write
    outs = parent(x)  # the pre-hook cleared the entry: transformed afresh
    xnow = x.cpu().numpy()
    for y, lin in zip(outs, (parent.q, parent.k, parent.v)):
        c, nrm, ct = lin.o
        check_close(y.float().cpu().numpy(),
                    O.linear_apply(xnow, c, nrm, ct, 512).astype(np.float32), "after raw write")
    GLOBAL_FWHT_CACHE.clear()


def test_apply_under_inference_mode_without_hooks():
    """apply() at M = 64 (the materialised-transform range) on inference
    tensors with no scope hooks installed: no version counter is touched,
    nothing is cached, and each projection is right."""
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE
    say("apply under inference_mode, no hooks")
    parent = _qkv_parent(seed=720)
    GLOBAL_FWHT_CACHE.clear()
    with torch.inference_mode():
        x = to_dev(O.seeded_normal((64, 512), 1.0, 721))
        outs = parent(x)
        assert GLOBAL_FWHT_CACHE._result is None
        x.add_(1.0)  # in place between forwards: must not be served a stale transform
        outs2 = parent(x)
    for ys, xv in ((outs, O.seeded_normal((64, 512), 1.0, 721)), (outs2, None)):
        xnow = x.cpu().numpy() if xv is None else xv
        for y, lin in zip(ys, (parent.q, parent.k, parent.v)):
            c, nrm, ct = lin.o
            check_close(y.float().cpu().numpy(),
                        O.linear_apply(xnow, c, nrm, ct, 512).astype(np.float32), "inference")


def test_fwht_matmul_out_write_invalidates_cache():
    """The package's own raw-pointer writes into a caller tensor record a
    version bump, so a cached transform of that tensor misses (M = 64, the
    cached range)."""
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE, fwht_matmul
    say("fwht_matmul out= bumps the version")
    parent = _qkv_parent(seed=700)  # no hooks
    x = to_dev(O.seeded_normal((64, 512), 1.0, 701))
    GLOBAL_FWHT_CACHE.clear()
    parent.q(x)
    assert GLOBAL_FWHT_CACHE.get(x, 512) is not None
    fwht_matmul(to_dev(O.seeded_normal((64, 512), 1.0, 702)), out=x)
    assert GLOBAL_FWHT_CACHE.get(x, 512) is None
    y = parent.k(x)
    c, nrm, ct = parent.k.o
    check_close(y.float().cpu().numpy(),
                O.linear_apply(x.cpu().numpy(), c, nrm, ct, 512).astype(np.float32), "after out=")
    GLOBAL_FWHT_CACHE.clear()


# ---------------------------------------------------------------------------
# Reference split-K names
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [4, 5])
def test_polar_gemv_splitk_names(bits):
    from polarengine_vllm.kernels.polar_gemv_splitk import (polar_gemv_packed_splitk,
                                                            polar_gemv_splitk)
    say(f"splitk names q{bits}")
    rng = np.random.default_rng(710 + bits)
    n, k = 12288, 4096
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x_tf = O.fwht_blocks(rng.standard_normal((1, k)).astype(np.float32))[0]
    want = O.hadamard_domain_matmul(codes, norms, ct, x_tf[None])[0]
    dcodes, nib = dev_codes(codes, bits)
    outs = []
    for split_k, atomic in ((None, False), (4, False), (8, True)):
        if nib:
            y = polar_gemv_packed_splitk(dcodes, to_dev(x_tf), to_dev(norms), to_dev(ct), n,
                                         k // 2, k // 128, split_k=split_k, use_atomic=atomic)
        else:
            y = polar_gemv_splitk(dcodes, to_dev(x_tf), to_dev(norms), to_dev(ct), n, k,
                                  k // 128, split_k=split_k, use_atomic=atomic)
        check_close(y.cpu().numpy(), want, f"splitk q{bits} split_k={split_k}")
        outs.append(y)
    assert all(torch.equal(outs[0], o) for o in outs[1:])
    with pytest.raises(ValueError):
        polar_gemv_splitk(dcodes, to_dev(x_tf), to_dev(norms), to_dev(ct), n, k, k // 128,
                          split_k=0)


@pytest.mark.parametrize("m", [1, 64])
def test_apply_compiles_fullgraph(m):
    """torch.compile(fullgraph=True) of a module whose forward calls
    PolarQuantLinearMethod.apply traces through the polarengine::linear_apply
    custom op and equals the eager forward bit for bit (aot_eager: no code
    generation, the op runs the same kernels)."""
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE
    say(f"torch.compile fullgraph linear m={m}")
    parent = _qkv_parent(seed=730)
    x = to_dev(O.seeded_normal((m, 512), 1.0, 731))
    GLOBAL_FWHT_CACHE.clear()
    eager = parent(x)
    torch._dynamo.reset()
    comp = torch.compile(parent, fullgraph=True, backend="aot_eager")
    got = comp(x)
    torch.cuda.synchronize()
    for a, b in zip(got, eager):
        assert a.dtype == b.dtype and a.shape == b.shape
        assert torch.equal(a, b)
    GLOBAL_FWHT_CACHE.clear()


def test_moe_apply_compiles_fullgraph():
    """The same for PolarQuantMoEMethod.apply (polarengine::moe_routed and,
    after a traced custom routing function, polarengine::moe_given)."""
    from test_gpu_kernels import _moe_layer
    say("torch.compile fullgraph moe")
    rng = np.random.default_rng(740)
    meth, layer, _ = _moe_layer(rng, 16, 512, 384, 3, 4, True)

    class Block(torch.nn.Module):
        def __init__(self, given):
            super().__init__()
            self.given = given

        def forward(self, x, logits):
            if self.given:
                def route(hidden_states, gating_output, topk, renormalize):
                    w, ids = torch.topk(torch.softmax(gating_output.float(), -1), topk, -1)
                    return w / w.sum(-1, keepdim=True), ids
                return meth.apply(layer, x, logits, 4, True, custom_routing_function=route)
            return meth.apply(layer, x, logits, 4, True)

    x = to_dev(O.seeded_normal((48, 512), 1.0, 741))
    logits = to_dev(O.seeded_normal((48, 16), 1.0, 742, np.float32))
    for given in (False, True):
        blk = Block(given)
        eager = blk(x, logits)
        torch._dynamo.reset()
        got = torch.compile(blk, fullgraph=True, backend="aot_eager")(x, logits)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"given={given}"


def test_measurement_helpers():
    """pe_copy copies exactly (whole 16-byte units, a ragged tail of the last
    workgroup); pe_stream_read folds every word it reads: on zero data the
    fold is 0, so magic 0 makes every lane write its sink word and any other
    magic none."""
    from polarengine_vllm import _lib
    say("measurement helpers")
    L = _lib.lib()
    st = _lib.stream_ptr(torch.device(DEV))
    for nbytes in (16, 16384, (1 << 20) + 48):
        src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=DEV)
        dst = torch.zeros_like(src)
        _lib.check(L.pe_copy(dst.data_ptr(), src.data_ptr(), nbytes, st), "pe_copy")
        torch.cuda.synchronize()
        assert torch.equal(dst, src), nbytes
        zero = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
        sink = torch.full((L.pe_stream_read_sink_bytes(nbytes) // 4,), 7, dtype=torch.int32,
                          device=DEV)
        _lib.check(L.pe_stream_read(zero.data_ptr(), nbytes, sink.data_ptr(), 0x9E3779B9, st),
                   "pe_stream_read")
        torch.cuda.synchronize()
        assert bool((sink == 7).all())
        _lib.check(L.pe_stream_read(zero.data_ptr(), nbytes, sink.data_ptr(), 0, st),
                   "pe_stream_read")
        torch.cuda.synchronize()
        assert bool((sink == 0).all())


# ---------------------------------------------------------------------------
# empty batches: a serving engine can hand a layer zero tokens
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(0, 512), (3, 0, 512)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_apply_empty_batch(shape, dtype):
    """apply on zero rows returns an empty result of the right shape and
    dtype, launches nothing, and the layer still computes right afterwards."""
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    say(f"empty batch apply {shape} {dtype}")
    n, k, bits = 256, 512, 4
    codes, norms, ct = rand_layer(np.random.default_rng(640), n, k, bits)
    layer = torch.nn.Module()
    meth = PolarQuantLinearMethod(128, bits)
    meth.create_weights(layer, k, [n], k, n, dtype)
    layer.to(DEV)
    layer.codes.copy_(to_dev(codes))
    layer.norms.copy_(to_dev(norms))
    meth.process_weights_after_loading(layer)
    y0 = meth.apply(layer, torch.empty(shape, dtype=dtype, device=DEV), None)
    torch.cuda.synchronize()
    assert y0.shape == shape[:-1] + (n,) and y0.dtype == dtype
    x = O.seeded_normal((2, k), 1.0, 641, np.float32)
    xd = to_dev(x, dtype)
    y = meth.apply(layer, xd, None)
    want = O.linear_apply(xd.float().cpu().numpy(), codes, norms, ct, k)
    check_close(y.float().cpu().numpy(), want.astype(np.float32), "after an empty batch")
    meth._fwht_cache.clear()


@pytest.mark.parametrize("routed", [True, False], ids=["logits", "given_ids"])
def test_moe_apply_empty_batch(routed):
    """The MoE method on zero tokens: an empty result, nothing launched, and
    the next call is unaffected (the routing counters are left as they were)."""
    from test_gpu_kernels import _moe_layer
    say(f"empty batch moe routed={routed}")
    meth, layer, (w13, w2) = _moe_layer(np.random.default_rng(642), 16, 512, 384, 3, 4)

    def call(x, logits):
        if routed:
            return meth.apply(layer, x, logits, 4, True)

        def fixed(hidden_states, gating_output, topk, renormalize):
            w, ids = O.moe_route(gating_output.float().cpu().numpy(), topk, renormalize)
            return to_dev(w), to_dev(ids.astype(np.int32))
        return meth.apply(layer, x, logits, 4, True, custom_routing_function=fixed)

    y0 = call(torch.empty(0, 512, dtype=torch.float16, device=DEV),
              torch.empty(0, 16, dtype=torch.float32, device=DEV))
    torch.cuda.synchronize()
    assert y0.shape == (0, 512) and y0.dtype == torch.float16
    x = O.seeded_normal((9, 512), 1.0, 643, np.float32)
    logits = O.seeded_normal((9, 16), 1.0, 644, np.float32)
    xd = to_dev(x, torch.float16)
    y = call(xd, to_dev(logits))
    w_ref, ids_ref = O.moe_route(logits, 4, True)
    want = O.moe_forward(xd.float().cpu().numpy(), w_ref, ids_ref, w13, w2).astype(np.float32)
    check_close(y.float().cpu().numpy(), want, f"moe after an empty batch routed={routed}")


@pytest.mark.parametrize("m", [4, 64])
def test_apply_strided_input(m):
    """A column slice of a wider tensor (row stride above in_f, as a split of
    a fused projection's output is) gives the same result as its copy."""
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    say(f"strided input apply m={m}")
    n, k, bits = 384, 512, 4
    codes, norms, ct = rand_layer(np.random.default_rng(650 + m), n, k, bits)
    layer = torch.nn.Module()
    meth = PolarQuantLinearMethod(128, bits)
    meth.create_weights(layer, k, [n], k, n, torch.float16)
    layer.to(DEV)
    layer.codes.copy_(to_dev(codes))
    layer.norms.copy_(to_dev(norms))
    meth.process_weights_after_loading(layer)
    big = to_dev(O.seeded_normal((m, k + 192), 1.0, 651 + m, np.float32), torch.float16)
    x = big[:, 64:64 + k]
    assert not x.is_contiguous()
    y = meth.apply(layer, x, None)
    y_copy = meth.apply(layer, x.contiguous(), None)
    torch.cuda.synchronize()
    assert torch.equal(y, y_copy)
    want = O.linear_apply(x.float().cpu().numpy(), codes, norms, ct, k)
    check_close(y.float().cpu().numpy(), want.astype(np.float32), f"strided m={m}")
    meth._fwht_cache.clear()
