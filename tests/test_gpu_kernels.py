"""GPU parity: the HIP library (through its C ABI) against the CPU oracle on
identical seeded inputs.

Tolerances: fp16 outputs within normwise
||y - y_ref||_inf / ||y_ref||_inf <= 1e-2 and cosine >= 0.9999 of the fp32
oracle; code unpacking and indexing bit-exact (one-hot probe, pack kernels).
"""

import math
import sys

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import stratified_rows

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
NORMWISE_TOL = 1e-2
COS_TOL = 0.9999


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def check_close(got, want, what):
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    w = np.asarray(want, dtype=np.float64).reshape(-1)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - w).max() / max(np.abs(w).max(), 1e-30)
    cos = float(g @ w / (np.linalg.norm(g) * np.linalg.norm(w) + 1e-300))
    assert err <= NORMWISE_TOL, f"{what}: normwise err {err:.3e}"
    assert cos >= COS_TOL, f"{what}: cosine {cos:.7f}"
    return err, cos


def rand_layer(rng, n, kp, bits):
    codes = rng.integers(0, 1 << bits, (n, kp), dtype=np.int64).astype(np.uint8).view(np.int8)
    norms = (np.abs(rng.standard_normal((n, kp // 128))) * 0.2 + 0.05).astype(np.float16)
    return codes, norms, O.ct_scaled(bits)


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t if dtype is None else t.to(dtype)


def dev_codes(codes, bits):
    """Runtime layout: nibbles for bits <= 4, int8 otherwise."""
    if bits <= 4:
        return to_dev(O.pack_nibble(codes)), True
    return to_dev(codes), False


# ---------------------------------------------------------------------------
# FWHT
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,k", [(1, 4096), (4, 12288), (37, 384), (2048, 4096)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_fwht_natural_layouts(m, k, dt):
    from polarengine_vllm.kernels.fwht import fwht_matmul
    _say(f"fwht m={m} k={k} dt={dt}")
    x = torch.from_numpy(O.seeded_normal((m, k), 1.0, 11, np.float32)).to(dt)
    want = O.fwht_blocks(x.float().numpy())
    got = fwht_matmul(x.to(DEV)).float().cpu().numpy()
    tol = {torch.float32: 2e-6, torch.float16: 2e-3, torch.bfloat16: 1e-2}[dt]
    np.testing.assert_allclose(got, want, atol=tol * 4, rtol=tol)
    if dt == torch.float32:
        xi = x.to(DEV).clone()
        fwht_matmul(xi, out=xi)  # in place (the CUDA fwht_)
        np.testing.assert_allclose(xi.cpu().numpy(), want, atol=1e-5)
        fp16_out = torch.empty(m, k, dtype=torch.float16, device=DEV)
        fwht_matmul(x.to(DEV), out=fp16_out)
        np.testing.assert_allclose(fp16_out.float().cpu().numpy(), want, atol=4e-3, rtol=2e-3)


def test_fwht_pair_layout():
    from polarengine_vllm.kernels.fwht import fwht_pairs
    _say("fwht pair layout")
    x = O.seeded_normal((3, 512), 1.0, 12)
    want = O.fwht_blocks(x.astype(np.float32)).reshape(3, 4, 128)
    p = fwht_pairs(to_dev(x)).cpu().numpy().view(np.float16).reshape(3, 4, 64, 2)
    np.testing.assert_allclose(p[..., 0], want[..., :64], atol=4e-3, rtol=2e-3)
    np.testing.assert_allclose(p[..., 1], want[..., 64:], atol=4e-3, rtol=2e-3)


# ---------------------------------------------------------------------------
# Packing kernels: bit-exact
# ---------------------------------------------------------------------------

def test_pack_nibble_kernel_bit_exact():
    from polarengine_vllm.packing import pack_codes_half_block
    _say("pack_nibble")
    rng = np.random.default_rng(0)
    for shape in [(300, 4096), (7, 128), (12288, 384)]:
        c = rng.integers(0, 16, shape).astype(np.int8)
        got = pack_codes_half_block(to_dev(c)).cpu().numpy()
        assert np.array_equal(got, O.pack_nibble(c)), shape
    for v in (0, 15):
        c = np.full((64, 1024), v, dtype=np.int8)
        assert np.array_equal(pack_codes_half_block(to_dev(c)).cpu().numpy(), O.pack_nibble(c))


def test_unpack_q5_kernel_bit_exact():
    from polarengine_vllm.packing import unpack_codes_q5
    _say("unpack_q5")
    rng = np.random.default_rng(1)
    for shape in [(1, 128), (64, 2688), (513, 4096)]:
        c = rng.integers(0, 32, shape).astype(np.int8)
        got = unpack_codes_q5(to_dev(O.pack_q5(c))).cpu().numpy()
        assert np.array_equal(got, c), shape


# ---------------------------------------------------------------------------
# Code indexing probe: one-hot x_tf, unit norms -> y[n] = ct[code[n, k]]
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_indexing_probe_bit_exact(bits):
    from polarengine_vllm.kernels.polar_gemv import polar_gemv, polar_gemv_packed
    _say(f"indexing probe bits={bits}")
    rng = np.random.default_rng(2)
    n, kp = 96, 1024
    codes, _, ct = rand_layer(rng, n, kp, bits)
    norms = np.ones((n, kp // 128), dtype=np.float16)
    dcodes, nib = dev_codes(codes, bits)
    # nibble paths carry the codebook as fp16; int8 paths in fp32
    ct_k = ct.astype(np.float16).astype(np.float32) if nib else ct
    for k in (0, 1, 15, 16, 17, 63, 64, 65, 100, 127, 128 + 5, 128 * 3 + 64, kp - 1):
        x = np.zeros(kp, dtype=np.float32)
        x[k] = 1.0
        if nib:
            y = polar_gemv_packed(dcodes, to_dev(x), to_dev(norms), to_dev(ct), n, kp // 2,
                                  kp // 128)
        else:
            y = polar_gemv(dcodes, to_dev(x), to_dev(norms), to_dev(ct), n, kp, kp // 128)
        want = ct_k[codes[:, k].view(np.uint8).astype(np.int64)]
        assert np.array_equal(y.cpu().numpy(), want), f"k={k}"


# ---------------------------------------------------------------------------
# Reference-API GEMV (f32 x_tf -> f32 out), shapes of tests/test_kernel_correctness.py
# ---------------------------------------------------------------------------

SHAPES = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288), (24576, 4096),
          (2048, 8192), (512, 4096), (1000, 1408)]


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("bits", [3, 4, 5, 6])
def test_polar_gemv_reference_api(n, k, bits):
    from polarengine_vllm.kernels.polar_gemv import polar_gemv, polar_gemv_packed
    _say(f"polar_gemv n={n} k={k} bits={bits}")
    rng = np.random.default_rng(n * 7 + k + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x_tf = O.fwht_blocks(rng.standard_normal(k).astype(np.float32)[None])[0]
    want = O.hadamard_domain_matmul(codes, norms, ct, x_tf[None])[0]
    dcodes, nib = dev_codes(codes, bits)
    fn = polar_gemv_packed if nib else polar_gemv
    y = fn(dcodes, to_dev(x_tf), to_dev(norms), to_dev(ct), n, k // 2 if nib else k, k // 128)
    assert y.shape == (n,) and y.dtype == torch.float32
    check_close(y.cpu().numpy(), want, f"gemv {n}x{k} q{bits}")
    y2 = fn(dcodes, to_dev(x_tf), to_dev(norms), to_dev(ct), n, k // 2 if nib else k, k // 128)
    assert torch.equal(y, y2), "non-deterministic"


# ---------------------------------------------------------------------------
# Fused linear forward, M = 1 (FWHT in the GEMV prologue), BASELINE shapes
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,k,bits", [(4096, 4096, 5), (12288, 4096, 3), (12288, 4096, 4),
                                      (4096, 12288, 4), (4096, 12288, 3), (1024, 4096, 5),
                                      (4096, 4096, 6), (2816, 2048, 3), (2048, 1408, 4),
                                      (512, 20480, 4), (256, 9216, 5)])
def test_linear_forward_m1(n, k, bits):
    from polarengine_vllm import _lib
    _say(f"linear m=1 n={n} k={k} bits={bits}")
    rng = np.random.default_rng(3 + n + bits)
    kp = (k + 127) // 128 * 128
    codes, norms, ct = rand_layer(rng, n, kp, bits)
    x = O.seeded_normal((1, k), 1.0, 5 + bits)
    bias = O.seeded_normal((n,), 0.1, 6)
    want = O.linear_apply(x, codes, norms, ct, k, bias)
    dcodes, nib = dev_codes(codes, bits)
    # device tensors stay referenced until the kernel has run
    xd = to_dev(np.pad(x, ((0, 0), (0, kp - k))))
    nd, cd, bd = to_dev(norms), to_dev(ct), to_dev(bias)
    y = torch.empty(1, n, dtype=torch.float16, device=DEV)
    L = _lib.lib()
    rc = L.pe_linear_forward(xd.data_ptr(), 0, 1, kp, kp, dcodes.data_ptr(), bits, int(nib),
                             nd.data_ptr(), cd.data_ptr(), None, 1 << bits, bd.data_ptr(),
                             y.data_ptr(), n, None, 0, _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    _lib.check(rc, "pe_linear_forward")
    check_close(y.float().cpu().numpy(), want.astype(np.float32), f"linear m=1 {n}x{k} q{bits}")


# ---------------------------------------------------------------------------
# Decode (M <= 16): MFMA decode GEMV with the FWHT fused (raw fp16 rows) or
# fed pair-f16 x_tf; shapes with nb < 8 (idle waves), ragged N, row stride
# ldx > in_f, every bit width, and M past the LDS limit (FWHT + small GEMM)
# ---------------------------------------------------------------------------

def pair_f16(x_tf):
    """[M, K] -> pair-f16 rows as uint32 [M, K/2]: (x[128b+p], x[128b+64+p])."""
    m, k = x_tf.shape
    h = np.ascontiguousarray(
        x_tf.astype(np.float16).reshape(m, k // 128, 2, 64).transpose(0, 1, 3, 2))
    return h.view(np.uint32).reshape(m, k // 2)


DECODE_CASES = [(1, 12288, 4096, 4), (1, 4096, 4096, 5), (2, 1000, 1408, 3),
                (3, 4096, 12288, 4), (4, 257, 384, 2), (5, 96, 640, 8), (7, 2816, 2048, 6),
                (8, 12288, 4096, 4), (12, 333, 1024, 7), (16, 4096, 2048, 4),
                (16, 1536, 1536, 5), (16, 4096, 4096, 4), (1, 512, 20480, 4),
                (1, 64, 128, 3), (2, 48, 256, 8),
                # K split over workgroups (M >= 8, or activations too large for
                # LDS): fp32 partials reduced by a second kernel
                (16, 12288, 4096, 4), (16, 4096, 12288, 3), (6, 2048, 24576, 4),
                (2, 700, 40960, 2), (10, 50, 640, 6),
                # 17 <= M <= 32: two m-tiles per weight lookup, K split; M = 33..64:
                # the prefill GEMM's K split or the small-M kernel
                (17, 12288, 4096, 4), (24, 4096, 12288, 3), (32, 12288, 4096, 4),
                (48, 1000, 2048, 5), (64, 12288, 4096, 4), (64, 4096, 12288, 4),
                (33, 700, 4096, 2), (40, 96, 640, 8), (64, 50, 256, 4), (17, 16, 384, 3)]


@pytest.mark.parametrize("m,n,k,bits", DECODE_CASES)
def test_decode_linear_forward(m, n, k, bits):
    from polarengine_vllm import _lib
    _say(f"decode m={m} n={n} k={k} bits={bits}")
    rng = np.random.default_rng(m * 1000 + n + k + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 50 + m)
    bias = O.seeded_normal((n,), 0.1, 51)
    want = O.linear_apply(x, codes, norms, ct, k, bias).astype(np.float32)
    dcodes, nib = dev_codes(codes, bits)
    ldx = k + 64  # rows of a wider buffer
    xb = np.zeros((m, ldx), dtype=np.float16)
    xb[:, :k] = x
    xd, nd, cd, bd = to_dev(xb), to_dev(norms), to_dev(ct), to_dev(bias)
    L = _lib.lib()
    wsb = L.pe_linear_workspace_size(m, k, n, bits, int(nib))
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=DEV)
    ct_host = np.ascontiguousarray(ct, dtype=np.float32)  # codebook by value
    outs = []
    for host in (None, ct_host.ctypes.data, None):
        y = torch.empty(m, n, dtype=torch.float16, device=DEV)
        rc = L.pe_linear_forward(xd.data_ptr(), 0, m, k, ldx, dcodes.data_ptr(), bits, int(nib),
                                 nd.data_ptr(), cd.data_ptr(), host, 1 << bits, bd.data_ptr(),
                                 y.data_ptr(), n, ws.data_ptr(), wsb,
                                 _lib.stream_ptr(torch.device(DEV)))
        torch.cuda.synchronize()
        _lib.check(rc, "pe_linear_forward")
        outs.append(y)
    check_close(outs[0].float().cpu().numpy(), want, f"decode {m}x{n}x{k} q{bits}")
    assert torch.equal(outs[0], outs[2]), "non-deterministic"
    assert torch.equal(outs[0], outs[1]), "codebook by value differs from the device codebook"


@pytest.mark.parametrize("m,n,k,bits", [(1, 12288, 4096, 4), (4, 1000, 1408, 3),
                                        (16, 2048, 2048, 5), (9, 200, 384, 8)])
def test_decode_linear_forward_xtf(m, n, k, bits):
    """Pair-f16 x_tf given (the QKV-shared transform): pe_linear_forward_xtf."""
    from polarengine_vllm import _lib
    _say(f"decode xtf m={m} n={n} k={k} bits={bits}")
    rng = np.random.default_rng(m + n + k + bits + 7)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 60 + m)
    x_tf = O.fwht_blocks(x.astype(np.float32)).astype(np.float16)
    want = O.hadamard_domain_matmul(codes, norms, ct, x_tf.astype(np.float32))
    dcodes, nib = dev_codes(codes, bits)
    xp, nd, cd = to_dev(pair_f16(x_tf)), to_dev(norms), to_dev(ct)
    L = _lib.lib()
    wsb = L.pe_linear_xtf_workspace_size(m, k, n, bits, int(nib))
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=DEV)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    rc = L.pe_linear_forward_xtf(xp.data_ptr(), m, k, dcodes.data_ptr(), bits, int(nib),
                                 nd.data_ptr(), cd.data_ptr(), None, 1 << bits, None, 0,
                                 y.data_ptr(), n, ws.data_ptr(), wsb,
                                 _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    _lib.check(rc, "pe_linear_forward_xtf")
    check_close(y.float().cpu().numpy(), want.astype(np.float32), f"decode xtf {m}x{n}x{k}")


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_decode_indexing_probe_bit_exact(bits):
    """One-hot pair-f16 rows, unit norms: y[m, n] = fp16(ct)[code[n, k_m]] exactly."""
    from polarengine_vllm import _lib
    _say(f"decode indexing probe bits={bits}")
    rng = np.random.default_rng(12 + bits)
    m, n, kp = 5, 80, 1024
    codes, _, ct = rand_layer(rng, n, kp, bits)
    norms = np.ones((n, kp // 128), dtype=np.float16)
    dcodes, nib = dev_codes(codes, bits)
    ct16 = ct.astype(np.float16)
    ct_host = np.ascontiguousarray(ct, dtype=np.float32)  # codebook by value
    nd, cd = to_dev(norms), to_dev(ct)
    L = _lib.lib()
    ks = [0, 1, 15, 16, 17, 63, 64, 65, 100, 127, 133, 448, 575, 700, kp - 1]
    for c in range(0, len(ks), m):
        sel = (ks[c:c + m] + ks[:m])[:m]
        x_tf = np.zeros((m, kp), dtype=np.float16)
        x_tf[np.arange(m), sel] = 1.0
        xp = to_dev(pair_f16(x_tf))
        y = torch.empty(m, n, dtype=torch.float16, device=DEV)
        rc = L.pe_linear_forward_xtf(xp.data_ptr(), m, kp, dcodes.data_ptr(), bits, int(nib),
                                     nd.data_ptr(), cd.data_ptr(), ct_host.ctypes.data, 1 << bits,
                                     None, 0,
                                     y.data_ptr(), n, None, 0, _lib.stream_ptr(torch.device(DEV)))
        torch.cuda.synchronize()
        _lib.check(rc, "pe_linear_forward_xtf")
        want = np.stack([ct16[codes[:, k].view(np.uint8).astype(np.int64)] for k in sel])
        assert np.array_equal(y.cpu().numpy(), want), f"k={sel}"


# ---------------------------------------------------------------------------
# Tiled-16 runtime layout (what process_weights_after_loading produces)
# ---------------------------------------------------------------------------

def tile16_np(codes_rt, norms):
    """numpy statement of the tiled-16 layout: [tiles][nb][16][bpb] and [tiles][nb][16]."""
    n, row_bytes = codes_rt.shape
    nb = norms.shape[1]
    bpb = row_bytes // nb
    npad = (n + 15) // 16 * 16
    c = np.zeros((npad, row_bytes), dtype=codes_rt.dtype)
    c[:n] = codes_rt
    g = np.zeros((npad, nb), dtype=norms.dtype)
    g[:n] = norms
    ct = c.reshape(npad // 16, 16, nb, bpb).transpose(0, 2, 1, 3).reshape(npad, row_bytes)
    gt = g.reshape(npad // 16, 16, nb).transpose(0, 2, 1).reshape(npad, nb)
    return np.ascontiguousarray(ct), np.ascontiguousarray(gt)


def dev_tiled(codes, norms, bits):
    from polarengine_vllm.packing import tile_weights_16
    dcodes, nib = dev_codes(codes, bits)
    ct, nt = tile_weights_16(dcodes, to_dev(norms))
    return ct, nt, nib


@pytest.mark.parametrize("n,k,bits", [(37, 384, 4), (64, 256, 6), (1000, 1408, 3), (16, 128, 8)])
def test_tile_weights_bit_exact(n, k, bits):
    _say(f"tile16 n={n} k={k} bits={bits}")
    rng = np.random.default_rng(n + k)
    codes, norms, _ = rand_layer(rng, n, k, bits)
    rt = O.pack_nibble(codes) if bits <= 4 else codes
    want_c, want_n = tile16_np(np.asarray(rt), norms)
    ct, nt, _ = dev_tiled(codes, norms, bits)
    torch.cuda.synchronize()
    assert np.array_equal(ct.cpu().numpy().view(np.uint8), want_c.view(np.uint8))
    assert np.array_equal(nt.cpu().numpy().view(np.uint16), want_n.view(np.uint16))


# includes the two-m-tile decode kernel (M = 17..32) and the M = 33..64
# prefill K split on the MLP shapes
TILED_CASES = [(1, 12288, 4096, 4), (1, 4096, 12288, 3), (1, 1000, 1408, 5), (4, 257, 384, 2),
               (16, 4096, 2048, 4), (16, 4096, 4096, 4), (33, 1000, 1408, 6), (256, 1536, 1024, 4),
               (300, 200, 640, 8), (1, 48, 256, 6), (24, 4096, 12288, 3), (32, 12288, 4096, 4),
               (64, 12288, 4096, 4), (20, 1000, 1408, 5),
               # M = 33..64 on the four-wave 64-row K split with int8 codes
               (64, 6144, 4096, 5), (40, 4096, 4096, 6)]


@pytest.mark.parametrize("m,n,k,bits", TILED_CASES)
def test_linear_forward_tiled_layout(m, n, k, bits):
    """Every dispatch (decode, small GEMM, prefill GEMM) on the tiled-16 layout."""
    from polarengine_vllm import _lib
    _say(f"tiled linear m={m} n={n} k={k} bits={bits}")
    rng = np.random.default_rng(m * 7 + n + k + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 70 + m)
    bias = O.seeded_normal((n,), 0.1, 71)
    want = O.linear_apply(x, codes, norms, ct, k, bias).astype(np.float32)
    dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
    fmt = (_lib.PE_PACK_NIBBLE if nib else 0) | _lib.PE_LAYOUT_TILE16
    xd, cd, bd = to_dev(x), to_dev(ct), to_dev(bias)
    L = _lib.lib()
    wsb = L.pe_linear_workspace_size(m, k, n, bits, fmt)
    ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=DEV)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    ct_host = np.ascontiguousarray(ct, dtype=np.float32)
    rc = L.pe_linear_forward(xd.data_ptr(), 0, m, k, k, dcodes.data_ptr(), bits, fmt,
                             dnorms.data_ptr(), cd.data_ptr(), ct_host.ctypes.data, 1 << bits,
                             bd.data_ptr(),
                             y.data_ptr(), n, ws.data_ptr(), wsb, _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    _lib.check(rc, "pe_linear_forward")
    check_close(y.float().cpu().numpy(), want, f"tiled {m}x{n}x{k} q{bits}")


# ---------------------------------------------------------------------------
# Batched (M > 1): reference API polar_matmul (f32 out) and the MFMA GEMM
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k,bits", [(2, 4096, 4096, 4), (4, 12288, 4096, 3),
                                        (16, 4096, 12288, 4), (33, 1000, 1408, 5),
                                        (16, 4096, 4096, 6), (256, 12288, 4096, 4),
                                        (300, 512, 2048, 3), (64, 1024, 4096, 8)])
def test_polar_matmul_reference_api(m, n, k, bits):
    from polarengine_vllm.kernels.polar_gemm import polar_matmul
    _say(f"polar_matmul m={m} n={n} k={k} bits={bits}")
    rng = np.random.default_rng(m + n + k + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x_tf = O.fwht_blocks(rng.standard_normal((m, k)).astype(np.float32))
    want = O.hadamard_domain_matmul(codes, norms, ct, x_tf)
    dcodes, nib = dev_codes(codes, bits)
    if nib:
        y = polar_matmul(None, to_dev(x_tf), to_dev(norms), to_dev(ct), n, k, k // 128,
                         packed=True, packed_codes=dcodes, in_f_half=k // 2)
    else:
        y = polar_matmul(dcodes, to_dev(x_tf), to_dev(norms), to_dev(ct), n, k, k // 128)
    assert y.shape == (m, n) and y.dtype == torch.float32
    check_close(y.cpu().numpy(), want, f"matmul {m}x{n}x{k} q{bits}")


@pytest.mark.parametrize("m,n,k,bits", [(2048, 12288, 4096, 4), (2048, 4096, 12288, 3),
                                        (8192, 12288, 4096, 4)])
def test_prefill_gemm_full_size_row_sample(m, n, k, bits):
    """BASELINE prefill shapes on the reference row-major layout: the oracle
    checks at least one row of every 128-row m-tile (the tiled layout's
    whole outputs are in test_gpu_layer.py)."""
    from polarengine_vllm import _lib
    _say(f"prefill m={m} n={n} k={k} bits={bits}")
    rng = np.random.default_rng(bits + m)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 21)
    dcodes, nib = dev_codes(codes, bits)
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    L = _lib.lib()
    wsb = L.pe_linear_workspace_size(m, k, n, bits, int(nib))
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    xd, nd, cd = to_dev(x), to_dev(norms), to_dev(ct)
    rc = L.pe_linear_forward(xd.data_ptr(), 0, m, k, k, dcodes.data_ptr(), bits, int(nib),
                             nd.data_ptr(), cd.data_ptr(), None, 1 << bits, None,
                             y.data_ptr(), n, ws.data_ptr(), wsb,
                             _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    _lib.check(rc, "pe_linear_forward")
    rows = stratified_rows(m, seed=bits + m)  # every 128-row m-tile, all columns
    want = O.linear_apply(x[rows], codes, norms, ct, k)
    got = y[torch.from_numpy(rows).to(DEV)].float().cpu().numpy()
    check_close(got, want.astype(np.float32), f"prefill {m}x{n}x{k}")
    assert torch.isfinite(y).all()


# Mid-size M with few output tiles: the eight-wave (M < 256) or four-wave
# kernel splits K over workgroups (fp32 partial sums, ordered reduction with
# the bias); odd M and N tails exercise the unaligned partial slabs
@pytest.mark.parametrize("m,n,k,bits", [(128, 4096, 12288, 4), (96, 12288, 4096, 3),
                                        (256, 4096, 12288, 5), (200, 700, 2048, 4),
                                        (512, 4096, 12288, 4), (65, 64, 4096, 2),
                                        # four-wave kernel with the K split (M >= 256)
                                        (256, 12288, 4096, 3), (300, 4100, 8192, 4),
                                        (257, 2050, 12288, 6)])
def test_prefill_ksplit_row_sample(m, n, k, bits):
    from polarengine_vllm import _lib
    _say(f"prefill k-split m={m} n={n} k={k} bits={bits}")
    rng = np.random.default_rng(bits + m + n)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 23)
    bias = O.seeded_normal((n,), 0.1, 24)
    dcodes, nib = dev_codes(codes, bits)
    L = _lib.lib()
    wsb = L.pe_linear_workspace_size(m, k, n, bits, int(nib))
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    xd, nd, cd, bd = to_dev(x), to_dev(norms), to_dev(ct), to_dev(bias)
    outs = []
    for _ in range(2):
        y = torch.empty(m, n, dtype=torch.float16, device=DEV)
        rc = L.pe_linear_forward(xd.data_ptr(), 0, m, k, k, dcodes.data_ptr(), bits, int(nib),
                                 nd.data_ptr(), cd.data_ptr(), None, 1 << bits, bd.data_ptr(),
                                 y.data_ptr(), n, ws.data_ptr(), wsb,
                                 _lib.stream_ptr(torch.device(DEV)))
        torch.cuda.synchronize()
        _lib.check(rc, "pe_linear_forward")
        outs.append(y)
    assert torch.equal(outs[0], outs[1]), "k-split prefill not deterministic"
    rows = stratified_rows(m, seed=bits + m + n, tile=32, per_tile=2)
    want = O.linear_apply(x[rows], codes, norms, ct, k, bias)
    got = outs[0][torch.from_numpy(rows).to(DEV)].float().cpu().numpy()
    check_close(got, want.astype(np.float32), f"k-split prefill {m}x{n}x{k}")


# Shapes whose 128 x 256 tile count fills the CUs for one to four rounds take
# the four-wave prefill kernel: f16 and f32 outputs, nibble and int8 codes,
# masked small codebooks, bias, M and N tails, both weight layouts; the last
# two (nibble codes, 16-bit out) take its 384-column tiles, N ragged; the
# M = 300 ones its 64-row tiles (one round without a K split), M and N ragged.
FOUR_WAVE_CASES = [(2048, 4096, 4096, 4, "f16", False, True), (2000, 4200, 4096, 6, "f16", True, False),
                   (2048, 4096, 4096, 3, "f32", False, False), (2048, 4096, 2048, 8, "f32", False, False),
                   (1950, 4352, 1024, 2, "f16", True, True), (2048, 12200, 2048, 3, "f16", False, False),
                   (300, 10000, 2048, 3, "f16", True, False), (300, 10000, 2048, 5, "f16", False, True)]


@pytest.mark.parametrize("m,n,k,bits,out,with_bias,tiled", FOUR_WAVE_CASES)
def test_four_wave_prefill_row_sample(m, n, k, bits, out, with_bias, tiled):
    from polarengine_vllm import _lib
    _say(f"four-wave prefill m={m} n={n} k={k} bits={bits} out={out} bias={with_bias} tiled={tiled}")
    rng = np.random.default_rng(m + n + bits)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x = O.seeded_normal((m, k), 1.0, 23 + bits)
    bias = O.seeded_normal((n,), 0.1, 24) if with_bias else None
    if tiled:
        dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
        fmt = (_lib.PE_PACK_NIBBLE if nib else 0) | _lib.PE_LAYOUT_TILE16
    else:
        dcodes, nib = dev_codes(codes, bits)
        dnorms = to_dev(norms)
        fmt = _lib.PE_PACK_NIBBLE if nib else 0
    L = _lib.lib()
    cd = to_dev(ct)
    rows = stratified_rows(m, seed=m + n + bits, per_tile=2)
    if out == "f16":
        y = torch.empty(m, n, dtype=torch.float16, device=DEV)
        wsb = L.pe_linear_workspace_size(m, k, n, bits, fmt)
        ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=DEV)
        xd = to_dev(x)
        bd = to_dev(bias) if with_bias else None
        rc = L.pe_linear_forward(xd.data_ptr(), 0, m, k, k, dcodes.data_ptr(), bits, fmt,
                                 dnorms.data_ptr(), cd.data_ptr(), None, 1 << bits,
                                 bd.data_ptr() if bd is not None else None,
                                 y.data_ptr(), n, ws.data_ptr(), wsb,
                                 _lib.stream_ptr(torch.device(DEV)))
        torch.cuda.synchronize()
        _lib.check(rc, "pe_linear_forward")
        want = O.linear_apply(x[rows], codes, norms, ct, k, bias)
    else:
        # reference API: x_tf in f32, y in f32 (row-major weights only)
        assert not tiled and not with_bias
        x_tf = O.fwht_blocks(x)
        y = torch.empty(m, n, dtype=torch.float32, device=DEV)
        xt = to_dev(x_tf)
        wsb = L.pe_polar_matmul_workspace_size(m, k)
        ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device=DEV)
        rc = L.pe_polar_matmul(dcodes.data_ptr(), int(nib), xt.data_ptr(), m, dnorms.data_ptr(),
                               cd.data_ptr(), 1 << bits, y.data_ptr(), n, k,
                               ws.data_ptr(), wsb, _lib.stream_ptr(torch.device(DEV)))
        torch.cuda.synchronize()
        _lib.check(rc, "pe_polar_matmul")
        want = O.hadamard_domain_matmul(codes, norms, ct, x_tf[rows])
    got = y[torch.from_numpy(rows).to(DEV)].float().cpu().numpy()
    check_close(got, np.asarray(want, dtype=np.float32), f"four-wave {m}x{n}x{k} q{bits} {out}")
    assert torch.isfinite(y).all()


# ---------------------------------------------------------------------------
# Plugin path: PolarQuantLinearMethod with quantizer output
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m", [1, 3, 64])
@pytest.mark.parametrize("bits,n,k", [(5, 1024, 4096), (3, 2048, 1000), (4, 768, 2048),
                                      (6, 512, 512)])
def test_linear_method_apply(m, bits, n, k):
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    from polarengine_vllm.quantizer import PolarQuantizer
    _say(f"linear_method m={m} bits={bits} n={n} k={k}")
    w = torch.from_numpy(O.seeded_normal((n, k), 0.02, 31 + bits))
    q = PolarQuantizer(128).quantize_tensor(w.to(DEV), bits)
    layer = torch.nn.Module()
    meth = PolarQuantLinearMethod(128, bits)
    meth.create_weights(layer, k, [n], k, n, torch.float16)
    layer.to(DEV)
    layer.codes.copy_(q["codes"])
    layer.norms.copy_(q["norms"])
    meth.process_weights_after_loading(layer)
    assert layer.packed == (bits <= 4)
    x = O.seeded_normal((m, k), 1.0, 41)
    bias = O.seeded_normal((n,), 0.05, 42)
    y = meth.apply(layer, to_dev(x), to_dev(bias))
    assert y.shape == (m, n) and y.dtype == torch.float16
    want = O.linear_apply(x, q["codes"].cpu().numpy(), q["norms"].cpu().numpy(),
                          q["ct_scaled"].cpu().numpy(), k, bias)
    check_close(y.float().cpu().numpy(), want.astype(np.float32), "linear_method")
    meth._fwht_cache.clear()


def test_fwht_shared_across_qkv():
    """q/k/v modules on one hidden state above the decode range (M = 64):
    one transform, three projections."""
    from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE
    from polarengine_vllm.linear_method import PolarQuantLinearMethod
    _say("qkv sharing")
    rng = np.random.default_rng(9)
    k = 1024
    x = to_dev(O.seeded_normal((64, k), 1.0, 43))
    GLOBAL_FWHT_CACHE.clear()
    outs = []
    for n in (1024, 256, 256):
        codes, norms, ct = rand_layer(rng, n, k, 5)
        layer = torch.nn.Module()
        meth = PolarQuantLinearMethod(128, 5)
        meth.create_weights(layer, k, [n], k, n, torch.float16)
        layer.to(DEV)
        layer.codes.copy_(to_dev(codes))
        layer.norms.copy_(to_dev(norms))
        meth.process_weights_after_loading(layer)
        y = meth.apply(layer, x)
        outs.append((y, codes, norms, ct))
        assert GLOBAL_FWHT_CACHE.get(x, k) is not None
    for y, codes, norms, ct in outs:
        want = O.linear_apply(x.cpu().numpy(), codes, norms, ct, k)
        check_close(y.float().cpu().numpy(), want.astype(np.float32), "qkv")
    GLOBAL_FWHT_CACHE.clear()


def test_graph_replay_matches_eager():
    """The bench replays captured HIP graphs: every replay, with eager work in
    between, must equal the eager result (decode at M=1, with the transform on
    the matrix cores at M=4, the K split with its completion counters at
    M=16 and M=24 (two m-tiles), and the prefill GEMM)."""
    from polarengine_vllm import _lib
    _say("graph replay")
    rng = np.random.default_rng(12)
    L = _lib.lib()
    st = lambda: _lib.stream_ptr(torch.device(DEV))
    cases = []
    for m, n, k, bits in [(1, 4096, 4096, 4), (4, 2048, 4096, 3), (16, 12288, 4096, 4),
                          (24, 4096, 12288, 3), (80, 1024, 1024, 5)]:
        codes, norms, ct = rand_layer(rng, n, k, bits)
        dcodes, nib = dev_codes(codes, bits)
        x = to_dev(O.seeded_normal((m, k), 1.0, 50 + m))
        y = torch.empty(m, n, dtype=torch.float16, device=DEV)
        wsb = L.pe_linear_workspace_size(m, k, n, bits, int(nib))
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=DEV)
        args = (x, dcodes, to_dev(norms), to_dev(ct), y, ws, wsb, m, n, k, bits, nib)
        cases.append(args)

    def run(a):
        x, dc, nr, ct, y, ws, wsb, m, n, k, bits, nib = a
        _lib.check(L.pe_linear_forward(x.data_ptr(), 0, m, k, k, dc.data_ptr(), bits, int(nib),
                                       nr.data_ptr(), ct.data_ptr(), None, 1 << bits, None,
                                       y.data_ptr(),
                                       n, ws.data_ptr(), wsb, st()), "pe_linear_forward")

    eager = []
    for a in cases:
        run(a)
        eager.append(a[4].clone())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for a in cases:
            run(a)
    for rep in range(4):
        for a in cases:
            a[4].zero_()
        g.replay()
        torch.cuda.synchronize()
        for a, e in zip(cases, eager):
            assert torch.equal(a[4], e), f"replay {rep} differs"
        junk = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        torch.cuda.synchronize()
        del junk


# ---------------------------------------------------------------------------
# MoE: routing and the grouped quantized-expert forward (parity unpinned
# against vLLM's fused MoE, which the reference delegates to; pinned against
# the oracle's per-expert loop with the routing of nemotron_offload.py)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("with_bias", [False, True])
def test_moe_route_matches_oracle(scoring, renorm, with_bias):
    from polarengine_vllm.moe_method import PolarQuantMoEMethod
    _say(f"moe route {scoring} renorm={renorm} bias={with_bias}")
    logits = O.seeded_normal((128, 64), 1.0, 70, np.float32)
    bias = O.seeded_normal((64,), 0.5, 71, np.float32) if with_bias else None
    w_ref, ids_ref = O.moe_route(logits, 8, renorm, scoring, bias)
    meth = PolarQuantMoEMethod(128, 3, 4)
    w, ids = meth.select_experts(to_dev(logits), 8, renorm, scoring,
                                 None if bias is None else to_dev(bias))
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("t,e,k,scoring", [
    (7, 8, 2, "softmax"),      # fewer experts than one wave
    (33, 3, 3, "sigmoid"),     # top_k = E, odd E
    (50, 160, 6, "softmax"),   # 3 experts per lane on some lanes
    (9, 256, 16, "sigmoid"),   # the largest E and top_k
    (5, 64, 1, "softmax"),
])
def test_moe_route_shapes(t, e, k, scoring):
    from polarengine_vllm.moe_method import PolarQuantMoEMethod
    _say(f"moe route t={t} e={e} k={k} {scoring}")
    logits = O.seeded_normal((t, e), 1.0, 74 + e, np.float32)
    logits[0, : min(e, 4)] = 0.25  # exact ties: the lower expert id ranks first
    w_ref, ids_ref = O.moe_route(logits, k, True, scoring)
    meth = PolarQuantMoEMethod(128, 3, 4)
    w, ids = meth.select_experts(to_dev(logits), k, True, scoring)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)


def _moe_layer(rng, e, hdim, inter, b13, b2, tile=True):
    from polarengine_vllm.moe_method import PolarQuantMoEMethod
    ip = (inter + 127) // 128 * 128
    c13 = rng.integers(0, 1 << b13, (e, 2 * inter, hdim)).astype(np.int8)
    n13 = (np.abs(rng.standard_normal((e, 2 * inter, hdim // 128))) * 0.3 + 0.05).astype(np.float16)
    c2 = rng.integers(0, 1 << b2, (e, hdim, ip)).astype(np.int8)
    n2 = (np.abs(rng.standard_normal((e, hdim, ip // 128))) * 0.3 + 0.05).astype(np.float16)
    meth = PolarQuantMoEMethod(128, b13, b2, tile=tile)
    layer = torch.nn.Module()
    meth.create_weights(layer, e, hdim, inter, torch.float16)
    layer.to(DEV)
    layer.w13_codes.copy_(to_dev(c13))
    layer.w13_norms.copy_(to_dev(n13))
    layer.w2_codes.copy_(to_dev(c2))
    layer.w2_norms.copy_(to_dev(n2))
    meth.process_weights_after_loading(layer)
    oracle_w = ((c13, n13, O.ct_scaled(b13)), (c2, n2, O.ct_scaled(b2)))
    return meth, layer, oracle_w


@pytest.mark.parametrize("tile", [True, False])
@pytest.mark.parametrize("t,e,hdim,inter,k,b13,b2", [
    (128, 64, 2048, 1408, 8, 3, 4),   # the MoE config of BASELINE (C5)
    (5, 8, 256, 200, 2, 3, 4),        # I not a multiple of 128 (zero-padded h)
    (80, 4, 256, 256, 2, 4, 5),       # ~40 tokens per expert: several passes
    (3, 16, 512, 384, 1, 5, 6),       # most experts empty; int8 experts
    (40, 4, 384, 132, 3, 4, 3),       # 2I = 264 rows: w13 stays row-major
    # at least 64 rows per expert on average: 64-row passes (four m-tiles)
    (200, 4, 256, 256, 2, 3, 4),      # ~100 rows per expert, ragged
    (300, 8, 384, 200, 3, 4, 6),      # I not a multiple of 128, int8 w2
    (200, 2, 256, 384, 1, 5, 4),      # int8 w13, ~100 rows per expert
    # at least 128 rows per expert on average: the grouped prefill kernel
    # (128-row tiles of every expert in one launch per product)
    (256, 4, 256, 256, 2, 3, 4),      # ~128 rows per expert, ragged
    (1024, 4, 256, 256, 2, 3, 4),     # ~512 rows per expert, ragged
    (600, 8, 384, 256, 4, 4, 5),      # w13 over 3 blocks (odd), int8 w2
    (700, 4, 256, 384, 2, 5, 4),      # int8 w13, w2 over 3 blocks (odd)
])
def test_moe_forward_matches_oracle(t, e, hdim, inter, k, b13, b2, tile):
    _say(f"moe forward t={t} e={e} h={hdim} i={inter} k={k} q{b13}/q{b2} tile={tile}")
    rng = np.random.default_rng(t + e + hdim)
    meth, layer, (w13, w2) = _moe_layer(rng, e, hdim, inter, b13, b2, tile)
    assert layer.w13_tiled == (tile and (2 * inter) % 16 == 0)
    assert layer.w2_tiled == tile
    x = O.seeded_normal((t, hdim), 1.0, 72)
    logits = O.seeded_normal((t, e), 1.0, 73, np.float32)
    y = meth.apply(layer, to_dev(x), to_dev(logits), k, True)
    w_ref, ids_ref = O.moe_route(logits, k, True)
    want = O.moe_forward(x, w_ref, ids_ref, w13, w2).astype(np.float32)
    assert y.shape == (t, hdim) and y.dtype == torch.float16
    check_close(y.float().cpu().numpy(), want, f"moe t={t} e={e}")
    y2 = meth.apply(layer, to_dev(x), to_dev(logits), k, True)
    assert torch.equal(y, y2), "moe forward not deterministic"


# ---------------------------------------------------------------------------
# fwht_butterfly: whole-row transform of any power-of-two length
# (reference kernels/fwht.py:160-190)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_fwht_butterfly_matches_oracle(dtype):
    """pe_fwht_pow2 against the oracle's float64 butterfly for n = 1 .. 32768:
    fp32 within 2e-6 of max |y| (fp32 stages), fp16 / bf16 within one
    rounding of the output type (4e-3 / 8e-3 of max |y|); self-inverse."""
    from polarengine_vllm.kernels.fwht import fwht_butterfly
    tdt = getattr(torch, dtype)
    tol = {"float32": 2e-6, "float16": 4e-3, "bfloat16": 8e-3}[dtype]
    rng = np.random.default_rng(5)
    for logn in range(0, 16):
        n = 1 << logn
        for rows in (1, 3, 37):
            if rows * n > (1 << 21):
                continue
            _say(f"fwht_butterfly n={n} rows={rows} {dtype}")
            x = rng.standard_normal((rows, n)).astype(np.float32)
            xd = torch.from_numpy(x).to(tdt).to(DEV)
            y = fwht_butterfly(xd)
            assert y.dtype == tdt and y.shape == xd.shape
            want = O.fwht_butterfly(xd.float().cpu().numpy())
            err = np.abs(y.float().cpu().numpy() - want).max() / max(np.abs(want).max(), 1e-30)
            assert err <= tol, f"n={n} rows={rows}: normwise err {err:.3e}"
            if dtype == "float32":
                back = fwht_butterfly(y).cpu().numpy()
                assert np.abs(back - x).max() <= 4e-6 * max(np.abs(x).max(), 1.0)
    # the 128 case agrees with the blockwise kernel (fwht_matmul) to fp32 rounding
    x = torch.from_numpy(rng.standard_normal((64, 128)).astype(np.float32)).to(DEV)
    from polarengine_vllm.kernels.fwht import fwht_matmul
    assert torch.allclose(fwht_butterfly(x), fwht_matmul(x), atol=1e-5)
