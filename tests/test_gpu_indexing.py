"""Bit-exact code and norm indexing on every kernel family, on both weight
layouts: row-major (the reference's, packing.py:22-60) and tiled-16 (what
process_weights_after_loading produces).

Linear routes. Row m of the transformed activation is one-hot at k_m
(x_tf[m, k_m] = 1) and every norm is a power of two, so each output is ONE
exact product and every other term an exact zero:

    y[m, n] = round16(ct16[code[n, k_m]] * norm[n, k_m // 128])

(ct16: the codebook in fp16, the matrix cores' operand type). A wrong code
(nibble order, block, row, slab, tile, the 3-bit mask) or a wrong norm gives
another value, so the outputs are compared with np.array_equal. The rows of
one call probe different k; with M >= K every k of the matrix is probed,
otherwise a list that holds the half-block and slab edges (0, 63, 64, 127,
128, ...) and k in every K group of a split.

The raw-activation routes (FWHT fused into the decode GEMV) take rows that
are one row of the unnormalised Hadamard matrix times 1/8 in one 128-block:
their transform is v * e_{k} exactly (the butterfly adds equal magnitudes),
v = 16 / sqrt(128) rounded to fp16, and y = round16(ct16 * norm * v).

Each case names its kernel for a 256-CU MI355X (the planner's choice is a
function of the CU count); the probe is exact whatever kernel runs.

Matches: the reference's indexing probe idea, tests/test_kernel_correctness.py
:86-108 (Hadamard-domain product), and the nibble layout of packing.py:22-60.
"""

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import DEV, dev_codes, pair_f16, say, to_dev

pytestmark = pytest.mark.gpu

NIB_BITS = (2, 3, 4)
I8_BITS = (5, 6, 8)
ALL_BITS = NIB_BITS + I8_BITS


def _codes(rng, n, kp, bits):
    return rng.integers(0, 1 << bits, (n, kp), dtype=np.int64).astype(np.uint8).view(np.int8)


def _pow2_norms(n, nb, seed=0):
    """Powers of two 1/4 .. 4 that differ between neighbouring rows and blocks."""
    r = np.arange(n)[:, None]
    b = np.arange(nb)[None, :]
    e = (r * 3 + b * 5 + seed) % 5 - 2
    return np.ldexp(np.ones((n, nb)), e).astype(np.float16)


def _weights(codes, norms, bits, tiled):
    """Device codes and norms in the runtime layout, and the format flags."""
    from polarengine_vllm import _lib
    from polarengine_vllm.packing import tile_weights_16
    dcodes, nib = dev_codes(codes, bits)
    dnorms = to_dev(norms)
    if tiled:
        dcodes, dnorms = tile_weights_16(dcodes, dnorms)
    fmt = (_lib.PE_PACK_NIBBLE if nib else 0) | (_lib.PE_LAYOUT_TILE16 if tiled else 0)
    return dcodes, dnorms, fmt


def _expect(codes, norms, ct, ks, scale=1.0, out="f16"):
    """[M, N] exact expectation: round(ct16[code[n, k_m]] * norm[n, k_m // 128] * scale)."""
    ct16 = ct.astype(np.float16).astype(np.float32)
    cu = codes.view(np.uint8)[:, ks].astype(np.int64)         # [N, M]
    val = ct16[cu] * norms.astype(np.float32)[:, ks // 128]   # exact: pow2 norms
    val = (val * np.float32(scale)).astype(np.float32).T      # one rounding below
    if out == "f32":
        return val
    if out == "bf16":
        return torch.from_numpy(np.ascontiguousarray(val)).to(torch.bfloat16).float().numpy()
    return val.astype(np.float16)


def _probe_ks(m, kp, seed):
    """Row m's one-hot position: every k when m >= kp (a seeded permutation,
    repeated), else the half-block / slab / block edges first, then seeded
    fill, all distinct."""
    rng = np.random.default_rng(seed)
    if m >= kp:
        reps = -(-m // kp)
        return np.concatenate([rng.permutation(kp) for _ in range(reps)])[:m]
    edges = []
    for b in range(kp // 128):
        base = 128 * b
        edges += [base, base + 15, base + 16, base + 63, base + 64, base + 65, base + 127]
    edges = list(dict.fromkeys(e for e in edges if e < kp))
    head = [edges[i] for i in rng.permutation(len(edges))][:m]
    rest = [k for k in rng.permutation(kp) if k not in set(head)][:m - len(head)]
    return np.array(head + rest, dtype=np.int64)


def _xtf_call(xp, m, kp, dcodes, bits, fmt, dnorms, ct, ct_host, n, out_dtype=torch.float16):
    from polarengine_vllm import _lib
    L = _lib.lib()
    cd = to_dev(ct)
    y = torch.empty(m, n, dtype=out_dtype, device=DEV)
    wsb = L.pe_linear_xtf_workspace_size(m, kp, n, bits, fmt)
    ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=DEV)
    rc = L.pe_linear_forward_xtf(xp.data_ptr(), m, kp, dcodes.data_ptr(), bits, fmt,
                                 dnorms.data_ptr(), cd.data_ptr(),
                                 None if ct_host is None else ct_host.ctypes.data, 1 << bits,
                                 None, _lib.act_dtype(y), y.data_ptr(), n, ws.data_ptr(), wsb,
                                 _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    _lib.check(rc, "pe_linear_forward_xtf")
    return y


def _one_hot_pairs(m, kp, ks):
    x = np.zeros((m, kp), dtype=np.float32)
    x[np.arange(m), ks] = 1.0
    return to_dev(pair_f16(x))


def _assert_equal(got, want, what):
    if not np.array_equal(got, want):
        bad = np.argwhere(got != want)
        m, n = bad[0]
        raise AssertionError(f"{what}: {len(bad)} of {got.size} outputs differ; first at "
                             f"row {m} col {n}: got {got[m, n]!r}, want {want[m, n]!r}")


# ---------------------------------------------------------------------------
# (M, N, K, kernel at 256 CUs) through pe_linear_forward_xtf
# ---------------------------------------------------------------------------
XTF_CASES = [
    (1, 80, 1024, "decode GEMV, one m-tile"),
    (5, 96, 2048, "decode GEMV, M = 5"),
    (16, 200, 4096, "decode GEMV (K split over workgroups for the larger tables)"),
    (24, 64, 2048, "decode GEMV, two m-tiles, K split"),
    (32, 160, 1024, "decode GEMV, two m-tiles, K split"),
    (4, 96, 12288, "decode GEMV, 384 items beside a 64 KB table: swizzled rows"),
    (12, 80, 4096, "decode GEMV, 384 items beside a 64 KB table: swizzled rows"),
    (40, 200, 384, "small-M MFMA kernel (odd block count: no GEMM K split)"),
    (48, 4096, 256, "small-M MFMA kernel (two blocks: no K split)"),
    (64, 4096, 1024, "four-wave GEMM, 64 x 128 tiles, K split + ordered reduction"),
    (128, 4096, 1024, "four-wave GEMM, 64 x 128 tiles, K split"),
    (192, 4096, 1024, "four-wave GEMM, 64 x 256 tiles, K split"),
    (256, 4096, 1024, "four-wave GEMM, 128 x 128 tiles, K split"),
    (512, 4096, 2048, "four-wave GEMM, 64 x 128 tiles, one launch (short K)"),
    (512, 4096, 4608, "four-wave GEMM, 128-row tiles, K split"),
    (256, 12288, 256, "four-wave GEMM, 128 x 128 tiles, one launch"),
    (192, 12288, 256, "four-wave GEMM, 128 x 128 tiles, a third of the rows empty"),
    (320, 12288, 256, "four-wave GEMM, 64 x 256 tiles, one launch"),
    (512, 12288, 256, "four-wave GEMM, 64 x 384 tiles (nibbles), one launch"),
    (1024, 6144, 256, "four-wave GEMM, 128 x 256 tiles for 3/4 of a round (int8) / 64 x 384 (nibbles)"),
    (1536, 6144, 256, "four-wave GEMM, 64 x 128 tiles over 5 rounds (int8) / 128 x 384 (nibbles)"),
    (768, 6144, 256, "four-wave GEMM, 128 x 256 tiles for 9/16 of a round (int8) / 64 x 384 (nibbles)"),
    (2048, 4096, 256, "four-wave GEMM, 128 x 256 tiles"),
    (1024, 12288, 256, "four-wave GEMM, 128 x 384 tiles (nibbles) / 128 x 256 (int8)"),
    (512, 4096, 384, "eight-wave GEMM (odd block count)"),
    (128, 1024, 640, "eight-wave GEMM, K split (odd block count)"),
    (2048, 4096, 384, "eight-wave GEMM, 128 x 256 tiles (odd block count)"),
]


@pytest.mark.parametrize("tiled", [True, False], ids=["tile16", "rowmajor"])
@pytest.mark.parametrize("m,n,kp,kernel", XTF_CASES, ids=[f"m{c[0]}n{c[1]}k{c[2]}" for c in XTF_CASES])
def test_linear_xtf_indexing_bit_exact(m, n, kp, kernel, tiled):
    """Every route of pe_linear_forward_xtf, every code width, one-hot rows."""
    for bits in ALL_BITS:
        say(f"indexing xtf {kernel}: m={m} n={n} k={kp} bits={bits} tiled={tiled}")
        rng = np.random.default_rng(m * 131 + n + kp + bits)
        codes = _codes(rng, n, kp, bits)
        norms = _pow2_norms(n, kp // 128, bits)
        ct = O.ct_scaled(bits)
        dcodes, dnorms, fmt = _weights(codes, norms, bits, tiled)
        ks = _probe_ks(m, kp, bits + m)
        xp = _one_hot_pairs(m, kp, ks)
        host_ct = np.ascontiguousarray(ct, dtype=np.float32)
        for ct_host in ((host_ct, None) if m <= 32 else (host_ct,)):
            y = _xtf_call(xp, m, kp, dcodes, bits, fmt, dnorms, ct, ct_host, n)
            _assert_equal(y.cpu().numpy(), _expect(codes, norms, ct, ks),
                          f"{kernel} bits={bits} tiled={tiled} ct_host={ct_host is not None}")


@pytest.mark.parametrize("m,n,kp", [(1, 80, 1024), (16, 200, 4096), (48, 4096, 256),
                                    (128, 4096, 1024), (256, 12288, 256), (1024, 12288, 256),
                                    (512, 4096, 384), (512, 12288, 256), (512, 4096, 2048),
                                    (1024, 6144, 256)])
def test_linear_xtf_indexing_bf16_out(m, n, kp):
    """The bf16 epilogues: y = bf16(ct16 * norm), one rounding."""
    for bits in (3, 4, 6):
        say(f"indexing xtf bf16 out: m={m} n={n} k={kp} bits={bits}")
        rng = np.random.default_rng(m + n + kp + 7 * bits)
        codes = _codes(rng, n, kp, bits)
        norms = _pow2_norms(n, kp // 128, 1)
        ct = O.ct_scaled(bits)
        dcodes, dnorms, fmt = _weights(codes, norms, bits, True)
        ks = _probe_ks(m, kp, 3 * bits + m)
        y = _xtf_call(_one_hot_pairs(m, kp, ks), m, kp, dcodes, bits, fmt, dnorms, ct,
                      np.ascontiguousarray(ct, dtype=np.float32), n, out_dtype=torch.bfloat16)
        _assert_equal(y.float().cpu().numpy(), _expect(codes, norms, ct, ks, out="bf16"),
                      f"bf16 out bits={bits}")


# ---------------------------------------------------------------------------
# Raw activations: the decode GEMV with the FWHT fused into its prologue
# ---------------------------------------------------------------------------

def _hadamard_row_inputs(m, kp, ks):
    """x[m] = H128u[k_m % 128, :] / 8 in block k_m // 128, zero elsewhere, whose
    normalised block transform is 16 / sqrt(128) at k_m and exactly 0 elsewhere."""
    j = np.arange(128)
    x = np.zeros((m, kp), dtype=np.float32)
    for r, k in enumerate(ks):
        b, i = divmod(int(k), 128)
        sign = 1.0 - 2.0 * (np.array([bin(i & jj).count("1") & 1 for jj in j], dtype=np.float32))
        x[r, 128 * b:128 * b + 128] = sign / 8.0
    return x


# (4, 96, 12288) and (12, 80, 4096): 384 items, which beside a 64 KB table
# (4-bit and int8 codes) fill the LDS only without the per-row pad, so the
# activation rows are swizzled instead
RAW_CASES = [(1, 80, 1024), (1, 4096, 4096), (4, 96, 2048), (16, 200, 4096), (24, 64, 2048),
             (32, 160, 1024), (4, 96, 12288), (12, 80, 4096)]


@pytest.mark.parametrize("tiled", [True, False], ids=["tile16", "rowmajor"])
@pytest.mark.parametrize("m,n,kp", RAW_CASES)
def test_linear_raw_x_indexing_bit_exact(m, n, kp, tiled):
    """pe_linear_forward with the transform fused (butterfly at one item per
    lane group, matrix cores from two): y = round16(ct16 * norm * v)."""
    from polarengine_vllm import _lib
    L = _lib.lib()
    v16 = float(np.float16(16.0 / np.sqrt(128.0)))
    for bits in ALL_BITS:
        say(f"indexing raw x: m={m} n={n} k={kp} bits={bits} tiled={tiled}")
        rng = np.random.default_rng(m * 7 + n + kp + bits)
        codes = _codes(rng, n, kp, bits)
        norms = _pow2_norms(n, kp // 128, 2)
        ct = O.ct_scaled(bits)
        dcodes, dnorms, fmt = _weights(codes, norms, bits, tiled)
        calls = [_probe_ks(m, kp, bits + 11 * m)]
        if m == 1:  # one k per call: walk the edge list
            calls = [np.array([k]) for k in _probe_ks(12, kp, bits)]
        for ks in calls:
            x = to_dev(_hadamard_row_inputs(m, kp, ks), torch.float16)
            y = torch.empty(m, n, dtype=torch.float16, device=DEV)
            cd = to_dev(ct)
            host_ct = np.ascontiguousarray(ct, dtype=np.float32)
            wsb = L.pe_linear_workspace_size(m, kp, n, bits, fmt)
            ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=DEV)
            rc = L.pe_linear_forward(x.data_ptr(), _lib.PE_DTYPE_F16, m, kp, kp,
                                     dcodes.data_ptr(), bits, fmt, dnorms.data_ptr(),
                                     cd.data_ptr(), host_ct.ctypes.data, 1 << bits, None,
                                     y.data_ptr(), n, ws.data_ptr(), wsb,
                                     _lib.stream_ptr(torch.device(DEV)))
            torch.cuda.synchronize()
            _lib.check(rc, "pe_linear_forward")
            _assert_equal(y.cpu().numpy(), _expect(codes, norms, ct, ks, scale=v16),
                          f"raw x m={m} bits={bits} tiled={tiled} ks={list(ks[:4])}")


# ---------------------------------------------------------------------------
# Reference API: pe_polar_matmul (fp32 x_tf, fp32 out, row-major weights)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,kp", [(2, 96, 1024), (48, 1024, 512), (100, 1024, 384),
                                    (2048, 4096, 256)])
def test_polar_matmul_indexing_bit_exact(m, n, kp):
    """fp32 output routes (small-M kernel, eight-wave and four-wave GEMMs):
    y = ct16 * norm exactly."""
    from polarengine_vllm import _lib
    L = _lib.lib()
    for bits in ALL_BITS:
        say(f"indexing polar_matmul: m={m} n={n} k={kp} bits={bits}")
        rng = np.random.default_rng(m + 3 * n + kp + bits)
        codes = _codes(rng, n, kp, bits)
        norms = _pow2_norms(n, kp // 128, 3)
        ct = O.ct_scaled(bits)
        dcodes, nib = dev_codes(codes, bits)
        ks = _probe_ks(m, kp, bits * 5 + m)
        x = np.zeros((m, kp), dtype=np.float32)
        x[np.arange(m), ks] = 1.0
        xd, nd, cd = to_dev(x), to_dev(norms), to_dev(ct)
        out = torch.empty(m, n, dtype=torch.float32, device=DEV)
        wsb = L.pe_polar_matmul_workspace_size(m, kp)
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=DEV)
        rc = L.pe_polar_matmul(dcodes.data_ptr(), int(nib), xd.data_ptr(), m, nd.data_ptr(),
                               cd.data_ptr(), 1 << bits, out.data_ptr(), n, kp, ws.data_ptr(),
                               wsb, _lib.stream_ptr(torch.device(DEV)))
        torch.cuda.synchronize()
        _lib.check(rc, "pe_polar_matmul")
        _assert_equal(out.cpu().numpy(), _expect(codes, norms, ct, ks, out="f32"),
                      f"polar_matmul bits={bits}")


# ---------------------------------------------------------------------------
# Grouped experts: pe_moe_forward (both expert passes), exact by construction
# ---------------------------------------------------------------------------

def _moe_probe_weights(rng, e, hdim, inter, b13, b2, ks_by_expert):
    """Expert weights whose routed output is one exact product per output.

    Token t (x = one Hadamard row / 8 in block k_t // 128, so x_tf = v e_{k_t})
    routed to expert e sees, at column k_t of w13[e]: the top code in every gate
    row and, in the up rows of I-block beta_e, the top or bottom code following
    Hadamard row j_e (up rows outside beta_e have zero norms). So g is the same
    for every row, h = silu(g) * u is +-a on beta_e in the pattern of row j_e
    and 0 elsewhere, and its block transform is w_e * e_{128 beta_e + j_e},
    exactly. w2[e] has non-zero norms (powers of two) only on block beta_e of
    the rows n = e (mod E), so d_e[n] = round(ct2[code2[e][n, k2_e]] * norm * w_e)
    there and 0 elsewhere; the experts' output columns never overlap. Up norms
    2^(e % 4 - 2) give w_e = w_0 * 2^(e % 4 - 2) (all roundings scale exactly).
    """
    nb_h = hdim // 128
    ip = (inter + 127) // 128 * 128
    nb_i = ip // 128
    top13 = (1 << b13) - 1
    c13 = rng.integers(0, 1 << b13, (e, 2 * inter, hdim)).astype(np.uint8)
    n13 = np.ones((e, 2 * inter, nb_h), dtype=np.float16)
    c2 = rng.integers(0, 1 << b2, (e, hdim, ip)).astype(np.uint8)
    n2 = np.zeros((e, hdim, ip // 128), dtype=np.float16)
    beta, jrow, k2, scale = [], [], [], []
    for ex in range(e):
        bt = ex % (inter // 128) if inter >= 128 else 0
        j = (37 * ex + 5) % min(128, inter - 128 * bt)
        beta.append(bt)
        jrow.append(j)
        k2.append(128 * bt + j)
        scale.append(2.0 ** (ex % 4 - 2))
        up_rows = inter + 128 * bt + np.arange(min(128, inter - 128 * bt))
        n13[ex, inter:, :] = 0
        n13[ex, up_rows, :] = scale[-1]
        sign = np.array([bin(j & i).count("1") & 1 for i in range(len(up_rows))])
        for k in ks_by_expert.get(ex, []):
            c13[ex, :inter, k] = top13
            c13[ex, up_rows, k] = np.where(sign == 0, top13, 0)
        rows = np.arange(ex, hdim, e)
        n2[ex, rows, bt] = _pow2_norms(len(rows), 1, ex)[:, 0]
    return (c13.view(np.int8), n13, c2.view(np.int8), n2, np.array(k2), np.array(scale))


def _moe_layer_from(c13, n13, c2, n2, e, hdim, inter, b13, b2, tile):
    from polarengine_vllm.moe_method import PolarQuantMoEMethod
    meth = PolarQuantMoEMethod(128, b13, b2, tile=tile)
    layer = torch.nn.Module()
    meth.create_weights(layer, e, hdim, inter, torch.float16)
    layer.to(DEV)
    layer.w13_codes.copy_(to_dev(c13))
    layer.w13_norms.copy_(to_dev(n13))
    layer.w2_codes.copy_(to_dev(c2))
    layer.w2_norms.copy_(to_dev(n2))
    meth.process_weights_after_loading(layer)
    return meth, layer


MOE_CASES = [
    # t, e, hdim, inter, k, b13, b2
    (128, 64, 2048, 1408, 8, 3, 4),   # the MoE config of BASELINE (C5)
    (64, 8, 512, 384, 4, 4, 3),
    (48, 16, 512, 256, 2, 5, 6),      # int8 experts
    (400, 8, 512, 256, 2, 3, 4),      # ~100 rows per expert: 64-row passes
    (512, 8, 1024, 256, 2, 2, 8),     # ~128 rows per expert: the grouped prefill kernel
    (40, 4, 384, 132, 3, 4, 4),       # 2I = 264 rows: w13 stays row-major
    # more rows per expert on the grouped prefill kernel
    (512, 2, 512, 256, 2, 3, 4),
    (384, 2, 512, 384, 2, 5, 4),      # int8 w13; w2 over 3 blocks (odd)
    (300, 2, 384, 256, 2, 4, 5),      # w13 over 3 blocks (odd); int8 w2
]


@pytest.mark.parametrize("tile", [True, False], ids=["tile16", "rowmajor"])
@pytest.mark.parametrize("t,e,hdim,inter,k,b13,b2", MOE_CASES)
def test_moe_indexing_bit_exact(t, e, hdim, inter, k, b13, b2, tile):
    say(f"indexing moe t={t} e={e} h={hdim} i={inter} k={k} q{b13}/q{b2} tile={tile}")
    rng = np.random.default_rng(t * 3 + e + hdim + b13)
    assert t <= hdim
    ks = rng.permutation(hdim)[:t]                       # distinct one-hot columns
    ids = np.stack([rng.permutation(e)[:k] for _ in range(t)]).astype(np.int32)
    by_e = {}
    for tok in range(t):
        for ex in ids[tok]:
            by_e.setdefault(int(ex), []).append(int(ks[tok]))
    c13, n13, c2, n2, k2, scale = _moe_probe_weights(rng, e, hdim, inter, b13, b2, by_e)
    meth, layer = _moe_layer_from(c13, n13, c2, n2, e, hdim, inter, b13, b2, tile)
    x = to_dev(_hadamard_row_inputs(t, hdim, ks), torch.float16)
    wts = np.ones((t, k), dtype=np.float32)

    def given(hidden_states, gating_output, topk, renormalize):
        return to_dev(wts), to_dev(ids)

    logits = to_dev(np.zeros((t, e), np.float32))
    y = meth.apply(layer, x, logits, k, False, custom_routing_function=given)
    got = y.float().cpu().numpy()

    # expected: out[t, n] = round16(ct2_16[c2[e][n, k2_e]] * n2[e][n, beta_e] * w_0 * s_e)
    # for e = n mod E if e is among token t's experts, else 0; w_0 (the fp16 value
    # of h's transform for s = 1) is the one unknown, found by search
    ct2 = O.ct_scaled(b2).astype(np.float16).astype(np.float32)
    cols = np.arange(hdim)
    ex_of = cols % e
    c2u = c2.view(np.uint8)
    base = ct2[c2u[ex_of, cols, k2[ex_of]].astype(np.int64)] * \
        n2[ex_of, cols, k2[ex_of] // 128].astype(np.float32) * scale[ex_of].astype(np.float32)
    member = np.zeros((t, hdim), dtype=bool)
    for tok in range(t):
        member[tok] = np.isin(ex_of, ids[tok])
    assert np.all(got[~member] == 0.0), "output columns of experts the token does not use"
    # w_0 ~ |h| * sqrt(128) with |h| = silu(g) * |u| and, for an up norm of 1,
    # g = |u| = ct_top * v: search the fp16 values nearby
    g0 = float(np.float16(O.ct_scaled(b13)[-1])) * float(np.float16(16 / np.sqrt(128)))
    a = g0 / (1 + np.exp(-g0)) * g0
    w_guess = np.float16(a * np.sqrt(128.0))
    cand = np.arange(-256, 257, dtype=np.int64) + int(w_guess.view(np.uint16))
    cand = cand[(cand > 0) & (cand < 0x7c00)].astype(np.uint16).view(np.float16)
    sel = got[member]
    bsel = np.broadcast_to(base, (t, hdim))[member]
    hits = [w for w in cand if np.array_equal((bsel * np.float32(w)).astype(np.float16)
                                              .astype(np.float32), sel)]
    assert hits, (f"no single transform value explains the expert outputs (guess {w_guess}); "
                  "a code, norm, row or expert was read from the wrong place")
