"""Pins of the CPU oracle (oracle/polar_oracle.py).

Each check is independent of the oracle's own formula: golden vectors written
by the reference's functions, closed forms, textbook tables, brute force on
tiny inputs, or a second algebraic route. A plausible slip (transposed H,
missing 1/sqrt(n), wrong nibble half, wrong Q5 bit order, off-by-one in the
argmin, norms not applied) fails at least one of them.
"""

import itertools
import math

import numpy as np
import pytest

import polar_oracle as O

# ---------------------------------------------------------------------------
# Hadamard / FWHT
# ---------------------------------------------------------------------------


def _sylvester(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]]) / math.sqrt(2.0)
    return h


def test_hadamard_matches_reference_golden(golden):
    assert np.array_equal(O.hadamard(128), golden["hadamard128"])


def test_hadamard_small_exact():
    assert np.array_equal(O.hadamard(1), np.array([[1.0]], dtype=np.float32))
    h2 = np.array([[1, 1], [1, -1]], dtype=np.float64) / math.sqrt(2)
    np.testing.assert_allclose(O.hadamard(2), h2, atol=1e-7)


@pytest.mark.parametrize("n", [2, 4, 8, 16, 32, 64, 128, 256])
def test_hadamard_is_sylvester_orthogonal_symmetric(n):
    h = O.hadamard(n).astype(np.float64)
    np.testing.assert_allclose(h, _sylvester(n), atol=1e-7)
    np.testing.assert_allclose(h @ h, np.eye(n), atol=1e-5)
    assert np.array_equal(h, h.T)


def test_hadamard_rejects_non_power_of_two():
    for n in (0, 3, 7, 100):
        with pytest.raises(AssertionError):
            O.hadamard(n)


def test_fwht_matches_reference_golden(golden):
    np.testing.assert_allclose(O.fwht_blocks(golden["fwht_in"]), golden["fwht_out"], atol=1e-6)


def test_fwht_brute_force_n8():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 8)).astype(np.float32)
    want = np.zeros_like(x, dtype=np.float64)
    for r, i, j in itertools.product(range(3), range(8), range(8)):
        want[r, i] += (-1) ** bin(i & j).count("1") * float(x[r, j])
    want /= math.sqrt(8)
    np.testing.assert_allclose(O.fwht_blocks(x, 8), want, atol=1e-6)
    np.testing.assert_allclose(O.fwht_butterfly(x), want, atol=1e-12)


def test_fwht_dense_equals_butterfly_multiblock():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((32, 128 * 4)).astype(np.float32)
    dense = O.fwht_blocks(x)
    bf = O.fwht_butterfly(x.reshape(-1, 128)).reshape(x.shape)
    np.testing.assert_allclose(dense, bf, atol=1e-5)


def test_fwht_self_inverse_and_parseval():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 384)).astype(np.float32)
    y = O.fwht_blocks(x)
    np.testing.assert_allclose(O.fwht_blocks(y), x, atol=1e-5)
    nx = np.linalg.norm(x.reshape(-1, 128), axis=1)
    ny = np.linalg.norm(y.reshape(-1, 128), axis=1)
    np.testing.assert_allclose(nx, ny, rtol=1e-5)


def test_fwht_spike_is_hadamard_row():
    x = np.zeros((1, 128), dtype=np.float32)
    x[0, 37] = 1.0
    y = O.fwht_blocks(x)[0]
    signs = np.array([(-1) ** bin(37 & j).count("1") for j in range(128)])
    np.testing.assert_allclose(y, signs / math.sqrt(128), atol=1e-7)


# ---------------------------------------------------------------------------
# Lloyd-Max codebook
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("bits", range(2, 9))
def test_centroids_match_reference_golden(golden, bits):
    assert np.array_equal(O.get_centroids(bits), golden[f"centroids_b{bits}"])


# Max (1960) / Lloyd: optimal N(0,1) quantizer levels, positive half.
_MAX_TABLE = {
    2: [0.7979],
    4: [0.4528, 1.5104],
    8: [0.2451, 0.7560, 1.3439, 2.1519],
    16: [0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6180, 2.0690, 2.7326],
}


@pytest.mark.parametrize("n", [2, 4, 8, 16])
def test_lloyd_max_converges_to_textbook_levels(n):
    c = O.lloyd_max_centroids(n, n_iter=3000).astype(np.float64)
    pos = np.sort(c[c > 0])
    np.testing.assert_allclose(pos, _MAX_TABLE[n], atol=2e-4)
    np.testing.assert_allclose(c, -c[::-1], atol=1e-6)


def test_q3_codebook_matches_ggml_constants():
    # ggml-integration/polar_quants.h:40-43 of the reference
    ggml = np.array([-2.1519461, -1.3439096, -0.7560055, -0.2450942,
                     0.2450942, 0.7560055, 1.3439096, 2.1519461], dtype=np.float32)
    np.testing.assert_allclose(O.get_centroids(3), ggml, atol=2e-6)


@pytest.mark.parametrize("bits", range(2, 7))
def test_centroid_invariants(bits):
    c = O.get_centroids(bits)
    assert c.dtype == np.float32 and c.shape == (1 << bits,)
    assert np.all(np.diff(c) > 0)
    assert abs(float(c.sum())) < 0.1
    assert not np.isnan(c).any()


def test_centroid_bits_range():
    for b in (1, 9):
        with pytest.raises(ValueError):
            O.get_centroids(b)


# ---------------------------------------------------------------------------
# Quantizer
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("bits", range(2, 7))
def test_quantizer_matches_reference_golden(golden, bits):
    q = O.quantize_tensor(golden["quant_w"].astype(np.float32), bits)
    assert np.array_equal(q["codes"], golden[f"quant_codes_b{bits}"])
    assert np.array_equal(q["norms"], golden[f"quant_norms_b{bits}"])
    assert np.array_equal(q["ct_scaled"], golden[f"quant_ct_scaled_b{bits}"])


def test_quantizer_invariants():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((8, 300)) * 0.02).astype(np.float32)
    q = O.quantize_tensor(w, 4)
    kp = 384
    wp = np.pad(w.astype(np.float64), ((0, 0), (0, kp - 300))).reshape(8, 3, 128)
    norms = np.linalg.norm(wp, axis=2)
    np.testing.assert_array_equal(q["norms"], norms.astype(np.float16))
    rot = (wp / norms[..., None]) @ _sylvester(128) * math.sqrt(128)
    ct = O.get_centroids(4).astype(np.float64)
    chosen = ct[q["codes"].reshape(8, 3, 128).astype(np.int64)]
    best = np.abs(rot[..., None] - ct).min(-1)
    assert np.all(np.abs(rot - chosen) <= best + 1e-5)
    np.testing.assert_allclose(q["ct_scaled"], O.get_centroids(4) / np.float32(math.sqrt(128)))


# ---------------------------------------------------------------------------
# Packing (bit-exact)
# ---------------------------------------------------------------------------


def test_nibble_kats():
    codes = np.zeros((128, 512), dtype=np.int8)
    b = codes.reshape(128, -1, 128)
    b[:, :, :64] = 3
    b[:, :, 64:] = 12
    assert np.all(O.pack_nibble(codes) == 0xC3)
    b[:, :, :64] = 15
    b[:, :, 64:] = 0
    assert np.all(O.pack_nibble(codes) == 0x0F)


def test_nibble_golden_and_roundtrip(golden):
    assert np.array_equal(O.pack_nibble(golden["pack_codes16"]), golden["pack_nibble"])
    rng = np.random.default_rng(4)
    c = rng.integers(0, 16, (64, 1024)).astype(np.int8)
    assert np.array_equal(O.unpack_nibble(O.pack_nibble(c)), c)
    with pytest.raises(AssertionError):
        O.pack_nibble(np.full((1, 128), 16, dtype=np.int8))


def test_q5_golden_kats_roundtrip(golden):
    assert np.array_equal(O.pack_q5(golden["pack_codes32"]), golden["pack_q5"])
    assert np.array_equal(O.unpack_q5(golden["pack_q5"]), golden["pack_codes32"])
    c = np.zeros((1, 128), dtype=np.int8)
    c[0, 1] = 31  # c1 = 0b11111 -> b0 bits 5..7 = 111, b1 bits 0..1 = 11
    p = O.pack_q5(c)
    assert p[0, 0] == 0xE0 and p[0, 1] == 0x03 and not p[0, 2:].any()
    c[0, 1] = 0
    c[0, 7] = 1  # c7 at b4 bits 3..7
    assert O.pack_q5(c)[0, 4] == 0x08
    rng = np.random.default_rng(5)
    for shape in [(1, 128), (64, 2688), (7, 1792)]:
        r = rng.integers(0, 32, shape).astype(np.int8)
        assert np.array_equal(O.unpack_q5(O.pack_q5(r)), r)


def test_q5_hlwq_golden_kats_roundtrip(golden):
    assert np.array_equal(O.pack_q5_hlwq(golden["pack_codes32"]), golden["pack_q5_hlwq"])
    assert np.array_equal(O.pack_q5_hlwq(golden["pack_codes32_odd"]), golden["pack_q5_hlwq_odd"])
    c = np.zeros((1, 8), dtype=np.int8)
    c[0, 0] = 31  # MSB-first: c0 in b0 bits 3..7
    assert O.pack_q5_hlwq(c)[0, 0] == 0xF8
    odd = golden["pack_codes32_odd"]
    back = O.unpack_q5_hlwq(golden["pack_q5_hlwq_odd"], total=odd.shape[1])
    assert np.array_equal(back, odd)


# ---------------------------------------------------------------------------
# Dequant / matmul oracles
# ---------------------------------------------------------------------------


def _rand_layer(rng, n, kp, bits):
    codes = rng.integers(0, 1 << bits, (n, kp)).astype(np.int8 if bits < 8 else np.uint8)
    norms = (np.abs(rng.standard_normal((n, kp // 128))) + 0.1).astype(np.float16)
    return codes, norms, O.ct_scaled(bits)


def test_dequant_matches_reference_converter_golden(golden):
    deq = O.dequant_weight(golden["quant_codes_b4"], golden["quant_norms_b4"],
                           golden["quant_ct_scaled_b4"])
    # the reference converter ends in a bf16 cast: one bf16 ulp
    ref = golden["dequant_b4_bf16_as_f32"]
    np.testing.assert_allclose(deq, ref, rtol=2 ** -7, atol=1e-6)


def test_dequant_reconstructs_quantized_weight():
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    q = O.quantize_tensor(w, 6)
    deq = O.dequant_weight(q["codes"], q["norms"], q["ct_scaled"])
    cos = (deq * w).sum() / np.linalg.norm(deq) / np.linalg.norm(w)
    assert cos > 0.995


@pytest.mark.parametrize("bits", [3, 5, 8])
def test_hadamard_domain_equals_dense_route(bits):
    rng = np.random.default_rng(7)
    codes, norms, ct = _rand_layer(rng, 48, 384, bits)
    x = rng.standard_normal((5, 384)).astype(np.float32)
    dense = x.astype(np.float64) @ O.dequant_weight(codes, norms, ct).astype(np.float64).T
    had = O.hadamard_domain_matmul(codes, norms, ct, O.fwht_blocks(x))
    np.testing.assert_allclose(had, dense, rtol=1e-4, atol=1e-4)


def test_hadamard_domain_row_chunks_equal_dense_route():
    """Enough rows that the product runs in three row chunks."""
    rng = np.random.default_rng(17)
    codes, norms, ct = _rand_layer(rng, 8192, 256, 4)
    x = rng.standard_normal((4300, 256)).astype(np.float32)
    dense = x.astype(np.float64) @ O.dequant_weight(codes, norms, ct).astype(np.float64).T
    had = O.hadamard_domain_matmul(codes, norms, ct, O.fwht_blocks(x))
    np.testing.assert_allclose(had, dense, rtol=1e-4, atol=1e-4)


def test_dequant_matmul_equals_linear_apply():
    rng = np.random.default_rng(19)
    w = (rng.standard_normal((72, 384)) * 0.02).astype(np.float32)
    q = O.quantize_tensor(w, 4)
    x = rng.standard_normal((6, 384)).astype(np.float16)
    bias = rng.standard_normal(72).astype(np.float16)
    wd = O.dequant_weight(q["codes"], q["norms"], q["ct_scaled"])
    got = O.dequant_matmul(x, wd, bias).astype(np.float32)
    want = O.linear_apply(x, q["codes"], q["norms"], q["ct_scaled"], 384, bias).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3)


def test_one_hot_probe_returns_codebook_entry():
    rng = np.random.default_rng(8)
    codes, _, ct = _rand_layer(rng, 16, 256, 4)
    norms = np.ones((16, 2), dtype=np.float16)
    x_tf = np.zeros((1, 256), dtype=np.float32)
    x_tf[0, 128 + 70] = 1.0
    y = O.hadamard_domain_matmul(codes, norms, ct, x_tf)[0]
    assert np.array_equal(y, ct[codes[:, 198].astype(np.int64)])


def test_linear_apply_matches_dense_with_bias_and_padding():
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((40, 200)) * 0.02).astype(np.float32)
    q = O.quantize_tensor(w, 5)
    x = rng.standard_normal((3, 200)).astype(np.float16)
    bias = rng.standard_normal(40).astype(np.float16)
    y = O.linear_apply(x, q["codes"], q["norms"], q["ct_scaled"], 200, bias)
    wd = O.dequant_weight(q["codes"], q["norms"], q["ct_scaled"])[:, :200]
    dense = (x.astype(np.float32) @ wd.T).astype(np.float16)
    want = (dense.astype(np.float32) + bias.astype(np.float32)).astype(np.float16)
    np.testing.assert_allclose(y.astype(np.float32), want.astype(np.float32), rtol=2e-3, atol=2e-3)


# ---------------------------------------------------------------------------
# MoE
# ---------------------------------------------------------------------------


def test_moe_route_invariants_and_brute_force():
    rng = np.random.default_rng(10)
    logits = rng.standard_normal((20, 16)).astype(np.float32)
    logits[0, 3] = logits[0, 5] = 9.0  # tie -> lower expert id first
    w, ids = O.moe_route(logits, 4, True)
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-6)
    assert ids[0, 0] == 3 and ids[0, 1] == 5
    for t in range(20):
        p = np.exp(logits[t] - logits[t].max())
        p /= p.sum()
        order = sorted(range(16), key=lambda e: (-p[e], e))[:4]
        assert list(ids[t]) == order
        np.testing.assert_allclose(w[t], p[order] / p[order].sum(), rtol=1e-5)
    w2, _ = O.moe_route(logits, 4, False)
    assert np.all(w2.sum(-1) < 1.0 + 1e-6)


def test_moe_forward_matches_per_token_loop():
    rng = np.random.default_rng(11)
    e, hdim, inter, t, k = 4, 256, 160, 6, 2
    kp2 = 256
    c13 = rng.integers(0, 8, (e, 2 * inter, hdim)).astype(np.int8)
    n13 = (np.abs(rng.standard_normal((e, 2 * inter, 2))) * 0.3 + 0.05).astype(np.float16)
    c2 = rng.integers(0, 16, (e, hdim, kp2)).astype(np.int8)
    n2 = (np.abs(rng.standard_normal((e, hdim, 2))) * 0.3 + 0.05).astype(np.float16)
    ct13, ct2 = O.ct_scaled(3), O.ct_scaled(4)
    x = rng.standard_normal((t, hdim)).astype(np.float16)
    w, ids = O.moe_route(rng.standard_normal((t, e)).astype(np.float32), k, True)
    got = O.moe_forward(x, w, ids, (c13, n13, ct13), (c2, n2, ct2)).astype(np.float32)
    want = np.zeros((t, hdim))
    for ti in range(t):
        for j in range(k):
            ex = ids[ti, j]
            w13 = O.dequant_weight(c13[ex], n13[ex], ct13).astype(np.float64)
            gu = w13 @ x[ti].astype(np.float64)
            g, u = gu[:inter], gu[inter:]
            hh = g / (1 + np.exp(-g)) * u
            w2 = O.dequant_weight(c2[ex], n2[ex], ct2).astype(np.float64)[:, :inter]
            want[ti] += w[ti, j] * (w2 @ hh)
    np.testing.assert_allclose(got, want, rtol=2e-2, atol=2e-3)


def test_moe_forward_duplicate_and_invalid_slots():
    """A token routed twice to one expert adds both slots (the same as one
    slot with the summed weight); ids outside 0..E-1 add nothing; a token
    without one valid slot is zero."""
    rng = np.random.default_rng(12)
    e, hdim, inter, t = 4, 128, 128, 4
    c13 = rng.integers(0, 8, (e, 2 * inter, hdim)).astype(np.int8)
    n13 = (np.abs(rng.standard_normal((e, 2 * inter, 1))) * 0.3 + 0.05).astype(np.float16)
    c2 = rng.integers(0, 16, (e, hdim, inter)).astype(np.int8)
    n2 = (np.abs(rng.standard_normal((e, hdim, 1))) * 0.3 + 0.05).astype(np.float16)
    w13, w2 = (c13, n13, O.ct_scaled(3)), (c2, n2, O.ct_scaled(4))
    x = rng.standard_normal((t, hdim)).astype(np.float16)
    ids = np.array([[1, 1], [2, -1], [-1, e], [3, 0]], np.int32)
    w = np.array([[0.25, 0.5], [0.75, 0.5], [0.5, 0.5], [0.6, 0.4]], np.float32)
    got = O.moe_forward(x, w, ids, w13, w2).astype(np.float32)
    one = O.moe_forward(x, np.array([[0.75, 0.0]] * t, np.float32),
                        np.array([[1, -1]] * t, np.int32), w13, w2).astype(np.float32)
    np.testing.assert_allclose(got[0], one[0], rtol=1e-3, atol=1e-4)
    two = O.moe_forward(x, np.array([[0.75, 0.0]] * t, np.float32),
                        np.array([[2, -1]] * t, np.int32), w13, w2).astype(np.float32)
    np.testing.assert_allclose(got[1], two[1], rtol=1e-3, atol=1e-5)
    assert np.all(got[2] == 0.0)
