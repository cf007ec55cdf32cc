"""CPU checks of the oracle's grouped top-k routing and bf16 output rounding
(no GPU): each is pinned by a route that a plausible mistake would fail."""

import itertools

import numpy as np
import pytest

import polar_oracle as O


def _scores(logits, scoring):
    lg = np.asarray(logits, dtype=np.float32)
    if scoring == "softmax":
        z = lg - lg.max(axis=-1, keepdims=True)
        p = np.exp(z)
        return (p / p.sum(axis=-1, keepdims=True)).astype(np.float32)
    return (1.0 / (1.0 + np.exp(-lg))).astype(np.float32)


def _brute_grouped(logits, top_k, renorm, n_group, topk_group, scoring, bias):
    """Plain-Python statement: every admissible set of kept groups is tried;
    the kept set is the one whose group scores are lexicographically best
    (ties: lower group index), then experts are ranked by sorted() on
    (-score, id)."""
    p = _scores(logits, scoring)
    t, e = p.shape
    epg = e // n_group
    ws, ids = [], []
    for r in range(t):
        rank_s = [float(np.float32(p[r, j] + (bias[j] if bias is not None else 0.0)))
                  for j in range(e)]
        gsc = []
        for g in range(n_group):
            vals = sorted(rank_s[g * epg:(g + 1) * epg], reverse=True)
            gsc.append(float(np.float32(vals[0] + vals[1])) if bias is not None else vals[0])
        best = None
        for combo in itertools.combinations(range(n_group), topk_group):
            key = sorted(((-gsc[g], g) for g in combo))
            if best is None or key < best[0]:
                best = (key, combo)
        kept = set(best[1])
        cand = sorted((-rank_s[j], j) for j in range(e) if j // epg in kept)[:top_k]
        sel = [j for _, j in cand]
        w = [float(p[r, j]) for j in sel]
        if renorm:
            s = np.float32(0.0)
            for v in w:
                s = np.float32(s + np.float32(v))
            w = [float(np.float32(v) / s) for v in w]
        ws.append(w)
        ids.append(sel)
    return np.array(ws, dtype=np.float32), np.array(ids, dtype=np.int32)


@pytest.mark.parametrize("t,e,g,tg,k,scoring,with_bias", [
    (12, 16, 4, 2, 4, "softmax", False),
    (12, 16, 4, 2, 4, "sigmoid", True),
    (9, 24, 6, 3, 5, "sigmoid", False),
    (7, 12, 3, 1, 2, "softmax", True),
    (5, 8, 8, 8, 3, "softmax", False),
])
def test_grouped_route_matches_brute_force(t, e, g, tg, k, scoring, with_bias):
    logits = O.seeded_normal((t, e), 1.0, 500 + e + g, np.float32)
    logits[0, :] = 0.5  # every score equal: ties everywhere resolve to lower ids
    bias = O.seeded_normal((e,), 0.3, 501, np.float32) if with_bias else None
    w, ids = O.moe_route_grouped(logits, k, True, g, tg, scoring, bias)
    bw, bids = _brute_grouped(logits, k, True, g, tg, scoring, bias)
    assert np.array_equal(ids, bids)
    np.testing.assert_allclose(w, bw, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
def test_grouped_route_reduces_to_plain_top_k(scoring):
    """All groups kept (no bias), or one group: the plain top-k route."""
    logits = O.seeded_normal((40, 32), 1.0, 510, np.float32)
    want_w, want_ids = O.moe_route(logits, 6, True, scoring)
    for g, tg in ((4, 4), (1, 1), (32, 32)):
        w, ids = O.moe_route_grouped(logits, 6, True, g, tg, scoring)
        assert np.array_equal(ids, want_ids), (g, tg)
        np.testing.assert_allclose(w, want_w, rtol=1e-6)


def test_grouped_route_only_kept_groups():
    logits = O.seeded_normal((64, 32), 1.0, 511, np.float32)
    bias = O.seeded_normal((32,), 0.5, 512, np.float32)
    w, ids = O.moe_route_grouped(logits, 4, False, 8, 2, "sigmoid", bias)
    p = _scores(logits, "sigmoid")
    for r in range(64):
        assert len({int(i) // 4 for i in ids[r]}) <= 2
        np.testing.assert_array_equal(w[r], p[r, ids[r]])  # unbiased scores, no renorm


def test_bf16_rounding_known_answers():
    """f32 -> bf16 bit patterns: exact values, ties to even, NaN, inf."""
    one = 1.0
    cases = {
        one: 0x3F80,
        one + 2.0 ** -8: 0x3F80,          # halfway, even below
        one + 3 * 2.0 ** -8: 0x3F82,      # halfway, even above
        one + 2.0 ** -8 + 2.0 ** -20: 0x3F81,  # just past halfway
        -2.5: 0xC020,
        float("inf"): 0x7F80,
        0.0: 0x0000,
    }
    x = np.array(list(cases), dtype=np.float32)
    got = O.f32_to_bf16_bits(x)
    assert [int(v) for v in got] == list(cases.values())
    nan = O.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_linear_apply_bf16_is_the_fp32_route_rounded():
    rng = np.random.default_rng(5)
    n, k = 48, 256
    codes = rng.integers(0, 16, (n, k)).astype(np.int8)
    norms = (np.abs(rng.standard_normal((n, 2))) * 0.2 + 0.05).astype(np.float16)
    ct = O.ct_scaled(4)
    x = O.seeded_normal((3, k), 1.0, 6, np.float32)
    bias = O.seeded_normal((n,), 0.1, 7, np.float32)
    y32 = O.hadamard_domain_matmul(codes, norms, ct, O.fwht_blocks(x))
    got = O.linear_apply(x, codes, norms, ct, k, None, out_dtype="bfloat16")
    assert np.array_equal(got, O.f32_to_bf16_bits(y32))
    gotb = O.linear_apply(x, codes, norms, ct, k, bias, out_dtype="bfloat16")
    bb = O.bf16_bits_to_f32(O.f32_to_bf16_bits(bias))
    want = O.f32_to_bf16_bits(O.bf16_bits_to_f32(O.f32_to_bf16_bits(y32)) + bb)
    assert np.array_equal(gotb, want)
    # and it is not the fp16 route
    assert not np.array_equal(got.view(np.uint16),
                              O.linear_apply(x, codes, norms, ct, k).view(np.uint16))
