"""CPU oracle for the PolarEngine quantized-linear path -- TEST INFRASTRUCTURE ONLY.

This module is a plain numpy/scipy restatement of the reference algorithm
(caiovicentino/polarengine-vllm). It exists to check the HIP product path:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker. The product package never
imports it and has no CPU fallback through it.

Every function cites the reference file:line whose behaviour it restates
(paths relative to the reference repository root).

How each function is pinned (a check that a plausible mistake would fail):

==========================  ===================================================
function                    pinned by
==========================  ===================================================
hadamard                    exact H1/H2 (tests/test_fwht.py:186-195), H@H=I,
                            symmetry, Sylvester recursion on tiny n, entries
                            bit-equal to fp32(2**-3.5)
fwht_blocks / _butterfly    dense == butterfly, self-inverse, Parseval,
                            brute-force sum on n<=8
lloyd_max_centroids         golden vectors from the reference's
                            utils.get_centroids (tests/golden), converged
                            textbook Max(1960) tables, Q3 ggml constants
                            (ggml-integration/polar_quants.h:40-43)
quantize_tensor             golden codes/norms from the reference quantizer
                            (tests/golden); argmin/normalisation invariants
pack/unpack nibble          KATs 0xC3/0x0F (tests/test_packing.py:78-108),
                            golden bytes, round trips
pack/unpack q5, q5_hlwq     golden bytes from the reference packers, round
                            trips, hand-computed single-code KATs
dequant_weight              W == blockwise (ct[c]*norm) @ H; reconstruction of
                            a quantized matrix has cosine > 0.99 to the source
hadamard_domain_matmul      equals x @ dequant_weight(...).T (two routes,
                            different algebra); one-hot probe returns
                            ct_scaled[code]*norm
linear_apply                equals the dense route; bias/half cast semantics
dequant_matmul              equals linear_apply (a different algebra: H folded
                            into W instead of applied to x)
kv_centroids                golden vectors from the reference's
                            kv_cache/cache.py get_centroids (tests/golden/
                            golden_kv.npz); symmetry, monotone levels
kv_pack / kv_unpack         golden bytes from the reference BitPacker, round
                            trips, hand-computed KATs of each bit order
kv_quantize / kv_dequantize golden packed codes, bf16 norms and bf16 outputs
                            of the reference PolarKVQuantizer (codes up to
                            fp32 near-ties of the rotation, outputs to 1 bf16
                            ulp: numpy's and torch's fp32 matmuls round
                            differently)
moe_route_grouped           equals moe_route when every group is kept (no
                            bias) and with one group; a plain-Python brute
                            force (explicit loops, sorted() on tuple keys) on
                            small cases with exact ties; vLLM itself (the
                            reference's dependency) is absent: its published
                            grouped_topk algorithm is restated, not run
linear_apply bf16 output    bf16 rounding pinned by hand-computed bit patterns
                            of f32_to_bf16_bits (RNE ties, NaN) and the fp32
                            route rounded once (bias: twice)
moe_forward                 parity unpinned against vLLM (the reference's MoE
                            compute lives in an absent dependency); pinned
                            against a per-token brute-force loop and the
                            routing invariants (weights sum to 1, top-k set)
==========================  ===================================================
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np

BLOCK_SIZE = 128

# ---------------------------------------------------------------------------
# Hadamard / FWHT
# ---------------------------------------------------------------------------


def hadamard(n: int) -> np.ndarray:
    """Normalised Sylvester Hadamard matrix, float32.

    Reference: polarengine_vllm/kernels/fwht.py:28-70 builds it recursively,
    ``[[h, h], [h, -h]] / sqrt(2)`` per level. The closed form used here is
    ``H[i, j] = (-1)**popcount(i & j) / sqrt(n)``.
    """
    if n < 1 or (n & (n - 1)) != 0:
        raise AssertionError(f"n must be a power of 2, got {n}")
    i = np.arange(n, dtype=np.int64)
    parity = np.zeros((n, n), dtype=np.int64)
    anded = i[:, None] & i[None, :]
    while anded.any():
        parity ^= anded & 1
        anded >>= 1
    sign = 1.0 - 2.0 * parity.astype(np.float64)
    return (sign / math.sqrt(n)).astype(np.float32)


def fwht_blocks(x: np.ndarray, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Blockwise FWHT as a dense product, float32.

    Reference: polarengine_vllm/kernels/fwht.py:77-108 (``fwht_matmul``):
    ``x.reshape(-1, bs) @ H`` per contiguous block of the last dimension.
    """
    x = np.asarray(x, dtype=np.float32)
    if x.shape[-1] % block_size != 0:
        raise AssertionError("in_features must be divisible by block_size")
    H = hadamard(block_size)
    return (x.reshape(-1, block_size) @ H).reshape(x.shape)


def fwht_butterfly(x: np.ndarray) -> np.ndarray:
    """In-place butterfly FWHT over the whole last dimension, float64 accumulate.

    Reference: polarengine_vllm/kernels/fwht.py:160-190 (``fwht_butterfly``):
    stages h = 1, 2, 4, ... pair (a, b) -> (a + b, a - b), then / sqrt(n).
    """
    x = np.array(x, dtype=np.float64, copy=True)
    n = x.shape[-1]
    if n < 1 or (n & (n - 1)) != 0:
        raise AssertionError(f"last dim must be power of 2, got {n}")
    lead = x.shape[:-1]
    h = 1
    while h < n:
        r = x.reshape(*lead, -1, 2 * h)
        a = r[..., :h].copy()
        b = r[..., h:].copy()
        r[..., :h] = a + b
        r[..., h:] = a - b
        x = r.reshape(*lead, n)
        h *= 2
    return x / math.sqrt(n)


# ---------------------------------------------------------------------------
# Lloyd-Max codebook
# ---------------------------------------------------------------------------

_CENTROIDS: Dict[int, np.ndarray] = {}


def lloyd_max_centroids(n_levels: int, n_iter: int = 100) -> np.ndarray:
    """Lloyd-Max levels for N(0, 1), float64 iteration, float32 result.

    Reference: polarengine_vllm/utils.py:21-68. Uniform boundaries on
    [-4, 4] with infinite ends; each iteration sets every centroid to the
    conditional mean (pdf(a) - pdf(b)) / (cdf(b) - cdf(a)) when that
    probability exceeds 1e-10 (midpoint otherwise), then boundaries to
    centroid midpoints. The reference runs exactly 100 iterations (not to
    convergence), so the count is part of the format.
    """
    from scipy.stats import norm

    boundaries = np.linspace(-4, 4, n_levels + 1)
    boundaries[0] = -np.inf
    boundaries[-1] = np.inf
    centroids = np.zeros(n_levels)
    for _ in range(n_iter):
        centroids = np.zeros(n_levels)
        for i in range(n_levels):
            a, b = boundaries[i], boundaries[i + 1]
            prob = norm.cdf(b) - norm.cdf(a)
            if prob > 1e-10:
                centroids[i] = (norm.pdf(a) - norm.pdf(b)) / prob
            else:
                centroids[i] = (a + b) / 2
        nb = np.zeros(n_levels + 1)
        nb[0] = -np.inf
        nb[-1] = np.inf
        for i in range(1, n_levels):
            nb[i] = (centroids[i - 1] + centroids[i]) / 2
        boundaries = nb
    return centroids.astype(np.float32)


def get_centroids(bits: int) -> np.ndarray:
    """Cached codebook for ``bits`` in [2, 8]. Reference: utils.py:78-100."""
    if bits < 2 or bits > 8:
        raise ValueError(f"bits must be in [2, 8], got {bits}")
    if bits not in _CENTROIDS:
        _CENTROIDS[bits] = lloyd_max_centroids(1 << bits)
    return _CENTROIDS[bits]


def ct_scaled(bits: int, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Centroids pre-divided by sqrt(block_size), float32.

    Reference: linear_method.py:131-135 and quantizer.py:251 (``ct / scale``).
    """
    return (get_centroids(bits) / np.float32(math.sqrt(block_size))).astype(np.float32)


# ---------------------------------------------------------------------------
# Quantizer
# ---------------------------------------------------------------------------


def quantize_tensor(weight: np.ndarray, bits: int, block_size: int = BLOCK_SIZE
                    ) -> Dict[str, np.ndarray]:
    """PolarQuant one matrix: normalise -> rotate -> nearest centroid.

    Reference: polarengine_vllm/quantizer.py:206-257. Pad K to a multiple of
    the block, per-block L2 norm clamped at 1e-10, unit blocks rotated by H
    and scaled by sqrt(bs), code = first index of the minimum |r - ct|.
    Returns int8 codes [N, Kp], fp16 norms [N, nb], fp32 ct_scaled [2**bits].
    """
    w = np.asarray(weight, dtype=np.float32)
    out_f, in_f = w.shape
    kp = ((in_f + block_size - 1) // block_size) * block_size
    nb = kp // block_size
    if kp != in_f:
        w = np.pad(w, ((0, 0), (0, kp - in_f)))
    blocks = w.reshape(out_f, nb, block_size)
    norms = np.sqrt((blocks.astype(np.float32) ** 2).sum(axis=2, dtype=np.float32))
    norms = np.maximum(norms, np.float32(1e-10)).astype(np.float32)
    unit = blocks / norms[:, :, None]
    H = hadamard(block_size)
    scale = np.float32(math.sqrt(block_size))
    ct = get_centroids(bits)
    codes = np.empty((out_f, nb, block_size), dtype=np.int8)
    for i in range(0, out_f, 64):
        e = min(i + 64, out_f)
        rot = (unit[i:e].reshape(-1, block_size) @ H) * scale
        d = np.abs(rot[:, :, None] - ct[None, None, :])
        codes[i:e] = d.argmin(axis=-1).astype(np.int8).reshape(e - i, nb, block_size)
    return {
        "codes": codes.reshape(out_f, kp),
        "norms": norms.astype(np.float16),
        "ct_scaled": (ct / scale).astype(np.float32),
    }


# ---------------------------------------------------------------------------
# Code packing (bit-exact integer work)
# ---------------------------------------------------------------------------


def pack_nibble(codes: np.ndarray, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Half-block nibble pack: ``byte[i] = code[bs/2 + i] << 4 | code[i]``.

    Reference: polarengine_vllm/packing.py:22-60 (and utils.py:211-260,
    kernels/polar_gemv.py:263-283, which are the same mapping).
    """
    c = np.asarray(codes).astype(np.uint8)
    if np.any(c > 15):
        raise AssertionError("All code values must be in [0, 15] for INT4 nibble packing.")
    *lead, k = c.shape
    if k % block_size:
        raise ValueError("K must be a multiple of block_size")
    half = block_size // 2
    b = c.reshape(*lead, k // block_size, block_size)
    return ((b[..., half:] << 4) | b[..., :half]).reshape(*lead, k // 2).astype(np.uint8)


def unpack_nibble(packed: np.ndarray, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Inverse of :func:`pack_nibble`. Reference: packing.py:63-94."""
    p = np.asarray(packed, dtype=np.uint8)
    *lead, kh = p.shape
    half = block_size // 2
    b = p.reshape(*lead, kh // half, half)
    lo = b & 0x0F
    hi = (b >> 4) & 0x0F
    return np.concatenate([lo, hi], axis=-1).reshape(*lead, kh * 2).astype(np.int8)


def pack_q5(codes: np.ndarray, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """On-disk Q5, LSB-first, 8 codes -> 5 bytes.

    Reference: polarengine_vllm/packing.py:97-160.
    """
    c = np.asarray(codes).astype(np.int64) & 0xFF
    if np.any(c > 31):
        raise AssertionError("All code values must be in [0, 31] for Q5 packing.")
    *lead, k = c.shape
    if k % block_size:
        raise AssertionError("K must be a multiple of block_size")
    g = c.reshape(*lead, k // 8, 8)
    c0, c1, c2, c3, c4, c5, c6, c7 = (g[..., i] for i in range(8))
    out = np.stack([
        (c0 | (c1 << 5)) & 0xFF,
        ((c1 >> 3) | (c2 << 2) | (c3 << 7)) & 0xFF,
        ((c3 >> 1) | (c4 << 4)) & 0xFF,
        ((c4 >> 4) | (c5 << 1) | (c6 << 6)) & 0xFF,
        ((c6 >> 2) | (c7 << 3)) & 0xFF,
    ], axis=-1)
    return out.astype(np.uint8).reshape(*lead, k * 5 // 8)


def unpack_q5(packed: np.ndarray, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Inverse of :func:`pack_q5`. Reference: packing.py:163-209."""
    p = np.asarray(packed).astype(np.int64)
    *lead, kp = p.shape
    if (kp * 8) % 5 or kp % (block_size * 5 // 8):
        raise AssertionError("invalid Q5 packed length")
    g = p.reshape(*lead, kp // 5, 5)
    b0, b1, b2, b3, b4 = (g[..., i] for i in range(5))
    out = np.stack([
        b0 & 0x1F,
        ((b0 >> 5) | (b1 << 3)) & 0x1F,
        (b1 >> 2) & 0x1F,
        ((b1 >> 7) | (b2 << 1)) & 0x1F,
        ((b2 >> 4) | (b3 << 4)) & 0x1F,
        (b3 >> 1) & 0x1F,
        ((b3 >> 6) | (b4 << 2)) & 0x1F,
        (b4 >> 3) & 0x1F,
    ], axis=-1)
    return out.astype(np.int8).reshape(*lead, kp * 8 // 5)


def pack_q5_hlwq(codes: np.ndarray) -> np.ndarray:
    """HLWQ ``bitpack_5``, MSB-first, zero-padded to a multiple of 8 codes.

    Reference: polarengine_vllm/packing.py:274-290.
    """
    c = np.asarray(codes).astype(np.int64)
    *lead, k = c.shape
    pad = (8 - k % 8) % 8
    if pad:
        c = np.concatenate([c, np.zeros((*lead, pad), dtype=np.int64)], axis=-1)
        k += pad
    g = c.reshape(*lead, k // 8, 8)
    c0, c1, c2, c3, c4, c5, c6, c7 = (g[..., i] for i in range(8))
    out = np.stack([
        ((c0 << 3) | (c1 >> 2)) & 0xFF,
        (((c1 & 3) << 6) | (c2 << 1) | (c3 >> 4)) & 0xFF,
        (((c3 & 0xF) << 4) | (c4 >> 1)) & 0xFF,
        (((c4 & 1) << 7) | (c5 << 2) | (c6 >> 3)) & 0xFF,
        (((c6 & 7) << 5) | c7) & 0xFF,
    ], axis=-1)
    return out.astype(np.uint8).reshape(*lead, k * 5 // 8)


def unpack_q5_hlwq(packed: np.ndarray, total: Optional[int] = None) -> np.ndarray:
    """Inverse of :func:`pack_q5_hlwq`. Reference: packing.py:229-271."""
    p = np.asarray(packed).astype(np.int64)
    *lead, kp = p.shape
    if kp % 5:
        raise AssertionError("HLWQ bit-packed codes require K_packed % 5 == 0")
    g = p.reshape(*lead, kp // 5, 5)
    b0, b1, b2, b3, b4 = (g[..., i] for i in range(5))
    out = np.stack([
        (b0 >> 3) & 0x1F,
        ((b0 & 7) << 2) | ((b1 >> 6) & 3),
        (b1 >> 1) & 0x1F,
        ((b1 & 1) << 4) | ((b2 >> 4) & 0xF),
        ((b2 & 0xF) << 1) | ((b3 >> 7) & 1),
        (b3 >> 2) & 0x1F,
        ((b3 & 3) << 3) | ((b4 >> 5) & 7),
        b4 & 0x1F,
    ], axis=-1).astype(np.int8).reshape(*lead, kp * 8 // 5)
    if total is not None:
        out = out[..., :total]
    return out


# ---------------------------------------------------------------------------
# Dequantize / matmul oracles
# ---------------------------------------------------------------------------


def _codes_u(codes: np.ndarray) -> np.ndarray:
    # torch's ct[codes.long()] with a negative int8 index wraps from the end,
    # which is the unsigned reading of the byte (bits 8 codes).
    return np.asarray(codes).astype(np.int64) & 0xFF


def dequant_weight(codes: np.ndarray, norms: np.ndarray, ct_sc: np.ndarray,
                   block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Dense fp32 weight W[N, Kp] from (codes, norms, ct_scaled).

    Reference: polarengine_vllm/kernels/polar_gemv.py:354-363 and
    weight_converter.py:34-67 (without its final bf16 cast):
    ``W = (ct_scaled[codes] * norm) @ H`` per block.
    """
    c = _codes_u(codes)
    n, kp = c.shape
    nb = kp // block_size
    vals = np.asarray(ct_sc, dtype=np.float32)[c].reshape(n, nb, block_size)
    vals = vals * np.asarray(norms, dtype=np.float32).reshape(n, nb, 1)
    H = hadamard(block_size)
    return (vals.reshape(-1, block_size) @ H).reshape(n, kp).astype(np.float32)


def hadamard_domain_matmul(codes: np.ndarray, norms: np.ndarray, ct_sc: np.ndarray,
                           x_tf: np.ndarray, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """y[m, n] = sum_b norm[n, b] * <ct_scaled[codes[n, b, :]], x_tf[m, b, :]>, fp32.

    Reference: tests/test_kernel_correctness.py:86-108 (einsum in the Hadamard
    domain) and the Triton kernels' math, polar_gemv.py:48-94.
    """
    c = _codes_u(codes)
    n, kp = c.shape
    nb = kp // block_size
    x2 = np.asarray(x_tf, dtype=np.float32).reshape(-1, kp)
    vals = np.asarray(ct_sc, dtype=np.float32)[c].reshape(n, nb, block_size)
    nrm = np.asarray(norms, dtype=np.float32)[None, :, :]
    out = np.empty((x2.shape[0], n), dtype=np.float32)
    # rows in chunks: the per-block partials [rows, n, nb] stay below ~128 MB
    step = max(1, (32 << 20) // max(1, n * nb))
    for r0 in range(0, x2.shape[0], step):
        xr = x2[r0:r0 + step].reshape(-1, nb, block_size)
        part = np.einsum("nbk,mbk->mnb", vals, xr, optimize=True)
        out[r0:r0 + step] = (part * nrm).sum(-1)
    return out


def dequant_matmul(x: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None
                   ) -> np.ndarray:
    """The reference's dense check path: y = x @ W.T in fp32 with W from
    :func:`dequant_weight` materialised once, then .half() and + bias
    (polar_gemv.py:354-363 and polar_gemm.py:607-615 build W this way; the
    fp16 cast and bias follow linear_method.py:219-221). x [M, Kp]."""
    y = (np.asarray(x, dtype=np.float32) @ np.asarray(w, dtype=np.float32).T).astype(np.float16)
    if bias is not None:
        y = (y + np.asarray(bias).astype(np.float16)).astype(np.float16)
    return y


def linear_apply(x: np.ndarray, codes: np.ndarray, norms: np.ndarray,
                 ct_sc: np.ndarray, in_f: int, bias: Optional[np.ndarray] = None,
                 block_size: int = BLOCK_SIZE, out_dtype: str = "float16") -> np.ndarray:
    """Full linear forward, fp32 compute, 16-bit result.

    Reference: polarengine_vllm/linear_method.py:184-221: x.float() -> pad to
    Kp -> blockwise FWHT -> Hadamard-domain GEMV/GEMM -> .half() -> + bias.
    out_dtype "bfloat16" casts to bf16 instead of .half() (x may then be given
    as float32 values of bf16 activations) and adds a bf16 bias the same way;
    the result is returned as bf16 bit patterns (uint16).
    """
    x2 = np.asarray(x, dtype=np.float32).reshape(-1, in_f)
    kp = np.asarray(codes).shape[1]
    if kp != in_f:
        x2 = np.pad(x2, ((0, 0), (0, kp - in_f)))
    y = hadamard_domain_matmul(codes, norms, ct_sc, fwht_blocks(x2, block_size), block_size)
    shape = (*np.asarray(x).shape[:-1], -1)
    if out_dtype == "bfloat16":
        yb = f32_to_bf16_bits(y)
        if bias is not None:
            bb = bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(bias, dtype=np.float32)))
            yb = f32_to_bf16_bits(bf16_bits_to_f32(yb) + bb)
        return yb.reshape(shape)
    y = y.astype(np.float16)
    if bias is not None:
        y = (y + np.asarray(bias).astype(np.float16)).astype(np.float16)
    return y.reshape(shape)


# ---------------------------------------------------------------------------
# MoE
# ---------------------------------------------------------------------------


def moe_route(router_logits: np.ndarray, top_k: int, renormalize: bool = True,
              scoring_func: str = "softmax",
              e_score_correction_bias: Optional[np.ndarray] = None
              ) -> Tuple[np.ndarray, np.ndarray]:
    """softmax/sigmoid -> top-k -> optional renormalise.

    Reference semantics: nemotron_offload.py:172-189 (scores, ``topk``,
    ``topk_weights / sum``) and the moe_method.py:74-78 argument list.
    Ties resolve to the lower expert index.
    """
    lg = np.asarray(router_logits, dtype=np.float32)
    if e_score_correction_bias is not None:
        lg = lg + np.asarray(e_score_correction_bias, dtype=np.float32)
    if scoring_func == "softmax":
        z = lg - lg.max(axis=-1, keepdims=True)
        p = np.exp(z)
        p = p / p.sum(axis=-1, keepdims=True)
    elif scoring_func == "sigmoid":
        p = 1.0 / (1.0 + np.exp(-lg))
    else:
        raise ValueError(f"unsupported scoring_func {scoring_func}")
    idx = np.argsort(-p, axis=-1, kind="stable")[:, :top_k]
    w = np.take_along_axis(p, idx, axis=-1)
    if renormalize:
        w = w / w.sum(axis=-1, keepdims=True)
    return w.astype(np.float32), idx.astype(np.int32)


def moe_route_grouped(router_logits: np.ndarray, top_k: int, renormalize: bool,
                      num_expert_group: int, topk_group: int, scoring_func: str = "softmax",
                      e_score_correction_bias: Optional[np.ndarray] = None
                      ) -> Tuple[np.ndarray, np.ndarray]:
    """Grouped top-k routing.

    The reference passes use_grouped_topk / num_expert_group / topk_group
    straight to vLLM's fused MoE (moe_method.py:74-89); the algorithm is that
    of vLLM's ``grouped_topk`` (fused_moe, vllm>=0.8.0 per setup.py:26; vLLM
    is not vendored): scores = softmax|sigmoid(logits); with a correction
    bias the ranking score is scores + bias and a group's score is the sum of
    its two best ranking scores, else a group's score is its best score; the
    topk_group best groups are kept; top_k experts of the kept groups by
    ranking score; weights = the unbiased scores of those experts,
    optionally renormalised. Ties resolve to the lower group / expert index;
    the result is sorted by descending ranking score.
    """
    lg = np.asarray(router_logits, dtype=np.float32)
    if scoring_func == "softmax":
        z = lg - lg.max(axis=-1, keepdims=True)
        p = np.exp(z)
        p = p / p.sum(axis=-1, keepdims=True)
    elif scoring_func == "sigmoid":
        p = 1.0 / (1.0 + np.exp(-lg))
    else:
        raise ValueError(f"unsupported scoring_func {scoring_func}")
    p = p.astype(np.float32)
    t, e = p.shape
    g = num_expert_group
    rank_s = p if e_score_correction_bias is None else (
        p + np.asarray(e_score_correction_bias, dtype=np.float32)).astype(np.float32)
    grouped = rank_s.reshape(t, g, e // g)
    if e_score_correction_bias is None:
        gscore = grouped.max(axis=-1)
    else:
        top2 = np.sort(grouped, axis=-1)[..., -2:]
        gscore = (top2[..., 1] + top2[..., 0]).astype(np.float32)
    keep_g = np.argsort(-gscore, axis=-1, kind="stable")[:, :topk_group]
    gmask = np.zeros((t, g), dtype=bool)
    np.put_along_axis(gmask, keep_g, True, axis=-1)
    emask = np.repeat(gmask, e // g, axis=-1)
    masked = np.where(emask, rank_s, -np.inf)
    idx = np.argsort(-masked, axis=-1, kind="stable")[:, :top_k]
    w = np.take_along_axis(p, idx, axis=-1)
    if renormalize:
        w = w / w.sum(axis=-1, keepdims=True)
    return w.astype(np.float32), idx.astype(np.int32)


def moe_forward(x: np.ndarray, topk_w: np.ndarray, topk_ids: np.ndarray,
                w13: Tuple[np.ndarray, np.ndarray, np.ndarray],
                w2: Tuple[np.ndarray, np.ndarray, np.ndarray],
                block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Per-expert SwiGLU MoE with PolarQuant experts, fp32, fp16 result.

    Reference semantics: nemotron_offload.py:203-226 (gate = first I columns
    of x @ w13.T, up = next I, silu(gate) * up, @ w2.T, weighted sum) with the
    weight layout of moe_method.py:56-72 (w13 [E, 2I, H], w2 [E, H, I]).
    Each expert matrix is PolarQuant (codes [E, rows, Kp] int8 unpacked,
    norms [E, rows, nb], ct_scaled [2**b]); each product follows
    :func:`linear_apply` without the final cast.
    """
    codes13, norms13, ct13 = w13
    codes2, norms2, ct2 = w2
    x = np.asarray(x, dtype=np.float32)
    t, hdim = x.shape
    e_count, two_i, _ = codes13.shape
    inter = two_i // 2
    out = np.zeros((t, hdim), dtype=np.float32)
    x_tf = fwht_blocks(x, block_size)
    kp2 = codes2.shape[2]
    for e in range(e_count):
        rows, slots = np.nonzero(topk_ids == e)
        if rows.size == 0:
            continue
        gu = hadamard_domain_matmul(codes13[e], norms13[e], ct13, x_tf[rows], block_size)
        g, u = gu[:, :inter], gu[:, inter:]
        h = (g / (1.0 + np.exp(-g))) * u
        if kp2 != inter:
            h = np.pad(h, ((0, 0), (0, kp2 - inter)))
        d = hadamard_domain_matmul(codes2[e], norms2[e], ct2, fwht_blocks(h, block_size),
                                   block_size)
        # np.add.at: a token routed to one expert in two slots adds both
        np.add.at(out, rows, topk_w[rows, slots][:, None] * d[:, :hdim])
    return out.astype(np.float16)


# ---------------------------------------------------------------------------
# KV-cache quantizer (reference: polarengine_vllm/kv_cache/cache.py)
# ---------------------------------------------------------------------------

_KV_CT: Dict[int, np.ndarray] = {}


def kv_centroids(nbits: int) -> np.ndarray:
    """Lloyd-Max levels of the KV cache, float32.

    Reference: kv_cache/cache.py:27-54. Unlike the weight codebook
    (utils.py:21-68) the interval ends are the finite +-4 of
    ``linspace(-4, 4, n + 1)``; centroids and boundaries live in float32
    tensors, so every iteration rounds them to float32; an interval with
    probability below 1e-12 takes its midpoint.
    """
    if nbits in _KV_CT:
        return _KV_CT[nbits]
    from scipy.stats import norm as sp_norm
    n = 1 << nbits
    bnd = np.linspace(-4.0, 4.0, n + 1).astype(np.float32)
    ct = np.zeros(n, dtype=np.float32)
    for _ in range(100):
        for i in range(n):
            a, b = float(bnd[i]), float(bnd[i + 1])
            pa, pb = sp_norm.cdf(a), sp_norm.cdf(b)
            if pb - pa < 1e-12:
                ct[i] = np.float32((a + b) / 2)
            else:
                ct[i] = np.float32((sp_norm.pdf(a) - sp_norm.pdf(b)) / (pb - pa))
        for i in range(1, n):
            bnd[i] = (ct[i - 1] + ct[i]) / np.float32(2)
    _KV_CT[nbits] = ct
    return ct


def kv_pack(codes: np.ndarray, nbits: int) -> np.ndarray:
    """BitPacker.pack (kv_cache/cache.py:98-128), rows of D codes, MSB first:
    2 bits 4 per byte ``c0<<6|c1<<4|c2<<2|c3``; 3 bits 8 codes in 3 bytes;
    4 bits ``c[2i]<<4 | c[2i+1]`` (the even code in the HIGH nibble, the
    reverse of the weights' half-block nibbles)."""
    c = np.asarray(codes).astype(np.int64)
    n = c.shape[0]
    if nbits == 2:
        g = c.reshape(n, -1, 4)
        out = (g[..., 0] << 6) | (g[..., 1] << 4) | (g[..., 2] << 2) | g[..., 3]
    elif nbits == 3:
        g = c.reshape(n, -1, 8)
        b0 = (g[..., 0] << 5) | (g[..., 1] << 2) | (g[..., 2] >> 1)
        b1 = ((g[..., 2] & 1) << 7) | (g[..., 3] << 4) | (g[..., 4] << 1) | (g[..., 5] >> 2)
        b2 = ((g[..., 5] & 3) << 6) | (g[..., 6] << 3) | g[..., 7]
        out = np.stack([b0, b1, b2], axis=-1).reshape(n, -1)
    elif nbits == 4:
        out = (c[:, 0::2] << 4) | c[:, 1::2]
    else:
        raise ValueError(f"nbits must be 2, 3 or 4, got {nbits}")
    return (out & 0xFF).astype(np.uint8)


def kv_unpack(packed: np.ndarray, nbits: int, d: int) -> np.ndarray:
    """BitPacker.unpack (kv_cache/cache.py:130-165) -> int64 codes [N, d]."""
    p = np.asarray(packed).astype(np.int64)
    n = p.shape[0]
    if nbits == 2:
        out = np.stack([(p >> 6) & 3, (p >> 4) & 3, (p >> 2) & 3, p & 3], axis=-1)
    elif nbits == 3:
        g = p.reshape(n, -1, 3)
        b0, b1, b2 = g[..., 0], g[..., 1], g[..., 2]
        out = np.stack([(b0 >> 5) & 7, (b0 >> 2) & 7, ((b0 & 3) << 1) | ((b1 >> 7) & 1),
                        (b1 >> 4) & 7, (b1 >> 1) & 7, ((b1 & 1) << 2) | ((b2 >> 6) & 3),
                        (b2 >> 3) & 7, b2 & 7], axis=-1)
    elif nbits == 4:
        out = np.stack([(p >> 4) & 0xF, p & 0xF], axis=-1)
    else:
        raise ValueError(f"nbits must be 2, 3 or 4, got {nbits}")
    return out.reshape(n, d)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even (torch's cast)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = (u & 0x7F800000) == 0x7F800000
    rounded = np.where(nan & ((u & 0x7FFFFF) != 0), (u >> 16) | 0x40, rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def kv_rotate(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Per-vector norm (clamped at 1e-10) and ``(x / norm) @ H * sqrt(D)``
    in float32 (kv_cache/cache.py:216-219)."""
    flat = np.asarray(x, dtype=np.float32)
    d = flat.shape[1]
    nrm = np.maximum(np.sqrt((flat * flat).sum(axis=1, dtype=np.float32)), np.float32(1e-10))
    rot = ((flat / nrm[:, None]) @ hadamard(d)) * np.float32(math.sqrt(d))
    return nrm.astype(np.float32), rot.astype(np.float32)


def kv_quantize(x: np.ndarray, nbits: int) -> Tuple[np.ndarray, np.ndarray]:
    """PolarKVQuantizer.quantize (kv_cache/cache.py:201-233) on x [N, D]:
    codes = first-index argmin |rot - ct|, BitPacker-packed; norms as bf16
    bit patterns. Returns (packed uint8, norms uint16)."""
    nrm, rot = kv_rotate(x)
    ct = kv_centroids(nbits)
    codes = np.abs(rot[:, :, None] - ct[None, None, :]).argmin(axis=-1)
    return kv_pack(codes, nbits), f32_to_bf16_bits(nrm)


def kv_dequantize(packed: np.ndarray, norms_bf16: np.ndarray, nbits: int, d: int) -> np.ndarray:
    """PolarKVQuantizer.dequantize (kv_cache/cache.py:235-256):
    ``((ct[codes] / sqrt(D)) @ H) * norm`` in float32, cast to bf16.
    Returns bf16 bit patterns [N, d]."""
    codes = kv_unpack(packed, nbits, d)
    vals = kv_centroids(nbits)[codes] / np.float32(math.sqrt(d))
    out = (vals.astype(np.float32) @ hadamard(d)) * bf16_bits_to_f32(norms_bf16)[:, None]
    return f32_to_bf16_bits(out)


# ---------------------------------------------------------------------------
# Seeded synthetic inputs shared by tests, smoke and the CPU baseline
# ---------------------------------------------------------------------------


def seeded_normal(shape, std: float, seed: int, dtype=np.float16) -> np.ndarray:
    """N(0, std) with numpy's PCG64 generator, cast to ``dtype``."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(dtype)
