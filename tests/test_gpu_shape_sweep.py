"""Seeded random shapes through pe_linear_forward, against the oracle.

The fixed-shape tests pin each kernel at the configs and at chosen edges;
this sweep draws 48 shapes from one seed so that the dispatch (decode with
and without the K split over workgroups, one or two m-tiles, the small-M
matmul, the prefill GEMM with and without its K split, the four-wave kernel)
meets ragged sizes it was not tuned on: N not a multiple of 16, K from one
128-block to 64, M across every route boundary (1, 16/17, 32/33, 64/65, 256),
every bit width 2..8, row-major and tiled-16 weights, fp16 and bf16
activations, with and without bias. Oracle: linear_apply (reference
linear_method.py:184-221), north-star tolerance."""

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import (bf16_dev, check_close, dev_codes, dev_tiled, linear_call, rand_layer, say,
                         to_dev)

pytestmark = pytest.mark.gpu

_M_CHOICES = [1, 1, 2, 3, 5, 8, 15, 16, 17, 24, 31, 32, 33, 40, 63, 64, 65, 96, 128, 200, 256, 300]


def _draw(n_cases=48, seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n_cases:
        m = int(rng.choice(_M_CHOICES))
        n = int(rng.integers(1, 48)) * 16 + int(rng.choice([0, 0, 0, 1, 7, 9]))
        if rng.random() < 0.25:
            n = int(rng.choice([4096, 3072, 1536]))
        k = 128 * int(rng.choice([1, 2, 3, 5, 8, 11, 16, 24, 32, 48, 64]))
        bits = int(rng.integers(2, 9))
        if m * n * k > 6e8:  # keep the CPU oracle to about a second
            continue
        cases.append((m, n, k, bits, bool(rng.random() < 0.6), bool(rng.random() < 0.5),
                      bool(rng.random() < 0.5), len(cases)))
    return cases


def _draw_prefill(n_cases=24, seed=2025):
    """Larger prefill shapes, where the four-wave tile forms are chosen by how
    many tiles fill a round of CUs (128 x 128 / 256 / 384, 64 x 128 / 256 /
    384, the K split): M 96..1536, N up to 12288 and ragged, odd block counts
    included."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n_cases:
        m = int(rng.choice([96, 160, 192, 200, 320, 384, 448, 512, 640, 768, 1024, 1280, 1536]))
        n = int(rng.choice([2048, 3072, 4096, 6144, 8192, 12288])) - int(rng.choice([0, 0, 16, 40]))
        k = 128 * int(rng.choice([2, 3, 4, 8, 16, 32]))
        bits = int(rng.integers(2, 9))
        if m * n * k > 3e9:
            continue
        cases.append((m, n, k, bits, bool(rng.random() < 0.6), bool(rng.random() < 0.5),
                      bool(rng.random() < 0.5), 100 + len(cases)))
    return cases


@pytest.mark.parametrize("m,n,k,bits,tiled,bf16,with_bias,idx", _draw() + _draw_prefill())
def test_random_shape(m, n, k, bits, tiled, bf16, with_bias, idx):
    from polarengine_vllm import _lib
    say(f"sweep #{idx} m={m} n={n} k={k} q{bits} tiled={tiled} bf16={bf16} bias={with_bias}")
    rng = np.random.default_rng(5000 + idx)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    x32 = O.seeded_normal((m, k), 1.0, 5100 + idx, np.float32)
    b32 = O.seeded_normal((n,), 0.1, 5200 + idx, np.float32) if with_bias else None
    if bf16:
        xd, x32 = bf16_dev(x32)
        bd = None
        if with_bias:
            bd, b32 = bf16_dev(b32)
    else:
        x32 = x32.astype(np.float16).astype(np.float32)
        xd = to_dev(x32.astype(np.float16))
        bd = to_dev(b32.astype(np.float16)) if with_bias else None
    if tiled:
        dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
        fmt = (_lib.PE_PACK_NIBBLE if nib else 0) | _lib.PE_LAYOUT_TILE16
    else:
        dcodes, nib = dev_codes(codes, bits)
        dnorms = to_dev(norms)
        fmt = _lib.PE_PACK_NIBBLE if nib else 0
    y = linear_call(xd, dcodes, dnorms, ct, bits, fmt, n, bd)
    assert y.dtype == (torch.bfloat16 if bf16 else torch.float16) and y.shape == (m, n)
    if bf16:
        want = O.bf16_bits_to_f32(O.linear_apply(x32, codes, norms, ct, k, b32,
                                                 out_dtype="bfloat16"))
    else:
        want = O.linear_apply(x32, codes, norms, ct, k,
                              None if b32 is None else b32.astype(np.float16)).astype(np.float32)
    check_close(y.float().cpu().numpy(), want, f"sweep #{idx} m={m} {n}x{k} q{bits}")
