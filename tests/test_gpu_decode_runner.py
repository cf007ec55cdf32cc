"""GPU test of the end-to-end decode runner (polarengine_vllm.decode_runner):
a two-layer model with explicit codes, teacher-forced over four positions,
against an fp32 statement of the same model in numpy whose quantized
linears are the oracle's linear_apply (the reference's linear forward,
linear_method.py:184-221) and whose attention keeps the whole history.

The runner's residual stream, attention products and linear outputs are
bf16 (as vLLM runs a bf16 model), so the logits are compared at a
bf16-pipeline tolerance: normwise
||d||_inf / ||ref||_inf <= 3e-2 and cosine >= 0.999 per step."""

import math

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import DEV, say

pytestmark = pytest.mark.gpu


def _bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def _rms(x, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)


def _rope(x, pos, theta, d):
    inv = 1.0 / (theta ** (np.arange(0, d, 2, dtype=np.float32) / d))
    ang = pos * inv
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def test_decode_runner_matches_fp32_statement():
    from polarengine_vllm.decode_runner import DecodeRunner, DecoderConfig
    say("decode runner: 2 layers, hidden 256, batch 2, 4 steps")
    cfg = DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, intermediate=384,
                        vocab=300)
    B, steps = 2, 4
    rng = np.random.default_rng(31)
    q_sz, kv_sz = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    shapes = {"qkv_proj": (q_sz + 2 * kv_sz, cfg.hidden), "o_proj": (cfg.hidden, q_sz),
              "gate_up_proj": (2 * cfg.intermediate, cfg.hidden),
              "down_proj": (cfg.hidden, cfg.intermediate)}
    layers = []
    for _ in range(cfg.layers):
        lw = {}
        for name, (n, k) in shapes.items():
            b = cfg.bits[name]
            codes = rng.integers(0, 1 << b, (n, k)).astype(np.int8)
            norms = ((rng.random((n, k // 128)) * 0.4 + 0.9) * math.sqrt(128 / k)).astype(np.float16)
            lw[name] = {"codes": codes, "norms": norms}
        layers.append(lw)
    embed = (rng.standard_normal((cfg.vocab, cfg.hidden)) * 0.5).astype(np.float32)
    lm_head = (rng.standard_normal((cfg.vocab, cfg.hidden)) / math.sqrt(cfg.hidden)).astype(np.float32)
    weights = {"embed": torch.from_numpy(embed).to(DEV),
               "lm_head": torch.from_numpy(lm_head).to(DEV),
               "layers": [{nm: {"codes": torch.from_numpy(w["codes"]).to(DEV),
                                "norms": torch.from_numpy(w["norms"]).to(DEV)}
                           for nm, w in lw.items()} for lw in layers]}
    run = DecodeRunner(cfg, B, 16, DEV, weights=weights)
    tokens = rng.integers(0, cfg.vocab, (steps, B))

    # fp32 statement; embeddings / lm_head as the runner holds them (bf16)
    emb, head = _bf16(embed), _bf16(lm_head)
    H, KVH, D, G = cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.heads // cfg.kv_heads
    kc = [np.zeros((B, KVH, 0, D), np.float32) for _ in range(cfg.layers)]
    vc = [np.zeros((B, KVH, 0, D), np.float32) for _ in range(cfg.layers)]

    def lin(x, name, lw):
        b = cfg.bits[name]
        return O.linear_apply(x, lw[name]["codes"], lw[name]["norms"].astype(np.float32),
                              O.ct_scaled(b), x.shape[-1]).astype(np.float32)

    for t in range(steps):
        got = run.step(torch.from_numpy(tokens[t]).to(DEV),
                       torch.tensor([t], dtype=torch.long, device=DEV)).cpu().numpy()
        x = emb[tokens[t]]
        for i, lw in enumerate(layers):
            qkv = lin(_rms(x, cfg.rms_eps), "qkv_proj", lw)
            q = _rope(qkv[:, :H * D].reshape(B, H, D), t, cfg.rope_theta, D)
            k = _rope(qkv[:, H * D:(H + KVH) * D].reshape(B, KVH, D), t, cfg.rope_theta, D)
            v = qkv[:, (H + KVH) * D:].reshape(B, KVH, D)
            kc[i] = np.concatenate([kc[i], k[:, :, None]], 2)
            vc[i] = np.concatenate([vc[i], v[:, :, None]], 2)
            qg = q.reshape(B, KVH, G, D)
            s = np.einsum("bkgd,bkld->bkgl", qg, kc[i]) / math.sqrt(D)
            p = np.exp(s - s.max(-1, keepdims=True))
            p /= p.sum(-1, keepdims=True)
            o = np.einsum("bkgl,bkld->bkgd", p, vc[i]).reshape(B, H * D)
            x = x + lin(o, "o_proj", lw)
            gu = lin(_rms(x, cfg.rms_eps), "gate_up_proj", lw)
            g, u = gu[:, :cfg.intermediate], gu[:, cfg.intermediate:]
            x = x + lin(g / (1 + np.exp(-g)) * u, "down_proj", lw)
        want = _rms(x, cfg.rms_eps) @ head.T
        err = np.abs(got - want).max() / np.abs(want).max()
        cos = (got * want).sum() / (np.linalg.norm(got) * np.linalg.norm(want))
        assert err <= 3e-2 and cos >= 0.999, f"step {t}: normwise {err:.3e}, cosine {cos:.6f}"


def test_decode_runner_graph_replay_advances():
    """The captured greedy step replays: positions advance and the measured
    rate is reported for the batch."""
    from polarengine_vllm.decode_runner import DecodeRunner, DecoderConfig
    say("decode runner graph replay")
    cfg = DecoderConfig(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, intermediate=384,
                        vocab=300)
    run = DecodeRunner(cfg, 4, 64, DEV, seed=5)
    r = run.greedy_tokens_per_s(start_pos=8, steps=16, warmup=2)
    assert r["tok_per_s"] > 0 and r["batch"] == 4 and r["steps"] == 16
    # the K cache holds the written positions (8 .. 8 + 2 + 1 + 16) and zeros past them
    kc = run.k_cache[0].float()
    assert kc[..., 8:27].abs().sum() > 0
    assert kc[..., 27:].abs().sum() == 0
