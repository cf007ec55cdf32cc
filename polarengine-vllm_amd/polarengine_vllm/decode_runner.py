"""Minimal decoder-only model runner for batched decode on one GPU, built on
the plugin's own classes.

vLLM is not installed in this image, so this module plays the part of its
model runner for the end-to-end decode measurement the reference quotes in
tokens/s (README.md:17-27, "PolarEngine v4 (Triton)": 34.2 tok/s on a 9B
model). Every linear of every layer is a ``PolarQuantLinearMethod`` layer in
vLLM's merged form (one qkv_proj, one gate_up_proj), called through
``apply`` exactly as vLLM's ``LinearBase.forward`` calls a quantization
method. Around them, in torch: token embedding, RMSNorm, rotary embedding, a
static bf16 KV cache, grouped-query attention over it, SiLU(gate) * up, a
bf16 residual stream, and a bf16 lm_head (vLLM keeps embeddings and lm_head
unquantized unless a checkpoint quantizes them). There is no scheduler,
sampler beyond argmax, paged cache or tokenizer.

One decode step (``DecodeRunner.step``) takes the batch's current tokens and
position (device tensors, so the step can be captured in a HIP graph and
replayed) and returns the logits; ``greedy_tokens_per_s`` replays it with
the argmax fed back.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

from polarengine_vllm.linear_method import PolarQuantLinearMethod


@dataclass
class DecoderConfig:
    hidden: int = 4096
    layers: int = 36
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 12288
    vocab: int = 151936
    rope_theta: float = 1.0e6
    rms_eps: float = 1e-6
    # bits per linear: the mixed assignment of one C4 decoder layer
    bits: Dict[str, int] = field(default_factory=lambda: {
        "qkv_proj": 5, "o_proj": 6, "gate_up_proj": 3, "down_proj": 4})


def qwen3_8b_shapes() -> DecoderConfig:
    """The layer shapes of Qwen3-8B (36 layers, hidden 4096, 32 query / 8 KV
    heads of 128, intermediate 12288, vocabulary 151936, RoPE theta 1e6)."""
    return DecoderConfig()


class QuantLinear(torch.nn.Module):
    """One quantized linear: the buffers create_weights registers, filled
    with codes and norms, then process_weights_after_loading's runtime
    layout; forward is PolarQuantLinearMethod.apply."""

    def __init__(self, in_f: int, out_sizes: List[int], bits: int, dev: torch.device,
                 gen: torch.Generator, codes: Optional[torch.Tensor] = None,
                 norms: Optional[torch.Tensor] = None) -> None:
        super().__init__()
        self.method = PolarQuantLinearMethod(128, bits)
        out_f = sum(out_sizes)
        self.method.create_weights(self, in_f, out_sizes, in_f, out_f, torch.bfloat16)
        self.to(dev)
        if codes is None:  # random codes and norms of a unit-variance weight
            codes = torch.randint(0, 1 << bits, self.codes.shape, generator=gen, device=dev,
                                  dtype=torch.int32).to(torch.int8)
            norms = (torch.rand(self.norms.shape, generator=gen, device=dev) * 0.4 + 0.9) \
                * math.sqrt(128.0 / in_f)
        self.codes.copy_(codes)
        self.norms.copy_(norms.to(torch.float16))
        self.method.process_weights_after_loading(self)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.method.apply(self, x)


def _rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """bf16 in and out (fp32 statistics inside the fused kernel)."""
    return torch.nn.functional.rms_norm(x, (x.shape[-1],), w.to(x.dtype), eps)


class DecodeRunner:
    """Random-weight decoder of ``cfg``'s shapes for a fixed batch and
    maximum length; the KV cache holds keys as [layer, batch, kv_head, dim,
    position] and values as [layer, batch, kv_head, position, dim], so both
    attention products take contiguous operands."""

    def __init__(self, cfg: DecoderConfig, batch: int, max_len: int, dev, seed: int = 0,
                 weights: Optional[dict] = None) -> None:
        self.cfg, self.batch, self.max_len = cfg, batch, max_len
        self.dev = torch.device(dev)
        g = torch.Generator(device=self.dev).manual_seed(seed)
        c, bf = cfg, torch.bfloat16
        q_sz, kv_sz = c.heads * c.head_dim, c.kv_heads * c.head_dim
        w = weights or {}
        self.embed = w.get("embed", torch.randn(c.vocab, c.hidden, generator=g, device=self.dev) * 0.02).to(bf)
        self.lm_head = w.get("lm_head", torch.randn(c.vocab, c.hidden, generator=g, device=self.dev)
                             / math.sqrt(c.hidden)).to(bf).contiguous()
        self.final_norm = torch.ones(c.hidden, device=self.dev, dtype=bf)
        self.layers = []
        for i in range(c.layers):
            lw = w.get("layers", [{}] * c.layers)[i]
            mk = lambda name, in_f, outs: QuantLinear(
                in_f, outs, c.bits[name], self.dev, g,
                *((lw[name]["codes"], lw[name]["norms"]) if name in lw else (None, None)))
            self.layers.append({
                "in_norm": torch.ones(c.hidden, device=self.dev, dtype=bf),
                "post_norm": torch.ones(c.hidden, device=self.dev, dtype=bf),
                "qkv_proj": mk("qkv_proj", c.hidden, [q_sz, kv_sz, kv_sz]),
                "o_proj": mk("o_proj", q_sz, [c.hidden]),
                "gate_up_proj": mk("gate_up_proj", c.hidden, [c.intermediate, c.intermediate]),
                "down_proj": mk("down_proj", c.intermediate, [c.hidden]),
            })
        self.k_cache = torch.zeros(c.layers, batch, c.kv_heads, c.head_dim, max_len, dtype=bf,
                                   device=self.dev)
        self.v_cache = torch.zeros(c.layers, batch, c.kv_heads, max_len, c.head_dim, dtype=bf,
                                   device=self.dev)
        inv = 1.0 / (c.rope_theta ** (torch.arange(0, c.head_dim, 2, device=self.dev).float()
                                      / c.head_dim))
        ang = torch.arange(max_len, device=self.dev).float()[:, None] * inv[None, :]
        self.cos, self.sin = ang.cos(), ang.sin()  # [max_len, head_dim / 2]
        self.positions = torch.arange(max_len, device=self.dev)

    def step(self, tokens: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """One decode step for the batch: tokens [B] int64, pos [1] int64 (the
        position every sequence of the batch writes); returns fp32 logits
        [B, vocab]."""
        c, B = self.cfg, self.batch
        H, KVH, D = c.heads, c.kv_heads, c.head_dim
        grp, hd = H // KVH, D // 2
        x = self.embed.index_select(0, tokens)  # residual stream, bf16
        # per step: the position's rotary factors and the attention mask
        cos = self.cos.index_select(0, pos)  # [1, D/2]
        sin = self.sin.index_select(0, pos)
        mask = torch.where(self.positions <= pos, 0.0, float("-inf")).to(torch.bfloat16)
        scale = 1.0 / math.sqrt(D)
        for i, ly in enumerate(self.layers):
            h = _rms_norm(x, ly["in_norm"], c.rms_eps)
            qkv = ly["qkv_proj"](h)
            # rotate-half RoPE on the q and k heads together
            qk = qkv[:, :(H + KVH) * D].reshape(B, H + KVH, D).float()
            x1, x2 = qk[..., :hd], qk[..., hd:]
            qk = torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1)
            q = (qk[:, :H] * scale).to(torch.bfloat16).reshape(B, KVH, grp, D)
            k = qk[:, H:].to(torch.bfloat16)
            v = qkv[:, (H + KVH) * D:].reshape(B, KVH, D)
            self.k_cache[i].index_copy_(3, pos, k.unsqueeze(-1))
            self.v_cache[i].index_copy_(2, pos, v.unsqueeze(2))
            # scores [B, KVH, grp, max_len] = q . K^T, positions past pos masked
            s = torch.matmul(q, self.k_cache[i]) + mask
            p = torch.softmax(s, -1, dtype=torch.float32).to(torch.bfloat16)
            o = torch.matmul(p, self.v_cache[i]).reshape(B, H * D)  # [B, H*D]
            x = x + ly["o_proj"](o)
            h = _rms_norm(x, ly["post_norm"], c.rms_eps)
            gu = ly["gate_up_proj"](h)
            a = torch.nn.functional.silu(gu[:, :c.intermediate]) * gu[:, c.intermediate:]
            x = x + ly["down_proj"](a)
        x = _rms_norm(x, self.final_norm, c.rms_eps)
        return torch.nn.functional.linear(x, self.lm_head).float()  # [B, vocab]

    def greedy_tokens_per_s(self, start_pos: int, steps: int, warmup: int = 2) -> dict:
        """Greedy decode from ``start_pos``: the step is captured in a HIP graph
        that also writes the argmax back as the next tokens and advances the
        position, then replayed ``steps`` times between two synchronizes
        (HIP events on the replay stream). Returns tokens/s for the batch."""
        dev = self.dev
        tokens = torch.zeros(self.batch, dtype=torch.long, device=dev)
        pos = torch.tensor([start_pos], dtype=torch.long, device=dev)
        if start_pos + warmup + 1 + steps > self.max_len:
            raise ValueError("max_len too small for the requested steps")

        def advance():
            logits = self.step(tokens, pos)
            tokens.copy_(logits.argmax(-1))
            pos.add_(1)

        s = torch.cuda.Stream(device=dev)
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            for _ in range(warmup):  # eager: workspaces and caches at full size
                advance()
            torch.cuda.synchronize(dev)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=s):
                advance()
            graph.replay()  # one untimed replay
            torch.cuda.synchronize(dev)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(s)
            for _ in range(steps):
                graph.replay()
            e1.record(s)
        torch.cuda.synchronize(dev)
        sec = e0.elapsed_time(e1) / 1e3
        return {"tok_per_s": self.batch * steps / sec, "ms_per_step": sec / steps * 1e3,
                "batch": self.batch, "steps": steps, "context_start": start_pos}
