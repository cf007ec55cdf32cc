"""MoE methods (reference: polarengine_vllm/moe_method.py).

* ``PolarQuantMoEMethod`` -- PolarQuant-quantized experts, all resident on
  the GPU, run by the grouped-expert HIP path (``pe_moe_forward_routed``:
  routing and experts in one call; ``pe_moe_forward`` when a custom routing
  function supplies the ids). The reference has no quantized expert compute (its
  experts stay bf16 in vLLM's fused MoE); the math follows its in-repo MoE
  forward (nemotron_offload.py:172-226): scores -> top-k -> renormalise ->
  SwiGLU(w13 = [gate; up]) -> w2 -> weighted sum.
* ``PolarPassthroughMoEMethod`` -- the reference's pass-through to vLLM's
  unquantized fused MoE, for checkpoints whose experts are not quantized
  (requires vLLM).

Expert weight layout follows the reference's fallback layout
(moe_method.py:56-72): w13 [E, 2I, H] (rows [0, I) gate, [I, 2I) up) and
w2 [E, H, I], here as PolarQuant codes / fp16 norms / ct_scaled per matrix.
After loading, codes with bits <= 4 are nibble-packed and, when each expert's
row count is a multiple of 16, both matrices are rearranged into the tiled-16
runtime layout (one 16-row x 128-block tile of codes is one contiguous read).
"""

from __future__ import annotations

import math
from typing import List, Optional

import torch

from polarengine_vllm import _lib
from polarengine_vllm.utils import get_centroids


def _layout(packed: bool, tiled: bool) -> int:
    """The packed argument of pe_moe_forward: 1 = nibbles, | 2 = tiled-16."""
    return int(bool(packed)) | (_lib.PE_LAYOUT_TILE16 if tiled else 0)


class PolarQuantMoEMethod:
    """Quantized fused-MoE method (vLLM FusedMoEMethodBase interface)."""

    def __init__(self, block_size: int = 128, bits13: int = 3, bits2: int = 4,
                 tile: bool = True) -> None:
        if block_size != 128:
            raise ValueError("the gfx950 kernels implement block_size 128")
        self.block_size = block_size
        self.bits13 = bits13
        self.bits2 = bits2
        self.tile = tile  # tiled-16 expert layout after loading (else row-major)

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype,
                       **kwargs) -> None:
        bs = self.block_size
        e, h, i = num_experts, hidden_size, intermediate_size_per_partition
        hp = (h + bs - 1) // bs * bs
        ip = (i + bs - 1) // bs * bs
        if hp != h:
            raise ValueError("hidden_size must be a multiple of 128")
        layer.register_buffer("w13_codes", torch.zeros(e, 2 * i, hp, dtype=torch.int8))
        layer.register_buffer("w13_norms", torch.zeros(e, 2 * i, hp // bs, dtype=torch.float16))
        layer.register_buffer("w13_ct_scaled", (get_centroids(self.bits13) / math.sqrt(bs)).clone())
        layer.register_buffer("w2_codes", torch.zeros(e, h, ip, dtype=torch.int8))
        layer.register_buffer("w2_norms", torch.zeros(e, h, ip // bs, dtype=torch.float16))
        layer.register_buffer("w2_ct_scaled", (get_centroids(self.bits2) / math.sqrt(bs)).clone())
        layer.num_experts = e
        layer.hidden_size = h
        layer.intermediate_size = i
        layer.w13_packed = False
        layer.w2_packed = False
        layer.w13_tiled = False
        layer.w2_tiled = False

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """ct to the codes' device; nibble-pack matrices with bits <= 4; then
        the tiled-16 layout per expert (``pe_tile_weights`` over the
        [E * rows, row_bytes] matrix: with rows a multiple of 16 no tile spans
        two experts)."""
        from polarengine_vllm.packing import pack_codes_half_block, tile_weights_16
        dev = layer.w13_codes.device
        layer.w13_ct_scaled = layer.w13_ct_scaled.to(dev, torch.float32).contiguous()
        layer.w2_ct_scaled = layer.w2_ct_scaled.to(dev, torch.float32).contiguous()
        if self.bits13 <= 4 and not layer.w13_packed:
            layer.w13_codes = pack_codes_half_block(layer.w13_codes.contiguous(), self.block_size)
            layer.w13_packed = True
        if self.bits2 <= 4 and not layer.w2_packed:
            layer.w2_codes = pack_codes_half_block(layer.w2_codes.contiguous(), self.block_size)
            layer.w2_packed = True
        if self.tile and dev.type == "cuda":
            for name in ("w13", "w2"):
                codes, norms = getattr(layer, f"{name}_codes"), getattr(layer, f"{name}_norms")
                e, rows, row_bytes = codes.shape
                if getattr(layer, f"{name}_tiled") or rows % 16:
                    continue
                ct, nt = tile_weights_16(codes.reshape(e * rows, row_bytes),
                                         norms.reshape(e * rows, norms.shape[2]))
                setattr(layer, f"{name}_codes", ct.view(e, rows, row_bytes))
                setattr(layer, f"{name}_norms", nt.view(e, rows, norms.shape[2]))
                setattr(layer, f"{name}_tiled", True)

    @staticmethod
    def _routing_args(router_logits: torch.Tensor, num_experts: int, scoring_func: str,
                      e_score_correction_bias: Optional[torch.Tensor], use_grouped_topk: bool,
                      num_expert_group: Optional[int], topk_group: Optional[int]):
        """fp32 logits, fp32 bias (or None), scoring code, and the group
        arguments of the C ABI (0, 0 for plain top-k)."""
        dev = _lib.require_device(router_logits)
        lg = router_logits.to(torch.float32).contiguous()
        if lg.dim() != 2 or lg.shape[1] != num_experts:
            raise ValueError(f"router logits of shape {tuple(lg.shape)} for {num_experts} experts")
        bias = None
        if e_score_correction_bias is not None:
            bias = e_score_correction_bias.to(device=dev, dtype=torch.float32).contiguous()
        scoring = {"softmax": 0, "sigmoid": 1}.get(scoring_func)
        if scoring is None:
            raise ValueError(f"unsupported scoring_func {scoring_func}")
        if not use_grouped_topk:
            return lg, bias, scoring, 0, 0
        if num_expert_group is None or topk_group is None:
            raise ValueError("grouped top-k needs num_expert_group and topk_group")
        return lg, bias, scoring, int(num_expert_group), int(topk_group)

    def select_experts(self, router_logits: torch.Tensor, top_k: int, renormalize: bool,
                       scoring_func: str = "softmax",
                       e_score_correction_bias: Optional[torch.Tensor] = None,
                       use_grouped_topk: bool = False, num_expert_group: Optional[int] = None,
                       topk_group: Optional[int] = None):
        """(topk_weights float32 [T, k], topk_ids int32 [T, k]) via pe_moe_route,
        or pe_moe_route_grouped for grouped top-k (vLLM's grouped_topk, the
        routing the reference's apply hands to vLLM with use_grouped_topk,
        moe_method.py:74-89). apply() routes inside pe_moe_forward_routed
        instead; this is the routing alone, for callers that want the ids."""
        lg, bias, scoring, n_group, t_group = self._routing_args(
            router_logits, router_logits.shape[-1], scoring_func, e_score_correction_bias,
            use_grouped_topk, num_expert_group, topk_group)
        dev = lg.device
        t = lg.shape[0]
        w = torch.empty(t, top_k, dtype=torch.float32, device=dev)
        ids = torch.empty(t, top_k, dtype=torch.int32, device=dev)
        if n_group:
            _lib.check(_lib.lib().pe_moe_route_grouped(
                lg.data_ptr(), t, lg.shape[1], top_k, int(bool(renormalize)), scoring,
                _lib.ptr(bias), n_group, t_group, w.data_ptr(), ids.data_ptr(),
                _lib.stream_ptr(dev)), "pe_moe_route_grouped")
            return w, ids
        _lib.check(_lib.lib().pe_moe_route(lg.data_ptr(), t, lg.shape[1], top_k,
                                           int(bool(renormalize)), scoring, _lib.ptr(bias),
                                           w.data_ptr(), ids.data_ptr(), _lib.stream_ptr(dev)),
                   "pe_moe_route")
        return w, ids

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, router_logits: torch.Tensor,
              top_k: int, renormalize: bool, use_grouped_topk: bool = False,
              topk_group: Optional[int] = None, num_expert_group: Optional[int] = None,
              custom_routing_function=None, scoring_func: str = "softmax",
              e_score_correction_bias: Optional[torch.Tensor] = None, **kwargs) -> torch.Tensor:
        """Routed quantized SwiGLU experts: [T, H] fp16 or bf16 -> [T, H] of the
        same dtype. Under torch.compile the call is the custom op
        ``polarengine::moe_routed`` (or ``polarengine::moe_given`` after a
        custom routing function), so a compiled model forward traces through it."""
        _lib.require_device(x, layer.w13_codes)
        _lib.act_dtype(x)
        e = layer.num_experts
        wts = (layer.w13_codes, layer.w13_norms, layer.w13_ct_scaled, layer.w2_codes,
               layer.w2_norms, layer.w2_ct_scaled)
        meta = [self.bits13, _layout(layer.w13_packed, layer.w13_tiled), self.bits2,
                _layout(layer.w2_packed, layer.w2_tiled), e, layer.hidden_size,
                layer.intermediate_size]
        compiling = torch.compiler.is_compiling()
        if custom_routing_function is None:
            # routing and experts in one call (the routing shares the first launch)
            t = x.numel() // layer.hidden_size
            # (the logits' own width, not -1: with zero tokens -1 is ambiguous)
            lg, bias, scoring, n_group, t_group = self._routing_args(
                router_logits.reshape(t, router_logits.shape[-1]), e, scoring_func,
                e_score_correction_bias, use_grouped_topk, num_expert_group, topk_group)
            route = [top_k, int(bool(renormalize)), scoring, n_group, t_group]
            if compiling:
                return torch.ops.polarengine.moe_routed(x, lg, bias, *wts, route, meta)
            return _moe_routed(x, lg, bias, *wts, route, meta)
        xs = x.reshape(-1, layer.hidden_size)
        w, ids = custom_routing_function(hidden_states=xs, gating_output=router_logits,
                                         topk=top_k, renormalize=renormalize)
        w = w.to(torch.float32).contiguous()
        ids = ids.to(torch.int32).contiguous()
        if compiling:
            return torch.ops.polarengine.moe_given(x, w, ids, *wts, meta)
        return _moe_given(x, w, ids, *wts, meta)

    def get_fused_moe_quant_config(self):
        return None


def _moe_weights(w13c, w13n, w13ct, w2c, w2n, w2ct, meta):
    b13, lay13, b2, lay2 = meta[:4]
    return (w13c.data_ptr(), b13, lay13, w13n.data_ptr(), w13ct.data_ptr(), 1 << b13,
            w2c.data_ptr(), b2, lay2, w2n.data_ptr(), w2ct.data_ptr(), 1 << b2)


def _moe_routed(x: torch.Tensor, lg: torch.Tensor, bias: Optional[torch.Tensor],
                w13c: torch.Tensor, w13n: torch.Tensor, w13ct: torch.Tensor, w2c: torch.Tensor,
                w2n: torch.Tensor, w2ct: torch.Tensor, route: List[int],
                meta: List[int]) -> torch.Tensor:
    """pe_moe_forward_routed: routing (route = top_k, renormalize, scoring,
    n_group, topk_group) and the experts (meta = bits13, layout13, bits2,
    layout2, E, H, I) in one call."""
    dev = x.device
    e, h, i = meta[4:]
    top_k, renorm, scoring, n_group, t_group = route
    xs = x.reshape(-1, h).contiguous()
    t = xs.shape[0]
    out = torch.empty_like(xs)
    if t == 0:
        return out.view(x.shape)
    L = _lib.lib()
    wsb = L.pe_moe_workspace_size(t, top_k, e, h, i)
    ws = _lib.workspace(dev, wsb)
    rc = L.pe_moe_forward_routed(
        xs.data_ptr(), _lib.act_dtype(xs), t, h, i, e, top_k, lg.data_ptr(), renorm, scoring,
        _lib.ptr(bias), n_group, t_group, *_moe_weights(w13c, w13n, w13ct, w2c, w2n, w2ct, meta),
        out.data_ptr(), _lib.ptr(ws), wsb, _lib.stream_ptr(dev))
    _lib.check(rc, "pe_moe_forward_routed")
    return out.view(x.shape)


def _moe_given(x: torch.Tensor, w: torch.Tensor, ids: torch.Tensor, w13c: torch.Tensor,
               w13n: torch.Tensor, w13ct: torch.Tensor, w2c: torch.Tensor, w2n: torch.Tensor,
               w2ct: torch.Tensor, meta: List[int]) -> torch.Tensor:
    """pe_moe_forward: the experts on given routing (fp32 weights, int32 ids [T, k])."""
    dev = x.device
    e, h, i = meta[4:]
    xs = x.reshape(-1, h).contiguous()
    t = xs.shape[0]
    out = torch.empty_like(xs)
    if t == 0:
        return out.view(x.shape)
    top_k = ids.shape[-1]
    L = _lib.lib()
    wsb = L.pe_moe_workspace_size(t, top_k, e, h, i)
    ws = _lib.workspace(dev, wsb)
    rc = L.pe_moe_forward(xs.data_ptr(), _lib.act_dtype(xs), t, h, i, e, top_k, w.data_ptr(),
                          ids.data_ptr(), *_moe_weights(w13c, w13n, w13ct, w2c, w2n, w2ct, meta),
                          out.data_ptr(), _lib.ptr(ws), wsb, _lib.stream_ptr(dev))
    _lib.check(rc, "pe_moe_forward")
    return out.view(x.shape)


# The two MoE calls as torch custom ops, for traced / compiled models; the
# fake implementations give the output's shape and dtype (x's).
torch.library.custom_op("polarengine::moe_routed", _moe_routed, mutates_args=())
torch.library.custom_op("polarengine::moe_given", _moe_given, mutates_args=())


@torch.library.register_fake("polarengine::moe_routed")
def _moe_routed_fake(x, lg, bias, w13c, w13n, w13ct, w2c, w2n, w2ct, route, meta):
    return torch.empty_like(x)


@torch.library.register_fake("polarengine::moe_given")
def _moe_given_fake(x, w, ids, w13c, w13n, w13ct, w2c, w2n, w2ct, meta):
    return torch.empty_like(x)


class PolarPassthroughMoEMethod:
    """Unquantized experts through vLLM's fused MoE (reference moe_method.py:18-98)."""

    def __init__(self):
        self._initialized = False
        self._inner = None

    def _lazy_init(self, layer):
        if self._initialized:
            return
        try:
            from vllm.model_executor.layers.fused_moe.unquantized_fused_moe_method import (  # type: ignore
                UnquantizedFusedMoEMethod)
            self._inner = UnquantizedFusedMoEMethod(moe=layer)
            self._initialized = True
        except (ImportError, AttributeError, TypeError):
            pass

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition,
                       params_dtype, **kwargs):
        self._lazy_init(layer)
        if not self._initialized:
            raise RuntimeError("PolarPassthroughMoEMethod needs vLLM's unquantized fused MoE")
        return self._inner.create_weights(
            layer, num_experts=num_experts, hidden_size=hidden_size,
            intermediate_size_per_partition=intermediate_size_per_partition,
            params_dtype=params_dtype, **kwargs)

    def apply(self, layer, x, router_logits, top_k, renormalize, **kwargs):
        self._lazy_init(layer)
        if not self._initialized:
            raise RuntimeError("PolarPassthroughMoEMethod: vLLM fused MoE not available")
        return self._inner.apply(layer, x, router_logits, top_k, renormalize, **kwargs)

    def get_fused_moe_quant_config(self):
        if self._initialized and hasattr(self._inner, "get_fused_moe_quant_config"):
            return self._inner.get_fused_moe_quant_config()
        return None


try:  # virtual subclass for vLLM's isinstance checks (reference moe_method.py:103-107)
    from vllm.model_executor.layers.fused_moe.layer import FusedMoEMethodBase  # type: ignore
    FusedMoEMethodBase.register(PolarQuantMoEMethod)
    FusedMoEMethodBase.register(PolarPassthroughMoEMethod)
except Exception:
    pass
