"""PolarQuant linear method for vLLM (reference: polarengine_vllm/linear_method.py).

Same buffers and interface as the reference (``create_weights``, ``apply``,
``process_weights_after_loading``), with the forward running on the gfx950
HIP library:

* M <= 32 (decode): one launch of ``pe_linear_forward`` -- the FWHT-128 of x
  is fused into the GEMV prologue;
* M > 32: ``pe_fwht128`` once into the pair-f16 layout (cached for Q/K/V and
  gate/up reading the same hidden state), then ``pe_linear_forward_xtf``
  (MFMA GEMM) per projection;
* bias and the fp16 output cast are fused into the kernel epilogue.

Differences from the reference, on purpose:
* the FWHT cache is process-wide (the reference's lives per method instance,
  linear_method.py:85, so separate q/k/v modules never shared it) and keyed
  safely (see kernels.fwht.FWHTCache);
* a bf16 activation gives a bf16 result (the reference casts every output to
  fp16, linear_method.py:219, which a bf16 model cannot add to its bf16
  residual stream without a promotion); fp16 stays fp16, and other float
  dtypes give fp16 as in the reference. The transformed activation enters the
  matrix cores as fp16 in every case.
"""

from __future__ import annotations

import logging
import math
from typing import Any, Dict, List, Optional

import numpy as np
import torch
import torch.nn.functional as F

from polarengine_vllm import _lib
from polarengine_vllm.kernels.fwht import GLOBAL_FWHT_CACHE, FWHTCache, fwht_pairs
from polarengine_vllm.utils import get_centroids

try:
    from vllm.model_executor.utils import set_weight_attrs  # type: ignore
except Exception:  # vLLM absent: plain attribute setter

    def set_weight_attrs(weight: torch.Tensor, attrs: Dict[str, Any]) -> None:
        for key, value in attrs.items():
            setattr(weight, key, value)

logger = logging.getLogger(__name__)

# M above which the transformed activation is materialised (one FWHT launch)
# and shared through the FWHT cache. Up to it the decode GEMV transforms the
# activations in its own prologue (on the matrix cores from M = 2), which
# costs less than the extra launch even when q/k/v are separate modules that
# each transform the same input; vLLM's merged qkv_proj / gate_up_proj have
# one consumer per input, so there is nothing to share.
_FUSED_FWHT_MAX_M = 32


class PolarQuantLinearMethod:
    """vLLM linear method for PolarQuant layers (codes + fp16 norms + ct_scaled)."""

    def __init__(self, block_size: int = 128, bits: int = 4,
                 layer_meta: Optional[Dict[str, Any]] = None) -> None:
        if block_size != 128:
            raise ValueError("the gfx950 kernels implement block_size 128")
        self.block_size = block_size
        self.bits = bits
        self.layer_meta = layer_meta or {}
        self._fwht_cache = GLOBAL_FWHT_CACHE

    # ------------------------------------------------------------------
    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: list, input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs: Any) -> None:
        """Register ``codes`` int8 [out_f, Kp], ``norms`` fp16 [out_f, nb] and
        ``ct_scaled`` fp32 [2**bits] (reference: linear_method.py:91-151)."""
        bs = self.block_size
        in_f = input_size
        out_f = sum(output_partition_sizes)
        kp = (in_f + bs - 1) // bs * bs
        nb = kp // bs
        layer.register_buffer("codes", torch.zeros(out_f, kp, dtype=torch.int8))
        layer.register_buffer("norms", torch.zeros(out_f, nb, dtype=torch.float16))
        layer.register_buffer("ct_scaled", (get_centroids(self.bits) / math.sqrt(bs)).clone())
        layer.in_f = in_f
        layer.out_f = out_f
        layer.in_f_padded = kp
        layer.n_blocks = nb
        layer.bits = self.bits
        layer.block_size = bs
        layer.packed = False
        layer.tiled = False
        set_weight_attrs(layer.codes, {"input_dim": 1, "output_dim": 0})
        set_weight_attrs(layer.norms, {"input_dim": 1, "output_dim": 0})

    # ------------------------------------------------------------------
    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """Move ct to the codes' device; nibble-pack bits <= 4 on the GPU
        (``pe_pack_nibble``) and free the int8 codes
        (reference: linear_method.py:228-258); then re-lay codes and norms out
        in the tiled-16 runtime layout (``pe_tile_weights``: one 16-row x
        block tile is one contiguous read for the decode and GEMM kernels)."""
        device = layer.codes.device if hasattr(layer, "codes") else layer.codes_packed.device
        layer.ct_scaled = layer.ct_scaled.to(device=device, dtype=torch.float32).contiguous()
        # host copy of the codebook: the decode kernel takes it by value
        layer.ct_host = np.ascontiguousarray(layer.ct_scaled.cpu().numpy(), dtype=np.float32)
        layer.ct_host_list = [float(v) for v in layer.ct_host]  # the same, for the custom op
        if layer.norms.dtype != torch.float16:
            layer.norms = layer.norms.to(torch.float16)
        layer.norms = layer.norms.contiguous()
        if layer.bits <= 4 and not getattr(layer, "packed", False):
            from polarengine_vllm.packing import pack_codes_half_block
            layer.codes_packed = pack_codes_half_block(layer.codes.contiguous(), layer.block_size)
            layer.in_f_half = layer.n_blocks * (layer.block_size // 2)
            layer.packed = True
            del layer.codes
            logger.debug("packed codes to nibbles: out_f=%d in_f_half=%d bits=%d",
                         layer.out_f, layer.in_f_half, layer.bits)
        if not getattr(layer, "tiled", False):
            from polarengine_vllm.packing import tile_weights_16
            name = "codes_packed" if layer.packed else "codes"
            codes_t, norms_t = tile_weights_16(getattr(layer, name), layer.norms)
            setattr(layer, name, codes_t)
            layer.norms = norms_t
            layer.tiled = True

    # ------------------------------------------------------------------
    def apply(self, layer: torch.nn.Module, x: torch.Tensor,
              bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Quantized forward: y = x . W^T (+ bias), [..., out_f].

        fp16 and bf16 activations give a result of the same dtype; any other
        float dtype is transformed from its own precision and gives fp16, the
        reference's output dtype (linear_method.py:184-221 casts x.float()
        and returns .half()). Under torch.compile the call is the custom op
        ``polarengine::linear_apply`` (same kernels, no FWHT cache), so a
        compiled model forward traces through it."""
        packed = bool(getattr(layer, "packed", False))
        codes = layer.codes_packed if packed else layer.codes
        fmt = (_lib.PE_PACK_NIBBLE if packed else 0) | (
            _lib.PE_LAYOUT_TILE16 if getattr(layer, "tiled", False) else 0)
        if torch.compiler.is_compiling():
            ct_list = getattr(layer, "ct_host_list", None) or []
            return torch.ops.polarengine.linear_apply(
                x, codes, layer.norms, layer.ct_scaled, bias, layer.bits, fmt, layer.in_f,
                layer.in_f_padded, layer.out_f, ct_list)
        ct_host = getattr(layer, "ct_host", None)
        return _linear_forward(x, codes, layer.norms, layer.ct_scaled, ct_host, bias, layer.bits,
                               fmt, layer.in_f, layer.in_f_padded, layer.out_f, self._fwht_cache)


def _linear_forward(x: torch.Tensor, codes: torch.Tensor, norms: torch.Tensor,
                    ct_scaled: torch.Tensor, ct_host: Optional[np.ndarray],
                    bias: Optional[torch.Tensor], bits: int, fmt: int, in_f: int, kp: int,
                    out_f: int, cache: Optional[FWHTCache]) -> torch.Tensor:
    """The forward of PolarQuantLinearMethod.apply on explicit buffers:

    * M <= 32 with a 16-bit x: ``pe_linear_forward`` (FWHT fused into the
      decode GEMV);
    * otherwise ``fwht_pairs`` (through ``cache`` when given) and
      ``pe_linear_forward_xtf``."""
    orig_shape = x.shape
    dev = _lib.require_device(x, codes)
    if not x.is_floating_point():
        raise TypeError(f"PolarEngine linear takes floating-point activations, got {x.dtype}")
    out_dtype = x.dtype if x.dtype in (torch.float16, torch.bfloat16) else torch.float16
    x2 = x.reshape(-1, in_f)
    m = x2.shape[0]
    y = torch.empty(m, out_f, dtype=out_dtype, device=dev)
    if m == 0:
        return y.view(*orig_shape[:-1], out_f)
    b = None
    if bias is not None:
        b = bias.to(device=dev, dtype=out_dtype).contiguous()
    L = _lib.lib()
    st = _lib.stream_ptr(dev)
    n_levels = ct_scaled.numel()
    ct_ptr = None if ct_host is None else ct_host.ctypes.data
    out_code = _lib.act_dtype(y)

    if m > _FUSED_FWHT_MAX_M or x.dtype != out_dtype:
        x_tf = cache.get(x, in_f) if cache is not None else None
        if x_tf is None:
            xp = x2 if kp == in_f else F.pad(x2, (0, kp - in_f))
            x_tf = fwht_pairs(xp)
            if cache is not None:
                cache.put(x, in_f, x_tf)
        ws_bytes = L.pe_linear_xtf_workspace_size(m, kp, out_f, bits, fmt)
        ws = _lib.workspace(dev, ws_bytes)
        rc = L.pe_linear_forward_xtf(
            x_tf.data_ptr(), m, kp, codes.data_ptr(), bits, fmt, norms.data_ptr(),
            ct_scaled.data_ptr(), ct_ptr, n_levels, _lib.ptr(b), out_code, y.data_ptr(), out_f,
            _lib.ptr(ws), ws_bytes, st)
        _lib.check(rc, "pe_linear_forward_xtf")
    else:
        xc = x2 if kp == in_f else F.pad(x2, (0, kp - in_f))
        xc = xc.contiguous()
        ws_bytes = L.pe_linear_workspace_size(m, kp, out_f, bits, fmt)
        ws = _lib.workspace(dev, ws_bytes)
        rc = L.pe_linear_forward(
            xc.data_ptr(), out_code, m, kp, kp, codes.data_ptr(), bits, fmt, norms.data_ptr(),
            ct_scaled.data_ptr(), ct_ptr, n_levels, _lib.ptr(b), y.data_ptr(), out_f,
            _lib.ptr(ws), ws_bytes, st)
        _lib.check(rc, "pe_linear_forward")
    return y.view(*orig_shape[:-1], out_f)


# The linear forward as a torch custom op, for traced / compiled models
# (torch.compile cannot trace the raw-pointer ctypes call). The fake
# implementation gives the output's shape and dtype.
@torch.library.custom_op("polarengine::linear_apply", mutates_args=())
def _linear_apply_op(x: torch.Tensor, codes: torch.Tensor, norms: torch.Tensor,
                     ct_scaled: torch.Tensor, bias: Optional[torch.Tensor], bits: int, fmt: int,
                     in_f: int, in_f_padded: int, out_f: int,
                     ct_host: List[float]) -> torch.Tensor:
    host = np.asarray(ct_host, dtype=np.float32) if ct_host else None
    return _linear_forward(x, codes, norms, ct_scaled, host, bias, bits, fmt, in_f, in_f_padded,
                           out_f, None)


@_linear_apply_op.register_fake
def _linear_apply_fake(x, codes, norms, ct_scaled, bias, bits, fmt, in_f, in_f_padded, out_f,
                       ct_host):
    out_dtype = x.dtype if x.dtype in (torch.float16, torch.bfloat16) else torch.float16
    return x.new_empty((*x.shape[:-1], out_f), dtype=out_dtype)


def create_fwht_clear_hook(linear_method: PolarQuantLinearMethod):
    """Forward pre-hook clearing the FWHT cache (reference: linear_method.py:265-288)."""

    def hook(module: torch.nn.Module, args):
        linear_method._fwht_cache.clear()

    return hook


def install_fwht_cache_hooks(model: torch.nn.Module, cache: Optional[FWHTCache] = None) -> int:
    """Scope the FWHT cache to every forward of each module that has a
    PolarQuant linear as a direct child (e.g. a decoder layer's attention and
    MLP blocks): a forward pre-hook empties the cache and opens a scope, a
    forward hook (also run when the forward raises) empties it and closes the
    scope. Returns how many modules were hooked.

    Sibling projections called inside one such forward (q/k/v on the same
    hidden state, gate/up) share one transform, also for inference tensors,
    which the cache serves only inside a scope; a new forward of the parent
    always starts empty, so a hidden-state buffer rewritten outside torch
    between forwards can never be served a stale transform, and the
    transform is released when the parent's forward returns. The reference
    defines the clearing hook (linear_method.py:265-288) but registers it
    nowhere."""
    cache = GLOBAL_FWHT_CACHE if cache is None else cache

    def pre_hook(module: torch.nn.Module, args):
        cache.enter_scope()

    def post_hook(module: torch.nn.Module, args, output):
        cache.exit_scope()

    n = 0
    for parent in model.modules():
        if any(isinstance(getattr(child, "quant_method", None), PolarQuantLinearMethod)
               for child in parent.children()):
            if not getattr(parent, "_polar_fwht_hook", False):
                parent.register_forward_pre_hook(pre_hook)
                parent.register_forward_hook(post_hook, always_call=True)
                parent._polar_fwht_hook = True
                n += 1
    return n
