"""PolarQuant quantization config for vLLM (reference: polarengine_vllm/config.py).

Parses ``polar_config.json`` and picks a quantize method per layer. Works
without vLLM (stub base classes), as the reference does.
"""

from __future__ import annotations

import logging
from typing import Any, Dict, List, Optional

import torch

logger = logging.getLogger(__name__)

_VLLM_AVAILABLE = True
try:
    from vllm.model_executor.layers.quantization.base_config import (  # type: ignore
        QuantizationConfig, QuantizeMethodBase)
except Exception:
    _VLLM_AVAILABLE = False

    class QuantizationConfig:  # type: ignore[no-redef]
        """Stub base class used when vLLM is not installed."""

    class QuantizeMethodBase:  # type: ignore[no-redef]
        """Stub base class used when vLLM is not installed."""

_register = None
try:
    from vllm.model_executor.layers.quantization import register_quantization_config  # type: ignore
    _register = register_quantization_config
except Exception:
    pass

_KNOWN_FORMATS = {"polar_engine_v4", "polar_engine_v5", "hlwq-q5", "hlwq-q4", "hlwq-q3"}


def _build(decorator):
    @decorator("polarengine") if decorator else (lambda cls: cls)
    class PolarQuantConfig(QuantizationConfig):
        """Config of a PolarEngine model: block size, bit rules, per-layer meta."""

        def __init__(self, block_size: int = 128,
                     bit_assignment: Optional[Dict[str, int]] = None,
                     layers_meta: Optional[Dict[str, Dict[str, Any]]] = None) -> None:
            self.block_size = block_size
            self.bit_assignment: Dict[str, int] = bit_assignment or {}
            self.layers_meta: Dict[str, Dict[str, Any]] = layers_meta or {}
            self.packed_modules_mapping: Dict[str, Any] = {}

        def __repr__(self) -> str:
            bits = sorted(set(self.bit_assignment.values())) if self.bit_assignment else []
            return (f"<polarengine quantization: {len(self.layers_meta)} layer entries, "
                    f"bit widths {bits}, {self.block_size}-wide blocks>")

        @staticmethod
        def get_name() -> str:
            return "polarengine"

        @staticmethod
        def get_supported_act_dtypes() -> List[torch.dtype]:
            # reference list; the gfx950 kernels compute on float16 operands
            return [torch.float16, torch.bfloat16]

        @staticmethod
        def get_min_capability() -> int:
            return 70

        @staticmethod
        def get_config_filenames() -> List[str]:
            return ["polar_config.json"]

        @classmethod
        def from_config(cls, config: Dict[str, Any]) -> "PolarQuantConfig":
            fmt = config.get("format", "polar_engine_v4")
            if fmt not in _KNOWN_FORMATS:
                logger.warning("polar_config.json declares format %r, which this build does "
                               "not know; continuing with the split-tensor reader", fmt)
            return cls(block_size=config.get("block_size", 128),
                       bit_assignment=config.get("bit_assignment", {}),
                       layers_meta=config.get("layers", {}))

        def get_quant_method(self, layer: torch.nn.Module, prefix: str):
            """Method for ``layer``: PolarQuant linear / MoE, or unquantized.

            Without vLLM, layers that stay unquantized get ``None`` (there is
            no vLLM UnquantizedLinearMethod to return).
            """
            from polarengine_vllm.linear_method import PolarQuantLinearMethod
            cls_name = type(layer).__name__
            if "Embedding" in cls_name:
                return _unquantized_embedding()
            if "MoE" in cls_name or "Moe" in cls_name or "moe" in cls_name or hasattr(layer, "num_experts"):
                from polarengine_vllm.moe_method import PolarQuantMoEMethod
                b13 = self._resolve_bits(prefix + ".w13") or self._resolve_bits("gate_up_proj")
                b2 = self._resolve_bits(prefix + ".w2") or self._resolve_bits("down_proj")
                if b13 is None or b2 is None:
                    return _unquantized_moe(layer)
                return PolarQuantMoEMethod(block_size=self.block_size, bits13=b13, bits2=b2)
            if not isinstance(layer, torch.nn.Linear) and "Linear" not in cls_name:
                return _unquantized_linear()
            bits = self._resolve_bits(prefix)
            if bits is None:
                return _unquantized_linear()
            return PolarQuantLinearMethod(block_size=self.block_size, bits=bits,
                                          layer_meta=self.layers_meta.get(prefix, {}))

        def _resolve_bits(self, prefix: str) -> Optional[int]:
            """Exact ``layers[prefix].bits``, else the longest matching
            ``bit_assignment`` key, else None (reference: config.py:220-245)."""
            meta = self.layers_meta.get(prefix)
            if meta and "bits" in meta:
                return int(meta["bits"])
            best = None
            for pattern in self.bit_assignment:
                if pattern in prefix and (best is None or len(pattern) > len(best)):
                    best = pattern
            return None if best is None else int(self.bit_assignment[best])

    return PolarQuantConfig


def _unquantized_linear():
    if not _VLLM_AVAILABLE:
        return None
    from vllm.model_executor.layers.linear import UnquantizedLinearMethod  # type: ignore
    return UnquantizedLinearMethod()


def _unquantized_embedding():
    if not _VLLM_AVAILABLE:
        return None
    from vllm.model_executor.layers.vocab_parallel_embedding import (  # type: ignore
        UnquantizedEmbeddingMethod)
    return UnquantizedEmbeddingMethod()


def _unquantized_moe(layer):
    if not _VLLM_AVAILABLE:
        return None
    from polarengine_vllm.moe_method import PolarPassthroughMoEMethod
    return PolarPassthroughMoEMethod()


PolarQuantConfig = _build(_register)

if _VLLM_AVAILABLE and _register is None:
    try:
        from vllm.model_executor.layers.quantization import QUANTIZATION_METHODS  # type: ignore
        QUANTIZATION_METHODS.setdefault("polarengine", PolarQuantConfig)
    except Exception:
        logger.warning("Could not register PolarEngine quantization with vLLM.")
