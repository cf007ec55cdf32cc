"""Checkpoint loading for PolarEngine models (reference: polarengine_vllm/loader.py).

A PolarEngine checkpoint is a directory holding ``polar_config.json``, the
safetensors shard(s) (with ``model.safetensors.index.json`` when sharded) and
optionally the HuggingFace ``config.json``. Two on-disk formats carry the
quantized layers:

* ``polar_engine_v4`` / ``polar_engine_v5`` (split tensors): ``<layer>.codes``
  (int8 ``[N, Kp]``, or uint8 nibbles ``[N, Kp/2]`` for bits <= 4, or Q5 bytes
  ``[N, Kp*5/8]`` when the layer's metadata says ``packed_q5``),
  ``<layer>.norms`` (fp16 ``[N, nb]``) and ``<layer>.ct_scaled`` (fp32) or
  ``<layer>.ct`` (unscaled; divided by sqrt(block_size) at load);
* ``hlwq-q5`` (and the ``hlwq-q4`` / ``hlwq-q3`` names): ``<layer>.weight__packed``
  (``bitpack_5``, MSB-first), ``<layer>.weight__norms`` and
  ``<layer>.weight__meta`` = ``[out_f, n_blocks, block_size, total_codes(, in_f)]``;
  the codebook is the 32-level Lloyd-Max table scaled by 1/sqrt(block_size),
  whatever the format's name says (as the reference does, loader.py:369-386).

What differs from the reference, on purpose:

* Q5 and HLWQ codes are unpacked on the GPU by the HIP kernels
  ``pe_unpack_q5`` / ``pe_unpack_q5_hlwq`` when the loader's device is a GPU
  (``PolarWeightLoader(..., device="cuda")``); the reference unpacks on the CPU;
* :meth:`PolarWeightLoader.is_packed` reads the codes tensor's shape from the
  safetensors header instead of loading the tensor (reference: loader.py:514-529);
* :func:`merged_weight_loader` and :func:`load_weights_into_layer` put the
  loaded tensors into the buffers that ``PolarQuantLinearMethod.create_weights``
  registers, including merged QKV / gate_up layers whose shards arrive one at a
  time. The reference registers those buffers but gives vLLM no loader for
  them, and instead patches vLLM to dequantize the codes into bf16 weights
  (reference __init__.py:41-92, weight_converter.py:70-184).
"""

from __future__ import annotations

import json
import logging
import math
import os
from pathlib import Path
from typing import Any, Callable, Dict, List, Optional, Sequence, Set, Tuple, Union

import torch
from safetensors import safe_open

from polarengine_vllm.packing import unpack_codes_q5, unpack_codes_q5_hlwq
from polarengine_vllm.utils import get_centroids

logger = logging.getLogger(__name__)

SPLIT_FORMATS = ("polar_engine_v4", "polar_engine_v5")
HLWQ_FORMATS = ("hlwq-q5", "hlwq-q4", "hlwq-q3")
# tensor-name suffixes of the split format's quantized components
POLAR_SUFFIXES = (".codes", ".norms", ".ct_scaled", ".ct")
_HLWQ_SUFFIXES = (".weight__packed", ".weight__norms", ".weight__meta")


# ---------------------------------------------------------------------------
# config and weight map
# ---------------------------------------------------------------------------

def load_polar_config(model_dir: str) -> dict:
    """Parse ``polar_config.json`` (reference: loader.py:35-66).

    Raises FileNotFoundError when it is missing; an unknown ``format`` is
    logged and loading proceeds."""
    path = os.path.join(model_dir, "polar_config.json")
    if not os.path.isfile(path):
        raise FileNotFoundError(f"{model_dir} holds no polar_config.json (not a PolarEngine "
                                f"checkpoint directory)")
    with open(path, "r") as f:
        config = json.load(f)
    fmt = str(config.get("format", "unknown"))
    if fmt not in SPLIT_FORMATS and fmt.lower() not in HLWQ_FORMATS:
        logger.warning("checkpoint format %r is not one this loader knows; trying the "
                       "split-tensor layout", fmt)
    return config


def get_weight_map(model_dir: str) -> Dict[str, str]:
    """Tensor name -> shard file name (reference: loader.py:73-120).

    Uses ``model.safetensors.index.json`` when present, else scans every
    ``*.safetensors`` file of the directory."""
    index = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.isfile(index):
        with open(index, "r") as f:
            return dict(json.load(f).get("weight_map", {}))
    files = sorted(Path(model_dir).glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"{model_dir} has neither a safetensors index nor any "
                                f"*.safetensors shard")
    weight_map: Dict[str, str] = {}
    for path in files:
        with safe_open(str(path), framework="pt", device="cpu") as f:
            for key in f.keys():
                weight_map[key] = path.name
    return weight_map


def _is_polar_component(key: str) -> bool:
    return key.endswith(POLAR_SUFFIXES) or key.endswith(_HLWQ_SUFFIXES)


def load_polar_model(model_dir: str, device: str = "cuda",
                     dtype: torch.dtype = torch.float16) -> Tuple[Dict[str, torch.Tensor], dict, dict]:
    """Every tensor of the checkpoint as a flat state dict on ``device``
    (reference: loader.py:127-199). Floating-point tensors that are not
    quantized components are cast to ``dtype``; codes, norms and centroids
    keep their stored dtypes. Returns ``(state_dict, hf_config, polar_config)``."""
    polar_config = load_polar_config(model_dir)
    hf_config: dict = {}
    hf_path = os.path.join(model_dir, "config.json")
    if os.path.isfile(hf_path):
        with open(hf_path, "r") as f:
            hf_config = json.load(f)
    by_shard: Dict[str, List[str]] = {}
    for key, shard in get_weight_map(model_dir).items():
        by_shard.setdefault(shard, []).append(key)
    state: Dict[str, torch.Tensor] = {}
    for shard, keys in by_shard.items():
        with safe_open(os.path.join(model_dir, shard), framework="pt", device="cpu") as f:
            for key in keys:
                t = f.get_tensor(key)
                if not _is_polar_component(key) and t.is_floating_point():
                    t = t.to(dtype)
                state[key] = t.to(device) if device != "cpu" else t
    return state, hf_config, polar_config


# ---------------------------------------------------------------------------
# per-layer loader
# ---------------------------------------------------------------------------

def _default_device() -> str:
    return "cuda" if torch.cuda.is_available() else "cpu"


class PolarWeightLoader:
    """Per-layer access to a PolarEngine checkpoint (reference: loader.py:206-559).

    ``load_layer_weights(name)`` returns ``codes`` (int8 ``[N, Kp]``, or uint8
    nibbles ``[N, Kp/2]`` as stored), ``norms`` fp16 ``[N, nb]``, ``ct_scaled``
    fp32 and ``bias`` when present, on the loader's device; a layer that is not
    quantized gives ``weight`` (and ``bias``). Shard files stay open until
    :meth:`close` (also a context manager)."""

    def __init__(self, model_dir: str, polar_config: dict,
                 device: Optional[Union[str, torch.device]] = None) -> None:
        self.model_dir = model_dir
        self.polar_config = polar_config
        self.device = torch.device(device if device is not None else _default_device())
        self.weight_map = get_weight_map(model_dir)
        self._open_files: Dict[str, Any] = {}
        self._quantized_layers: Set[str] = set(polar_config.get("layers", {}).keys())

    # -- files --------------------------------------------------------------
    def _get_file(self, shard: str) -> Any:
        if shard not in self._open_files:
            self._open_files[shard] = safe_open(os.path.join(self.model_dir, shard),
                                                framework="pt", device="cpu")
        return self._open_files[shard]

    def close(self) -> None:
        self._open_files.clear()

    def __enter__(self) -> "PolarWeightLoader":
        return self

    def __exit__(self, *args: Any) -> None:
        self.close()

    # -- tensors ------------------------------------------------------------
    def load_tensor(self, key: str, device: Optional[Union[str, torch.device]] = None) -> torch.Tensor:
        """One tensor by name; KeyError (listing a few names) when absent."""
        if key not in self.weight_map:
            raise KeyError(f"no tensor named {key!r} in the checkpoint (it has "
                           f"{len(self.weight_map)}, e.g. {list(self.weight_map)[:10]})")
        t = self._get_file(self.weight_map[key]).get_tensor(key)
        dev = torch.device(device) if device is not None else self.device
        return t if dev.type == "cpu" else t.to(dev)

    def tensor_shape(self, key: str) -> Tuple[int, ...]:
        """Shape of a stored tensor from the safetensors header (no data read)."""
        if key not in self.weight_map:
            raise KeyError(f"no tensor named {key!r} in the checkpoint")
        return tuple(self._get_file(self.weight_map[key]).get_slice(key).get_shape())

    def _format(self) -> str:
        return str(self.polar_config.get("format", "polar_engine_v4")).lower()

    def _layer_meta(self, layer_name: str) -> dict:
        return self.polar_config.get("layers", {}).get(layer_name, {}) or {}

    def load_layer_weights(self, layer_name: str) -> Dict[str, torch.Tensor]:
        """The components of one layer (reference: loader.py:300-445)."""
        out: Dict[str, torch.Tensor] = {}
        if self.is_quantized_layer(layer_name):
            if self._format() in HLWQ_FORMATS:
                out.update(self._load_hlwq(layer_name))
            else:
                out.update(self._load_split(layer_name))
        else:
            if layer_name + ".weight" in self.weight_map:
                out["weight"] = self.load_tensor(layer_name + ".weight")
            elif layer_name in self.weight_map:  # bare parameter name
                out["weight"] = self.load_tensor(layer_name)
            else:
                raise KeyError(f"unquantized layer {layer_name!r} has no weight: neither "
                               f"{layer_name + '.weight'!r} nor {layer_name!r} is stored")
        if layer_name + ".bias" in self.weight_map:
            out["bias"] = self.load_tensor(layer_name + ".bias")
        return out

    def _load_split(self, layer_name: str) -> Dict[str, torch.Tensor]:
        out = {"codes": self.load_tensor(layer_name + ".codes"),
               "norms": self.load_tensor(layer_name + ".norms")}
        if layer_name + ".ct_scaled" in self.weight_map:
            out["ct_scaled"] = self.load_tensor(layer_name + ".ct_scaled")
        elif layer_name + ".ct" in self.weight_map:
            bs = int(self.polar_config.get("block_size", 128))
            out["ct_scaled"] = self.load_tensor(layer_name + ".ct") / math.sqrt(bs)
        else:
            raise KeyError(f"layer {layer_name!r} stores no codebook: expected "
                           f"{layer_name + '.ct_scaled'!r} or {layer_name + '.ct'!r}")
        meta = self._layer_meta(layer_name)
        if meta.get("packed_q5", False):
            bs = int(meta.get("block_size", self.polar_config.get("block_size", 128)))
            out["codes"] = unpack_codes_q5(out["codes"], bs)
        return out

    def _load_hlwq(self, layer_name: str) -> Dict[str, torch.Tensor]:
        packed_key = layer_name + ".weight__packed"
        if packed_key not in self.weight_map:
            raise KeyError(f"bit-packed (HLWQ) layer {layer_name!r} lacks {packed_key!r}; "
                           f"stored under that prefix: "
                           f"{[k for k in self.weight_map if k.startswith(layer_name)][:5]}")
        packed = self.load_tensor(packed_key)
        norms = self.load_tensor(layer_name + ".weight__norms")
        meta = [int(v) for v in self.load_tensor(layer_name + ".weight__meta", "cpu").reshape(-1).tolist()]
        out_f, n_blocks, bs, total = meta[0], meta[1], meta[2], meta[3]
        in_f = meta[4] if len(meta) >= 5 else n_blocks * bs
        codes = unpack_codes_q5_hlwq(packed.reshape(-1), total=total)
        return {"codes": codes.reshape(out_f, n_blocks * bs).to(torch.int8),
                "norms": norms.to(torch.float16),
                "ct_scaled": (get_centroids(5) / math.sqrt(bs)).to(torch.float32).to(norms.device),
                "_hlwq_in_f": torch.tensor([in_f], dtype=torch.int64)}

    # -- metadata -----------------------------------------------------------
    def is_quantized_layer(self, layer_name: str) -> bool:
        """Listed in ``layers``, or a ``.codes`` / ``.weight__packed`` tensor
        exists (reference: loader.py:447-472)."""
        return (layer_name in self._quantized_layers
                or layer_name + ".codes" in self.weight_map
                or layer_name + ".weight__packed" in self.weight_map)

    def get_layer_bits(self, layer_name: str) -> int:
        """Per-layer ``bits``, else the longest ``bit_assignment`` pattern
        contained in the name, else 5 (reference: loader.py:474-505)."""
        meta = self._layer_meta(layer_name)
        if "bits" in meta:
            return int(meta["bits"])
        best: Optional[str] = None
        for pattern in self.polar_config.get("bit_assignment", {}):
            if pattern in layer_name and (best is None or len(pattern) > len(best)):
                best = pattern
        return int(self.polar_config["bit_assignment"][best]) if best is not None else 5

    def is_packed(self, layer_name: str) -> bool:
        """Codes stored packed: Q5 bytes (``packed_q5``) or, for bits <= 4,
        nibbles -- decided by the stored codes' last dimension against
        ``in_f_padded`` when the layer has metadata (reference: loader.py:507-533)."""
        meta = self._layer_meta(layer_name)
        if meta.get("packed_q5", False):
            return True
        if self.get_layer_bits(layer_name) > 4:
            return False
        if meta:
            key = layer_name + ".codes"
            if key in self.weight_map:
                return self.tensor_shape(key)[-1] == int(meta.get("in_f_padded", 0)) // 2
        return True

    def get_all_layer_names(self) -> List[str]:
        return sorted(self.polar_config.get("layers", {}).keys())


# ---------------------------------------------------------------------------
# tensor parallelism helpers (reference: loader.py:563-650)
# ---------------------------------------------------------------------------

def _shard_rows(t: torch.Tensor, tp_rank: int, tp_size: int, what: str) -> torch.Tensor:
    rows = t.shape[0]
    if rows % tp_size:
        raise ValueError(f"{rows} {what} do not split evenly over {tp_size} tensor-parallel "
                         f"ranks")
    n = rows // tp_size
    return t[tp_rank * n:(tp_rank + 1) * n].contiguous()


def shard_codes_for_tp(codes: torch.Tensor, tp_rank: int, tp_size: int, dim: int = 0) -> torch.Tensor:
    """Column-parallel (dim 0): this rank's rows; row-parallel (dim 1): the
    whole tensor (every rank needs all codes of its output rows)."""
    if tp_size <= 1 or dim == 1:
        return codes
    return _shard_rows(codes, tp_rank, tp_size, "output rows")


def shard_norms_for_tp(norms: torch.Tensor, tp_rank: int, tp_size: int, n_blocks: int,
                       dim: int = 0) -> torch.Tensor:
    """Same split as :func:`shard_codes_for_tp` for the ``[N, nb]`` norms."""
    if tp_size <= 1 or dim == 1:
        return norms
    return _shard_rows(norms, tp_rank, tp_size, "norm rows")


# ---------------------------------------------------------------------------
# filling the registered buffers
# ---------------------------------------------------------------------------

_QKV_IDS = {"q": 0, "k": 1, "v": 2}


def merged_weight_loader(output_partition_sizes: Sequence[int], tp_rank: int = 0,
                         tp_size: int = 1) -> Callable[..., None]:
    """A vLLM ``weight_loader`` for the ``codes`` / ``norms`` buffers of a
    (possibly merged) column-parallel layer.

    vLLM calls ``loader(param, loaded_weight, loaded_shard_id)`` once per
    stored shard of a merged layer (ids ``"q"``/``"k"``/``"v"`` or ``0``/``1``
    for gate/up) and once with ``loaded_shard_id=None`` for a plain layer.
    Each shard's rows land at the row offset of its partition; under tensor
    parallelism the rank's slice of the shard is taken first. Nibble-packed or
    int8 rows are copied as stored (the buffer is resized to the stored row
    width on the first call)."""
    sizes = [int(s) for s in output_partition_sizes]
    offsets = [sum(sizes[:i]) for i in range(len(sizes))]

    def load(param: torch.Tensor, loaded_weight: torch.Tensor,
             loaded_shard_id: Optional[Union[int, str]] = None) -> None:
        src = shard_codes_for_tp(loaded_weight, tp_rank, tp_size)
        if loaded_shard_id is None:  # the whole (unmerged) tensor
            if tuple(param.shape) != tuple(src.shape) or param.dtype != src.dtype:
                param.data = torch.empty(src.shape, dtype=src.dtype, device=param.device)
            param.data.copy_(src)
            return
        if isinstance(loaded_shard_id, str):
            if loaded_shard_id not in _QKV_IDS:
                raise ValueError(f"unknown shard id {loaded_shard_id!r}")
            idx = _QKV_IDS[loaded_shard_id]
        else:
            idx = int(loaded_shard_id)
        if not 0 <= idx < len(sizes):
            raise ValueError(f"shard id {loaded_shard_id!r} outside {len(sizes)} partitions")
        if src.shape[0] != sizes[idx]:
            raise ValueError(f"shard {loaded_shard_id!r} has {src.shape[0]} rows, "
                             f"partition expects {sizes[idx]}")
        if tuple(param.shape[1:]) != tuple(src.shape[1:]) or param.dtype != src.dtype:
            # the first shard decides the stored row width and element type
            # (int8 codes, uint8 nibbles, fp16 norms)
            param.data = torch.zeros((sum(sizes),) + tuple(src.shape[1:]), dtype=src.dtype,
                                     device=param.device)
        param.data[offsets[idx]:offsets[idx] + sizes[idx]].copy_(src)

    return load


def load_weights_into_layer(layer: torch.nn.Module, weights: Dict[str, torch.Tensor],
                            method: Any = None) -> None:
    """Put one layer's loaded components into the buffers registered by
    ``PolarQuantLinearMethod.create_weights`` and run
    ``process_weights_after_loading`` (when ``method`` is given).

    ``codes`` may be int8 ``[N, Kp]`` or stored nibbles uint8 ``[N, Kp/2]``
    (then they become ``layer.codes_packed`` and the in-memory pack step is
    skipped). Shapes are checked against the layer's dimensions."""
    n, kp = layer.out_f, layer.in_f_padded
    codes = weights["codes"]
    norms = weights["norms"]
    ct = weights["ct_scaled"]
    dev = layer.codes.device if hasattr(layer, "codes") else codes.device
    if tuple(norms.shape) != (n, layer.n_blocks):
        raise ValueError(f"norms shape {tuple(norms.shape)} != {(n, layer.n_blocks)}")
    if ct.numel() != layer.ct_scaled.numel():
        raise ValueError(f"codebook has {ct.numel()} levels, layer expects {layer.ct_scaled.numel()}")
    if tuple(codes.shape) == (n, kp):
        layer.codes = codes.to(device=dev, dtype=torch.int8).contiguous()
        layer.packed = False
    elif tuple(codes.shape) == (n, kp // 2) and layer.bits <= 4:
        layer.codes_packed = codes.to(device=dev).view(torch.uint8).contiguous()
        layer.in_f_half = kp // 2
        layer.packed = True
        if hasattr(layer, "codes"):
            del layer.codes
    else:
        raise ValueError(f"codes shape {tuple(codes.shape)} fits neither {(n, kp)} "
                         f"nor the nibble layout {(n, kp // 2)}")
    layer.norms = norms.to(device=dev, dtype=torch.float16).contiguous()
    layer.ct_scaled = ct.to(device=dev, dtype=torch.float32).contiguous()
    if "bias" in weights:
        layer.bias = weights["bias"].to(device=dev, dtype=torch.float16).contiguous()
    if method is not None:
        method.process_weights_after_loading(layer)
