"""ctypes binding of libpolarengine_amd.so (the C ABI in include/polarengine_amd.h).

The library is the only compute path of this package: there is no CPU or
PyTorch fallback. If the shared object is missing, every kernel entry point
raises ``RuntimeError`` naming the build command.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get(
    "POLARENGINE_AMD_LIB",
    os.path.join(os.path.dirname(_HERE), "lib", "libpolarengine_amd.so"),
)

PE_OK = 0
# status codes of include/polarengine_amd.h
PE_ERR_NULL, PE_ERR_DIMS, PE_ERR_BITS, PE_ERR_ALIGN = 1, 2, 3, 4
PE_ERR_DTYPE, PE_ERR_WORKSPACE, PE_ERR_LAUNCH, PE_ERR_DEVICE = 5, 6, 7, 8
PE_ERR_SCRATCH = 9
PE_PACK_NIBBLE, PE_LAYOUT_TILE16 = 1, 2
PE_DTYPE_F16, PE_DTYPE_BF16, PE_DTYPE_F32 = 0, 1, 2
PE_XTF_F32, PE_XTF_F16, PE_XTF_PAIR_F16, PE_XTF_BF16 = 0, 1, 2, 3

_c_int, _c_i64, _c_sz, _vp = ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/polarengine_amd.h
_SIGNATURES = {
    "pe_status_string": (ctypes.c_char_p, [_c_int]),
    "pe_abi_version": (_c_int, []),
    "pe_fwht128": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp]),
    "pe_fwht_pow2": (_c_int, [_vp, _c_int, _c_i64, _c_i64, _c_i64, _vp, _c_int, _vp]),
    "pe_polar_gemv": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "pe_polar_gemv_packed": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_int, _vp]),
    "pe_polar_matmul_workspace_size": (_c_sz, [_c_i64, _c_int]),
    "pe_polar_matmul": (_c_int, [_vp, _c_int, _vp, _c_i64, _vp, _vp, _c_int, _vp, _c_int, _c_int,
                                 _vp, _c_sz, _vp]),
    "pe_linear_workspace_size": (_c_sz, [_c_i64, _c_int, _c_int, _c_int, _c_int]),
    "pe_linear_forward": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_i64, _vp, _c_int, _c_int, _vp,
                                   _vp, _vp, _c_int, _vp, _vp, _c_int, _vp, _c_sz, _vp]),
    "pe_linear_noalloc_max_bytes": (_c_sz, []),
    "pe_linear_forward_noalloc": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_i64, _vp, _c_int,
                                           _c_int, _vp, _vp, _vp, _c_int, _vp, _vp, _c_int, _vp]),
    "pe_linear_xtf_workspace_size": (_c_sz, [_c_i64, _c_int, _c_int, _c_int, _c_int]),
    "pe_linear_forward_xtf": (_c_int, [_vp, _c_i64, _c_int, _vp, _c_int, _c_int, _vp, _vp, _vp,
                                       _c_int, _vp, _c_int, _vp, _c_int, _vp, _c_sz, _vp]),
    "pe_pack_nibble": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "pe_unpack_q5": (_c_int, [_vp, _vp, _c_i64, _c_i64, _vp]),
    "pe_unpack_q5_hlwq": (_c_int, [_vp, _c_i64, _vp, _c_i64, _vp]),
    "pe_kv_quantize": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_i64, _vp, _c_int, _vp, _vp, _vp]),
    "pe_kv_dequantize": (_c_int, [_vp, _vp, _c_i64, _c_int, _vp, _c_int, _vp, _c_i64, _vp]),
    "pe_quantize": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_i64, _vp, _c_int, _c_int, _vp, _vp,
                             _vp]),
    "pe_tile_weights": (_c_int, [_vp, _vp, _c_i64, _c_int, _c_int, _vp, _vp, _vp]),
    "pe_moe_route": (_c_int, [_vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp]),
    "pe_moe_route_grouped": (_c_int, [_vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _c_int,
                                      _c_int, _vp, _vp, _vp]),
    "pe_moe_workspace_size": (_c_sz, [_c_i64, _c_int, _c_int, _c_int, _c_int]),
    "pe_moe_forward": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                _vp, _c_int, _c_int, _vp, _vp, _c_int,
                                _vp, _c_int, _c_int, _vp, _vp, _c_int,
                                _vp, _vp, _c_sz, _vp]),
    "pe_moe_forward_routed": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_int, _c_int, _c_int,
                                       _vp, _c_int, _c_int, _vp, _c_int, _c_int,
                                       _vp, _c_int, _c_int, _vp, _vp, _c_int,
                                       _vp, _c_int, _c_int, _vp, _vp, _c_int,
                                       _vp, _vp, _c_sz, _vp]),
}

# measurement helpers (include/polarengine_amd_bench.h)
_SIGNATURES.update({
    "pe_stream_read_sink_bytes": (_c_sz, [_c_i64]),
    "pe_stream_read": (_c_int, [_vp, _c_i64, _vp, ctypes.c_uint32, _vp]),
    "pe_copy": (_c_int, [_vp, _vp, _c_i64, _vp]),
})

_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load the shared library once; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"PolarEngine HIP library not found at {LIB_PATH}; build it with "
                "`python polarengine-vllm_amd/build_lib.py` (gfx950)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def exported_symbols():
    return list(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc != PE_OK:
        msg = lib().pe_status_string(rc).decode()
        raise RuntimeError(f"{what} failed: status {rc} ({msg})")


def stream_ptr(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one GPU; there is no CPU path."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "PolarEngine kernels run on the GPU only (got a tensor on "
                f"{t.device}); there is no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} vs {t.device}")
    if dev is None:
        raise RuntimeError("no tensor given")
    return dev


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def act_dtype(t: torch.Tensor) -> int:
    """PE_DTYPE_* code of a 16-bit activation tensor (fp16 or bf16)."""
    code = {torch.float16: PE_DTYPE_F16, torch.bfloat16: PE_DTYPE_BF16}.get(t.dtype)
    if code is None:
        raise TypeError(f"PolarEngine kernels take float16 or bfloat16 activations, got {t.dtype}")
    return code


_WS_CACHE: dict = {}
# Every buffer workspace() ever handed out, per key. A superseded buffer is
# never released: kernels receive workspaces as raw pointers, so a HIP graph
# captured before a growth keeps writing the old address on every replay, and
# its completion counters (which must stay zero between calls) must not be
# memory that the caching allocator has handed to someone else.
_WS_RETIRED: dict = {}


def _ws_key(device: torch.device):
    if device.type != "cuda":
        return (device, 0)
    return (device, torch.cuda.current_stream(device).cuda_stream)


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device, per-stream growable workspace (uint8), reused across calls.
    Zero-filled when allocated: the library keeps completion counters in its
    first 4 KB, which must start at zero and which every call leaves zero.
    Growth allocates a larger buffer and keeps the old one alive for the life
    of the process (see _WS_RETIRED)."""
    if nbytes <= 0:
        return None
    key = _ws_key(device)
    buf = _WS_CACHE.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _WS_RETIRED.setdefault(key, []).append(buf)
        # geometric growth: the retired buffers never add up to more than the live one
        size = max(nbytes, 1 << 20, 2 * buf.numel() if buf is not None else 0)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _WS_CACHE[key] = buf
    return buf
