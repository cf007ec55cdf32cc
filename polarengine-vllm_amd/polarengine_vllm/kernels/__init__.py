"""gfx950 kernels behind the reference's kernel-module names."""

from polarengine_vllm.kernels.fwht import FWHTCache, build_hadamard, fwht_matmul, fwht_pairs
from polarengine_vllm.kernels.polar_gemm import polar_gemm, polar_gemm_packed, polar_matmul
from polarengine_vllm.kernels.polar_gemv import pack_codes_int4, polar_gemv, polar_gemv_packed
from polarengine_vllm.kernels.polar_gemv_splitk import polar_gemv_packed_splitk, polar_gemv_splitk

__all__ = [
    "FWHTCache", "build_hadamard", "fwht_matmul", "fwht_pairs",
    "polar_gemm", "polar_gemm_packed", "polar_matmul",
    "pack_codes_int4", "polar_gemv", "polar_gemv_packed",
    "polar_gemv_packed_splitk", "polar_gemv_splitk",
]
