"""PolarEngine quantized-linear path for MI355X (gfx950).

vLLM plugin (entry point group ``vllm.general_plugins``, name ``polarengine``)
with the reference's API names: ``PolarQuantConfig`` ("polarengine"),
``PolarQuantLinearMethod``, the MoE methods, and the kernel modules under
``polarengine_vllm.kernels``. All per-token compute runs in the hand-written
HIP library ``libpolarengine_amd.so`` through its C ABI.
"""

__version__ = "0.6.0"


def register_polar_quant() -> None:
    """vLLM plugin entry point: import the config so it registers itself.

    The reference additionally monkey-patches vLLM's loader to dequantize
    codes into bf16 weights (reference __init__.py:41-92), which bypasses its
    own quantized kernels; this package keeps the codes quantized in memory
    and does not patch vLLM.
    """
    try:
        from polarengine_vllm.config import PolarQuantConfig  # noqa: F401
    except ImportError as exc:  # pragma: no cover - vLLM import problems
        import warnings
        warnings.warn(f"Failed to register PolarEngine quantization with vLLM: {exc}")
