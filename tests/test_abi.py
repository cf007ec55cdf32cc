"""The C-ABI library loads and exports every function declared in
include/*.h (no compute calls: this runs without a GPU)."""

import ctypes
import glob
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(pe_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = _declared()
    for n in ("pe_fwht128", "pe_polar_gemv", "pe_polar_gemv_packed", "pe_linear_forward",
              "pe_linear_forward_xtf", "pe_polar_matmul", "pe_pack_nibble", "pe_unpack_q5"):
        assert n in names


def test_library_exports_every_declared_symbol():
    from polarengine_vllm import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"library not built: {_lib.LIB_PATH}")
    handle = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(_declared()) if not hasattr(handle, n)]
    assert not missing, f"declared but not exported: {missing}"
    # the Python binding covers exactly the declared set
    assert set(_lib.exported_symbols()) == _declared()


def test_status_strings_and_version():
    from polarengine_vllm import _lib
    L = _lib.lib()
    assert L.pe_abi_version() >= 1
    assert L.pe_status_string(0) == b"ok"
    assert b"aligned" in L.pe_status_string(4)
    assert L.pe_status_string(999) == b"unknown status"


def test_argument_errors_without_gpu_work():
    """Validation happens before any launch: these return errors on a host
    without a GPU too."""
    from polarengine_vllm import _lib
    L = _lib.lib()
    # NULL pointers
    assert L.pe_fwht128(None, 0, 1, 128, 128, None, 2, None) == 1
    # K not a multiple of 128
    assert L.pe_pack_nibble(16, 16, 1, 100, None) == 2
    # misaligned
    assert L.pe_pack_nibble(17, 16, 1, 128, None) == 4
    # bad bits / packing combination
    assert L.pe_linear_forward(16, 0, 1, 128, 128, 16, 5, 1, 16, 16, None, 32, None, 16, 8,
                               None, 0, None) == 3
    # unknown weight-format flag
    assert L.pe_linear_forward(16, 0, 1, 128, 128, 16, 4, 4, 16, 16, None, 16, None, 16, 8,
                               None, 0, None) == 3


def test_no_cpu_fallback():
    import torch
    from polarengine_vllm.kernels.fwht import fwht_matmul
    with pytest.raises(RuntimeError, match="GPU only"):
        fwht_matmul(torch.randn(2, 128))
