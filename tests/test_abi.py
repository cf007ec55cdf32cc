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
    # whole-row FWHT: n not a power of two, above 32768, bad dtype
    assert L.pe_fwht_pow2(16, 2, 1, 96, 96, 16, 2, None) == 2
    assert L.pe_fwht_pow2(16, 2, 1, 65536, 65536, 16, 2, None) == 2
    assert L.pe_fwht_pow2(16, 7, 1, 64, 64, 16, 2, None) == 5
    # measurement helpers: sizes that are not whole 16-byte units, misaligned, NULL
    assert L.pe_stream_read(16, 100, 16, 0, None) == 2
    assert L.pe_copy(16, 32, 100, None) == 2
    assert L.pe_copy(16, 40, 128, None) == 4
    assert L.pe_copy(None, 32, 128, None) == 1
    assert L.pe_stream_read_sink_bytes(8192) == 1024 and L.pe_stream_read_sink_bytes(8193) == 2048
    # zero rows: valid arguments, nothing to do, nothing touched (the pointers
    # below are aligned placeholders, never dereferenced)
    assert L.pe_linear_forward(16, 0, 0, 128, 128, 16, 4, 1, 16, 16, None, 16, None, 16, 8,
                               None, 0, None) == 0
    assert L.pe_linear_forward_xtf(16, 0, 128, 16, 4, 1, 16, 16, None, 16, None, 0, 16, 8,
                                   None, 0, None) == 0


def test_no_cpu_fallback():
    import torch
    from polarengine_vllm.kernels.fwht import fwht_matmul
    with pytest.raises(RuntimeError, match="GPU only"):
        fwht_matmul(torch.randn(2, 128))


def _ru(v, a=256):
    return (v + a - 1) // a * a


def test_workspace_queries_cover_every_path():
    """Size queries (host code; 256 CUs assumed without a device) follow the
    path the call takes, M = 1 included: the fused decode kernel needs
    nothing; an M = 1 call past the decode kernel's limits on the tiled
    layout, or past the M = 1 GEMV's LDS budget on the row-major one, needs
    the pair-f16 transform; the reference-API matmul at M = 1 with int8 codes
    past 24576 needs its repacked activation."""
    from polarengine_vllm import _lib
    L = _lib.lib()
    NIB, T16 = _lib.PE_PACK_NIBBLE, _lib.PE_LAYOUT_TILE16
    # the headline decode shape: fused, no workspace
    assert L.pe_linear_workspace_size(1, 4096, 12288, 4, NIB | T16) == 0
    assert L.pe_linear_workspace_size(1, 12288, 4096, 3, NIB | T16) == 0
    # K = 53248 (416 blocks): too many activation registers for the decode
    # kernel at M = 1; tiled -> FWHT + matmul; row-major nibbles past 49152
    # too -> the same
    for fmt in (NIB | T16, NIB):
        assert L.pe_linear_workspace_size(1, 53248, 4096, 4, fmt) >= _ru(53248 * 2)
    # row-major int8, 128 blocks: the decode kernel holds x in LDS beside the
    # 256-entry table (64 KB + 32 KB): fused, no workspace
    assert L.pe_linear_workspace_size(1, 16384, 1000, 6, 0) == 0
    # reference-API matmul
    assert L.pe_polar_matmul_workspace_size(1, 4096) == 0
    assert L.pe_polar_matmul_workspace_size(1, 28672) >= 28672 * 2
    assert L.pe_polar_matmul_workspace_size(8, 4096) >= 8 * 4096 * 2
    # prefill: the pair-f16 transform at least
    assert L.pe_linear_workspace_size(2048, 4096, 12288, 4, NIB | T16) >= 2048 * 4096 * 2
    # invalid arguments: zero
    assert L.pe_linear_workspace_size(0, 4096, 4096, 4, NIB) == 0
    assert L.pe_linear_workspace_size(1, 4096, 4096, 9, 0) == 0


def test_workspace_checked_before_launch():
    """A call whose path needs workspace fails with PE_ERR_WORKSPACE (6)
    before launching anything when it gets none or too little."""
    from polarengine_vllm import _lib
    L = _lib.lib()
    NIB, T16 = _lib.PE_PACK_NIBBLE, _lib.PE_LAYOUT_TILE16
    need = L.pe_linear_workspace_size(1, 53248, 4096, 4, NIB | T16)
    assert need > 0
    assert L.pe_linear_forward(16, 0, 1, 53248, 53248, 16, 4, NIB | T16, 16, 16, None, 16, None,
                               16, 4096, None, 0, None) == 6
    assert L.pe_linear_forward(16, 0, 1, 53248, 53248, 16, 4, NIB | T16, 16, 16, None, 16, None,
                               16, 4096, 256, need - 256, None) == 6
    # unsupported activation dtype
    assert L.pe_linear_forward(16, 2, 1, 128, 128, 16, 4, NIB, 16, 16, None, 16, None, 16, 8,
                               None, 0, None) == 5
