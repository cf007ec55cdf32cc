"""Code packing formats of PolarEngine checkpoints (reference: packing.py).

* half-block nibbles (bits <= 4): ``byte[i] = code[bs/2 + i] << 4 | code[i]``
  per block -- the on-disk and runtime layout (packing.py:22-94);
* Q5 LSB-first, 8 codes in 5 bytes (packing.py:97-209) -- on disk only,
  unpacked to int8 at load (loader.py:412-417);
* HLWQ ``bitpack_5``, MSB-first (packing.py:212-290).

Device (GPU) tensors are packed/unpacked by the HIP kernels
``pe_pack_nibble`` / ``pe_unpack_q5`` / ``pe_unpack_q5_hlwq`` (bit-exact);
CPU tensors, which only appear in offline checkpoint tooling, use the torch
expressions below.
"""

from __future__ import annotations

from typing import Any

import torch


def _on_gpu(t: torch.Tensor) -> bool:
    return t.device.type == "cuda"


def pack_codes_half_block(codes: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """int8 codes [..., K] in [0, 15] -> uint8 [..., K/2] (half-block order)."""
    assert block_size % 2 == 0, f"block_size must be even, got {block_size}"
    *lead, k = codes.shape
    assert k % block_size == 0, f"in_f_padded ({k}) must be a multiple of block_size ({block_size})"
    u8 = codes.to(torch.uint8)
    assert bool((u8 <= 15).all()), (
        "All code values must be in [0, 15] for INT4 nibble packing. "
        f"Found max={int(u8.max())}")
    if _on_gpu(codes) and block_size == 128:
        from polarengine_vllm import _lib
        src = codes.contiguous()
        if src.dtype != torch.int8:
            src = src.to(torch.int8)
        rows = src.numel() // k if k else 0
        out = torch.empty(*lead, k // 2, dtype=torch.uint8, device=codes.device)
        _lib.check(_lib.lib().pe_pack_nibble(src.data_ptr(), out.data_ptr(), rows, k,
                                             _lib.stream_ptr(codes.device)), "pe_pack_nibble")
        return out
    half = block_size // 2
    b = u8.reshape(*lead, k // block_size, block_size)
    return ((b[..., half:] << 4) | b[..., :half]).reshape(*lead, k // 2)


def tile_weights_16(codes: torch.Tensor, norms: torch.Tensor):
    """Runtime tiled-16 layout of one matrix (``pe_tile_weights``, GPU only):
    codes [N, row_bytes] -> [ceil(N/16)*16, row_bytes] holding
    [tiles][nb][16][bpb], norms [N, nb] -> [ceil(N/16)*16, nb] holding
    [tiles][nb][16]; padded rows are zero. The shapes keep two dims so the
    buffers still read as rows x bytes."""
    from polarengine_vllm import _lib
    dev = _lib.require_device(codes, norms)
    n, row_bytes = codes.shape
    nb = norms.shape[1]
    npad = (n + 15) // 16 * 16
    src = codes.contiguous()
    nsrc = norms.to(torch.float16).contiguous()
    codes_t = torch.empty(npad, row_bytes, dtype=codes.dtype, device=dev)
    norms_t = torch.empty(npad, nb, dtype=torch.float16, device=dev)
    _lib.check(_lib.lib().pe_tile_weights(src.data_ptr(), nsrc.data_ptr(), n, row_bytes, nb,
                                          codes_t.data_ptr(), norms_t.data_ptr(),
                                          _lib.stream_ptr(dev)), "pe_tile_weights")
    return codes_t, norms_t


def unpack_codes_half_block(packed: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """uint8 [..., K/2] -> int8 codes [..., K]."""
    assert block_size % 2 == 0, f"block_size must be even, got {block_size}"
    half = block_size // 2
    *lead, kh = packed.shape
    assert kh % half == 0, f"Packed dim ({kh}) must be a multiple of half_bk ({half})"
    b = packed.reshape(*lead, kh // half, half)
    lo = b & 0x0F
    hi = (b >> 4) & 0x0F
    return torch.cat([lo, hi], dim=-1).reshape(*lead, kh * 2).to(torch.int8)


def pack_codes_q5(codes: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """int8 codes [..., K] in [0, 31] -> uint8 [..., 5K/8], LSB-first."""
    assert block_size % 8 == 0, f"block_size must be a multiple of 8, got {block_size}"
    *lead, k = codes.shape
    assert k % block_size == 0, f"Last dimension ({k}) must be a multiple of block_size ({block_size})"
    c = codes.to(torch.long) & 0xFF
    assert bool((c <= 31).all()), (
        "All code values must be in [0, 31] for Q5 packing. "
        f"Found max={int(c.max())}")
    g = c.reshape(*lead, k // 8, 8)
    c0, c1, c2, c3, c4, c5, c6, c7 = g.unbind(-1)
    out = torch.stack([
        c0 | (c1 << 5),
        (c1 >> 3) | (c2 << 2) | (c3 << 7),
        (c3 >> 1) | (c4 << 4),
        (c4 >> 4) | (c5 << 1) | (c6 << 6),
        (c6 >> 2) | (c7 << 3),
    ], dim=-1) & 0xFF
    return out.to(torch.uint8).reshape(*lead, k * 5 // 8)


def unpack_codes_q5(packed: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """Inverse of :func:`pack_codes_q5` -> int8 codes in [0, 31]."""
    assert block_size % 8 == 0, f"block_size must be a multiple of 8, got {block_size}"
    *lead, kp = packed.shape
    assert (kp * 8) % 5 == 0, f"Packed dimension ({kp}) is not valid for Q5 unpacking"
    assert kp % (block_size * 5 // 8) == 0, (
        f"Packed dimension ({kp}) must be a multiple of packed_block_bytes ({block_size * 5 // 8})")
    k = kp * 8 // 5
    if _on_gpu(packed) and block_size == 128:
        from polarengine_vllm import _lib
        src = packed.contiguous()
        rows = src.numel() // kp if kp else 0
        out = torch.empty(*lead, k, dtype=torch.int8, device=packed.device)
        _lib.check(_lib.lib().pe_unpack_q5(src.data_ptr(), out.data_ptr(), rows, k,
                                           _lib.stream_ptr(packed.device)), "pe_unpack_q5")
        return out
    p = packed.to(torch.long).reshape(*lead, kp // 5, 5)
    b0, b1, b2, b3, b4 = p.unbind(-1)
    out = torch.stack([
        b0,
        (b0 >> 5) | (b1 << 3),
        b1 >> 2,
        (b1 >> 7) | (b2 << 1),
        (b2 >> 4) | (b3 << 4),
        b3 >> 1,
        (b3 >> 6) | (b4 << 2),
        b4 >> 3,
    ], dim=-1) & 0x1F
    return out.to(torch.int8).reshape(*lead, k)


def unpack_codes_q5_hlwq(packed: torch.Tensor, total: int | None = None) -> torch.Tensor:
    """HLWQ ``bitpack_5`` (MSB-first) -> int8 codes, optionally truncated
    (reference: packing.py:229-271). GPU tensors: ``pe_unpack_q5_hlwq``."""
    *lead, kp = packed.shape
    assert kp % 5 == 0, f"HLWQ bit-packed codes require K_packed % 5 == 0, got {kp}"
    if _on_gpu(packed) and not lead:
        from polarengine_vllm import _lib
        src = packed.contiguous()
        n = kp * 8 // 5 if total is None else int(total)
        if n > kp * 8 // 5:
            raise ValueError(f"total={n} exceeds the {kp * 8 // 5} codes of the packed stream")
        out = torch.empty(n, dtype=torch.int8, device=packed.device)
        _lib.check(_lib.lib().pe_unpack_q5_hlwq(src.data_ptr(), kp, out.data_ptr(), n,
                                                _lib.stream_ptr(packed.device)),
                   "pe_unpack_q5_hlwq")
        return out
    p = packed.to(torch.long).reshape(*lead, kp // 5, 5)
    b0, b1, b2, b3, b4 = p.unbind(-1)
    out = torch.stack([
        (b0 >> 3) & 0x1F,
        ((b0 & 7) << 2) | ((b1 >> 6) & 3),
        (b1 >> 1) & 0x1F,
        ((b1 & 1) << 4) | ((b2 >> 4) & 0xF),
        ((b2 & 0xF) << 1) | ((b3 >> 7) & 1),
        (b3 >> 2) & 0x1F,
        ((b3 & 3) << 3) | ((b4 >> 5) & 7),
        b4 & 0x1F,
    ], dim=-1).to(torch.int8).reshape(*lead, kp * 8 // 5)
    return out if total is None else out[..., :total]


def pack_codes_q5_hlwq(codes: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`unpack_codes_q5_hlwq`; zero-pads K to a multiple of 8."""
    *lead, k = codes.shape
    pad = (8 - k % 8) % 8
    if pad:
        codes = torch.cat([codes, torch.zeros(*lead, pad, dtype=codes.dtype, device=codes.device)], -1)
        k += pad
    c = codes.to(torch.long).reshape(*lead, k // 8, 8)
    c0, c1, c2, c3, c4, c5, c6, c7 = c.unbind(-1)
    out = torch.stack([
        (c0 << 3) | (c1 >> 2),
        ((c1 & 3) << 6) | (c2 << 1) | (c3 >> 4),
        ((c3 & 0xF) << 4) | (c4 >> 1),
        ((c4 & 1) << 7) | (c5 << 2) | (c6 >> 3),
        ((c6 & 7) << 5) | c7,
    ], dim=-1) & 0xFF
    return out.to(torch.uint8).reshape(*lead, -1)


def pack_model_codes(model: Any, block_size: int = 128) -> dict:
    """Nibble-pack the ``codes`` buffer of every module with ``bits <= 4``.

    Replaces the buffer by ``codes_packed`` and marks ``_codes_packed``
    (reference: packing.py:293-364). Returns the VRAM accounting dict.
    """
    n, before, after = 0, 0, 0
    for _, module in model.named_modules():
        bits = getattr(module, "bits", None)
        if bits is None or bits > 4:
            continue
        codes = getattr(module, "codes", None)
        if codes is None:
            continue
        before += codes.numel() * codes.element_size()
        src = codes if codes.dtype in (torch.int8, torch.uint8) else codes.to(torch.int8)
        packed = pack_codes_half_block(src, block_size)
        after += packed.numel() * packed.element_size()
        if "codes" in getattr(module, "_buffers", {}):
            del module._buffers["codes"]
            module.register_buffer("codes_packed", packed)
        else:
            module.codes = packed
            module.codes_packed = packed
        module._codes_packed = True
        n += 1
    return {"layers_packed": n, "vram_before": before, "vram_after": after,
            "saved_gb": (before - after) / (1024 ** 3)}


def verify_packing_roundtrip(codes: torch.Tensor, block_size: int = 128) -> bool:
    packed = pack_codes_half_block(codes, block_size)
    return torch.equal(codes.to(torch.uint8), unpack_codes_half_block(packed, block_size).to(torch.uint8))


def verify_packing_roundtrip_q5(codes: torch.Tensor, block_size: int = 128) -> bool:
    packed = pack_codes_q5(codes, block_size)
    return torch.equal(codes.to(torch.uint8), unpack_codes_q5(packed, block_size).to(torch.uint8))
