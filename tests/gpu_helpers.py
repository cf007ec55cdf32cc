"""Shared helpers of the GPU parity tests: device copies, the runtime weight
layouts, one C-ABI linear call, and the north-star comparison.

Tolerance: 16-bit outputs within normwise
||y - y_ref||_inf / ||y_ref||_inf <= 1e-2 and cosine >= 0.9999 of the fp32
oracle."""

import sys

import numpy as np
import torch

import polar_oracle as O

DEV = "cuda:0"
NORMWISE_TOL = 1e-2
COS_TOL = 0.9999


def say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def check_close(got, want, what, tol=NORMWISE_TOL, cos_tol=COS_TOL):
    g = np.asarray(got, dtype=np.float64).reshape(-1)
    w = np.asarray(want, dtype=np.float64).reshape(-1)
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    err = np.abs(g - w).max() / max(np.abs(w).max(), 1e-30)
    cos = float(g @ w / (np.linalg.norm(g) * np.linalg.norm(w) + 1e-300))
    assert err <= tol, f"{what}: normwise err {err:.3e}"
    assert cos >= cos_tol, f"{what}: cosine {cos:.7f}"
    return err, cos


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    return t if dtype is None else t.to(dtype)


def rand_layer(rng, n, kp, bits):
    codes = rng.integers(0, 1 << bits, (n, kp), dtype=np.int64).astype(np.uint8).view(np.int8)
    norms = (np.abs(rng.standard_normal((n, kp // 128))) * 0.2 + 0.05).astype(np.float16)
    return codes, norms, O.ct_scaled(bits)


def dev_codes(codes, bits):
    """Runtime layout: nibbles for bits <= 4, int8 otherwise."""
    if bits <= 4:
        return to_dev(O.pack_nibble(codes)), True
    return to_dev(codes), False


def dev_tiled(codes, norms, bits):
    from polarengine_vllm.packing import tile_weights_16
    dcodes, nib = dev_codes(codes, bits)
    ct, nt = tile_weights_16(dcodes, to_dev(norms))
    return ct, nt, nib


def pair_f16(x_tf):
    """[M, K] -> pair-f16 rows as uint32 [M, K/2]: (x[128b+p], x[128b+64+p])."""
    m, k = x_tf.shape
    h = np.ascontiguousarray(
        x_tf.astype(np.float16).reshape(m, k // 128, 2, 64).transpose(0, 1, 3, 2))
    return h.view(np.uint32).reshape(m, k // 2)


def bf16_dev(x_f32):
    """float32 array -> bf16 device tensor, and the float32 values it holds."""
    t = torch.from_numpy(np.ascontiguousarray(x_f32, dtype=np.float32)).to(torch.bfloat16)
    return t.to(DEV), t.float().numpy()


def linear_call(x, codes, norms, ct, bits, fmt, n, bias=None, ws_extra=0):
    """pe_linear_forward through the C ABI with a workspace of exactly the
    queried size (+ ws_extra); x is a [M, K] fp16 or bf16 device tensor, the
    result has x's dtype."""
    from polarengine_vllm import _lib
    L = _lib.lib()
    m, k = x.shape
    code = _lib.act_dtype(x)
    wsb = L.pe_linear_workspace_size(m, k, n, bits, fmt)
    ws = torch.zeros(wsb + ws_extra, dtype=torch.uint8, device=DEV) if wsb + ws_extra else None
    y = torch.empty(m, n, dtype=x.dtype, device=DEV)
    cd = ct if isinstance(ct, torch.Tensor) else to_dev(np.asarray(ct, dtype=np.float32))
    ct_host = np.ascontiguousarray(cd.cpu().numpy(), dtype=np.float32)
    rc = L.pe_linear_forward(x.data_ptr(), code, m, k, k, codes.data_ptr(), bits, fmt,
                             norms.data_ptr(), cd.data_ptr(), ct_host.ctypes.data, 1 << bits,
                             None if bias is None else bias.data_ptr(), y.data_ptr(), n,
                             None if ws is None else ws.data_ptr(), wsb + ws_extra,
                             _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    _lib.check(rc, "pe_linear_forward")
    return y


def stratified_rows(m, seed, tile=128, per_tile=1):
    """At least `per_tile` seeded rows from every `tile`-row m-tile, plus the
    first and last rows of the last (possibly partial) tile."""
    rng = np.random.default_rng(seed)
    rows = set()
    for t0 in range(0, m, tile):
        hi = min(m, t0 + tile)
        rows.update(int(r) for r in rng.choice(np.arange(t0, hi), min(per_tile, hi - t0),
                                               replace=False))
    last0 = (m - 1) // tile * tile
    rows.update({0, last0, m - 1})
    return np.array(sorted(rows))
