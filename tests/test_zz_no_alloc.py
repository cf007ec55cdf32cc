"""pe_linear_forward_noalloc (the allocation-free entry point, no reference
counterpart) against pe_linear_forward with its own workspace: bit-identical
results on every path that uses scratch, for two calls in a row with the
second on a smaller input; calls past the static maximum are refused."""

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import DEV, check_close, dev_tiled, linear_call, rand_layer, say, to_dev

pytestmark = pytest.mark.gpu


def _noalloc(x, codes, norms, ct, bits, fmt, n, bias=None):
    from polarengine_vllm import _lib
    L = _lib.lib()
    m, k = x.shape
    y = torch.empty(m, n, dtype=x.dtype, device=DEV)
    ct_host = np.ascontiguousarray(ct, dtype=np.float32)
    cd = to_dev(ct_host)
    rc = L.pe_linear_forward_noalloc(x.data_ptr(), _lib.act_dtype(x), m, k, k, codes.data_ptr(),
                                     bits, fmt, norms.data_ptr(), cd.data_ptr(),
                                     ct_host.ctypes.data, 1 << bits,
                                     None if bias is None else bias.data_ptr(), y.data_ptr(), n,
                                     _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    return rc, y


# (first M, second M, N, K, bits): the K-split decode (partial sums and
# completion counters in scratch, one and two m-tiles), the small-M and
# prefill matmuls (x_tf and K-split partials in scratch), the M = 1 path past
# the decode kernel (x_tf in scratch) and the fused M = 1 decode (no scratch)
CASES = [(16, 12, 12288, 4096, 4), (32, 20, 4096, 12288, 3), (200, 64, 4096, 4096, 5),
         (300, 130, 4096, 12288, 4), (1, 1, 4096, 53248, 4), (1, 1, 12288, 4096, 4)]


@pytest.mark.parametrize("m1,m2,n,k,bits", CASES)
def test_noalloc_matches_linear_forward(m1, m2, n, k, bits):
    from polarengine_vllm import _lib
    rng = np.random.default_rng(m1 + n + k)
    codes, norms, ct = rand_layer(rng, n, k, bits)
    dcodes, dnorms, nib = dev_tiled(codes, norms, bits)
    fmt = (_lib.PE_PACK_NIBBLE if nib else 0) | _lib.PE_LAYOUT_TILE16
    bias = to_dev(O.seeded_normal((n,), 0.1, 7))
    for call, m in enumerate((m1, m2)):
        assert _lib.lib().pe_linear_workspace_size(m, k, n, bits, fmt) <= 32 << 20
        say(f"noalloc call {call} m={m} n={n} k={k} q{bits}")
        x = to_dev(O.seeded_normal((m, k), 1.0, 800 + m))
        rc, y = _noalloc(x, dcodes, dnorms, ct, bits, fmt, n, bias)
        _lib.check(rc, "pe_linear_forward_noalloc")
        want = linear_call(x, dcodes, dnorms, ct, bits, fmt, n, bias)
        assert torch.equal(y, want), f"call {call}: differs from pe_linear_forward"
        if m <= 64:  # and the oracle (larger M: equality with the checked entry point)
            ref = O.linear_apply(x.cpu().numpy(), codes, norms, ct, k, bias.cpu().numpy())
            check_close(y.float().cpu().numpy(), ref.astype(np.float32), f"noalloc m={m}")


def test_noalloc_refuses_calls_past_its_scratch():
    from polarengine_vllm import _lib
    L = _lib.lib()
    say("noalloc limit")
    limit = L.pe_linear_noalloc_max_bytes()
    assert limit == 32 << 20
    m, n, k, bits = 4096, 4096, 12288, 4  # x_tf alone is 96 MiB
    assert L.pe_linear_workspace_size(m, k, n, bits, 3) > limit
    rng = np.random.default_rng(3)
    codes, norms, ct = rand_layer(rng, 256, 128, bits)  # never read: refused before launch
    dcodes, dnorms, _ = dev_tiled(codes, norms, bits)
    x = torch.zeros(m, k, dtype=torch.float16, device=DEV)
    y = torch.full((m, n), 7.0, dtype=torch.float16, device=DEV)
    cd = to_dev(ct)
    rc = L.pe_linear_forward_noalloc(x.data_ptr(), 0, m, k, k, dcodes.data_ptr(), bits, 3,
                                     dnorms.data_ptr(), cd.data_ptr(), None, 1 << bits, None,
                                     y.data_ptr(), n, _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    assert rc == _lib.PE_ERR_SCRATCH
    assert b"scratch" in L.pe_status_string(rc)
    assert bool((y == 7.0).all())  # nothing was launched
