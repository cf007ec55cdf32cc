"""GPU tests of the MoE call's first launch, which routes the tokens,
transforms x and buckets the pairs by expert (the last routing workgroup to
finish buckets them, signalled through the workspace's counter block):

* the routed entry (pe_moe_forward_routed, what apply() calls) and the
  ids-given entry (pe_moe_forward, apply() with a custom routing function)
  give bit-identical outputs on the same routing;
* slots with an id outside 0..E-1 are skipped, a token without one valid
  slot is exactly zero, a token routed twice to one expert adds both slots
  (oracle.moe_forward at the north-star tolerance);
* many routing workgroups (T = 2048: 512 of them), and the pair counts at
  the bucketing's limits (2048, 2049, 32768, 32776 pairs);
* the workspace's counter block is zero again after every call, and a
  second call on the same workspace repeats the first bit for bit."""

import numpy as np
import pytest
import torch

import polar_oracle as O
from gpu_helpers import DEV, check_close, say, to_dev

pytestmark = pytest.mark.gpu


def _layer(rng, e, hdim, inter, b13, b2, tile=True):
    from test_gpu_kernels import _moe_layer
    return _moe_layer(rng, e, hdim, inter, b13, b2, tile)


@pytest.mark.parametrize("tile", [True, False])
def test_routed_equals_given_ids(tile):
    say(f"moe routed vs given ids tile={tile}")
    rng = np.random.default_rng(901)
    meth, layer, _ = _layer(rng, 16, 512, 384, 3, 4, tile)
    x = to_dev(O.seeded_normal((64, 512), 1.0, 902))
    logits = to_dev(O.seeded_normal((64, 16), 1.0, 903, np.float32))
    w, ids = meth.select_experts(logits, 4, True)

    def given(hidden_states, gating_output, topk, renormalize):
        return w, ids

    y_routed = meth.apply(layer, x, logits, 4, True)
    y_given = meth.apply(layer, x, logits, 4, True, custom_routing_function=given)
    torch.cuda.synchronize()
    assert torch.equal(y_routed, y_given)


# w2 chunks of 256 (nibbles) and 128 (int8) columns; t = 800: 2400 pairs, bucketed
# by a launch of its own (above 2048 pairs)
@pytest.mark.parametrize("b2,t", [(4, 12), (6, 12), (4, 800)])
def test_invalid_and_duplicate_slots(b2, t):
    say(f"moe invalid/duplicate slots q{b2} t={t}")
    rng = np.random.default_rng(910 + b2 + t)
    e, hdim, inter, k = 8, 384, 256, 3
    meth, layer, (w13, w2) = _layer(rng, e, hdim, inter, 3, b2)
    x = O.seeded_normal((t, hdim), 1.0, 911)
    ids = rng.integers(0, e, (t, k)).astype(np.int32)
    ids[1, 2] = -1          # one slot without an expert
    ids[2, :] = -1          # no valid slot: a zero row
    ids[3, 0] = e           # an id past the experts
    ids[4, :] = [5, 5, 2]   # twice to one expert
    wts = (np.abs(O.seeded_normal((t, k), 1.0, 912, np.float32)) + 0.1).astype(np.float32)

    def given(hidden_states, gating_output, topk, renormalize):
        return to_dev(wts), to_dev(ids)

    logits = to_dev(np.zeros((t, e), np.float32))
    y = meth.apply(layer, to_dev(x), logits, k, True, custom_routing_function=given)
    want = O.moe_forward(x, wts, ids, w13, w2).astype(np.float32)
    got = y.float().cpu().numpy()
    assert np.all(got[2] == 0.0)
    check_close(got, want, f"moe slots q{b2}")


@pytest.mark.parametrize("tile", [True, False])
def test_grouped_gemm_route_empty_and_invalid(tile):
    """The prefill regime (>= 128 rows per expert on average: the grouped
    four-wave kernel) with most experts empty, one expert taking a single
    row, invalid slots and a token twice on one expert."""
    say(f"moe grouped route, empty experts tile={tile}")
    rng = np.random.default_rng(980)
    e, hdim, inter, t, k = 8, 256, 256, 1100, 2
    meth, layer, (w13, w2) = _layer(rng, e, hdim, inter, 3, 4, tile)
    x = O.seeded_normal((t, hdim), 1.0, 981)
    ids = np.tile(np.array([[1, 6]], np.int32), (t, 1))
    ids[0] = [3, 6]        # expert 3: one row
    ids[5] = [6, 6]        # twice to one expert
    ids[7, 1] = -1         # a slot without an expert
    ids[9, 0] = e          # an id past the experts
    wts = (np.abs(O.seeded_normal((t, k), 1.0, 982, np.float32)) + 0.1).astype(np.float32)

    def given(hidden_states, gating_output, topk, renormalize):
        return to_dev(wts), to_dev(ids)

    logits = to_dev(np.zeros((t, e), np.float32))
    y = meth.apply(layer, to_dev(x), logits, k, True, custom_routing_function=given)
    want = O.moe_forward(x, wts, ids, w13, w2).astype(np.float32)
    check_close(y.float().cpu().numpy(), want, "moe grouped route")
    y2 = meth.apply(layer, to_dev(x), logits, k, True, custom_routing_function=given)
    assert torch.equal(y, y2), "grouped route not deterministic"


@pytest.mark.parametrize("tile", [False, True])
def test_grouped_gemm_route_partial_tiles(tile):
    """The prefill regime with expert row counts on every side of the
    kernel's 32- and 64-row steps (a tile computes only the 32-row m-tiles
    that hold rows): 1, 32, 33, 64, 65 rows, and experts whose last tile
    holds 1, 20 or 40 rows after full ones."""
    say(f"moe grouped route, partial tiles tile={tile}")
    rng = np.random.default_rng(990)
    e, hdim, inter, t, k = 8, 256, 256, 600, 2
    meth, layer, (w13, w2) = _layer(rng, e, hdim, inter, 3, 4, tile)
    x = O.seeded_normal((t, hdim), 1.0, 991)
    first = np.concatenate([np.full(n, ex, np.int32) for ex, n in
                            ((0, 1), (1, 32), (2, 33), (3, 64), (4, 65), (5, 168), (6, 129))])
    first = np.concatenate([first, np.full(t - first.size, 5, np.int32)])  # expert 5: 276 rows
    ids = np.stack([rng.permutation(first), np.full(t, 7, np.int32)], axis=1).astype(np.int32)
    counts = np.bincount(ids.ravel(), minlength=e)
    assert list(counts) == [1, 32, 33, 64, 65, 276, 129, 600]
    wts = (np.abs(O.seeded_normal((t, k), 1.0, 992, np.float32)) + 0.1).astype(np.float32)

    def given(hidden_states, gating_output, topk, renormalize):
        return to_dev(wts), to_dev(ids)

    logits = to_dev(np.zeros((t, e), np.float32))
    y = meth.apply(layer, to_dev(x), logits, k, True, custom_routing_function=given)
    want = O.moe_forward(x, wts, ids, w13, w2).astype(np.float32)
    check_close(y.float().cpu().numpy(), want, "moe grouped route, partial tiles")


# (token, slot) pairs at the bucketing's limits: 2048 (bucketed by the routing
# launch's last workgroup, ids held in registers), 2049 (moe_bucket_kernel),
# 32768 (that kernel's largest), 32776 (the routing launch again, in batches)
@pytest.mark.parametrize("t,k", [(512, 4), (683, 3), (4096, 8), (4097, 8)])
def test_bucketing_at_pair_count_limits(t, k):
    """Against the oracle, and bit for bit against the same call without
    its last token: with 8 experts both stay on the grouped kernel (at least
    128 rows per expert), every stage after the bucketing works per pair row
    or per token, so a token's output cannot depend on which bucketing form
    ordered the rows (the prefixes of 2049 and 32776 pairs, 2046 and 32768,
    are bucketed by the other form)."""
    say(f"moe bucketing limits t={t} k={k} pairs={t * k}")
    rng = np.random.default_rng(950 + t)
    e, hdim, inter = 8, 256, 256
    meth, layer, (w13, w2) = _layer(rng, e, hdim, inter, 3, 4)
    x = O.seeded_normal((t, hdim), 1.0, 951)
    ids = rng.integers(0, e, (t, k)).astype(np.int32)
    wts = (np.abs(O.seeded_normal((t, k), 1.0, 952, np.float32)) + 0.1).astype(np.float32)

    def run(n):
        def given(hidden_states, gating_output, topk, renormalize):
            return to_dev(wts[:n]), to_dev(ids[:n])
        logits = to_dev(np.zeros((n, e), np.float32))
        return meth.apply(layer, to_dev(x[:n]), logits, k, True, custom_routing_function=given)

    y = run(t)
    want = O.moe_forward(x, wts, ids, w13, w2).astype(np.float32)
    check_close(y.float().cpu().numpy(), want, f"moe pairs={t * k}")
    y_prefix = run(t - 1)
    torch.cuda.synchronize()
    assert torch.equal(y[:-1], y_prefix), f"pairs={t * k}: rows depend on the bucketing form"


def test_many_routing_workgroups():
    say("moe T=2048 e=32 k=4")
    rng = np.random.default_rng(920)
    meth, layer, (w13, w2) = _layer(rng, 32, 256, 128, 3, 4)
    x = O.seeded_normal((2048, 256), 1.0, 921)
    logits = O.seeded_normal((2048, 32), 1.0, 922, np.float32)
    y = meth.apply(layer, to_dev(x), to_dev(logits), 4, True)
    w_ref, ids_ref = O.moe_route(logits, 4, True)
    want = O.moe_forward(x, w_ref, ids_ref, w13, w2).astype(np.float32)
    check_close(y.float().cpu().numpy(), want, "moe T=2048")


def test_counter_block_left_zero():
    say("moe counter block after calls")
    from polarengine_vllm import _lib
    from polarengine_vllm.moe_method import _layout
    L = _lib.lib()
    rng = np.random.default_rng(930)
    meth, layer, _ = _layer(rng, 16, 512, 384, 3, 4)
    t, e, h, i, k = 96, 16, 512, 384, 4
    x = to_dev(O.seeded_normal((t, h), 1.0, 931)).half()
    lg = to_dev(O.seeded_normal((t, e), 1.0, 932, np.float32))
    wsb = L.pe_moe_workspace_size(t, k, e, h, i)
    ws = torch.zeros(wsb, dtype=torch.uint8, device=DEV)
    outs = []
    for _ in range(2):
        out = torch.empty_like(x)
        rc = L.pe_moe_forward_routed(
            x.data_ptr(), _lib.PE_DTYPE_F16, t, h, i, e, k, lg.data_ptr(), 1, 0, None, 0, 0,
            layer.w13_codes.data_ptr(), 3, _layout(layer.w13_packed, layer.w13_tiled),
            layer.w13_norms.data_ptr(), layer.w13_ct_scaled.data_ptr(), 8,
            layer.w2_codes.data_ptr(), 4, _layout(layer.w2_packed, layer.w2_tiled),
            layer.w2_norms.data_ptr(), layer.w2_ct_scaled.data_ptr(), 16,
            out.data_ptr(), ws.data_ptr(), wsb, _lib.stream_ptr(torch.device(DEV)))
        torch.cuda.synchronize()
        _lib.check(rc, "pe_moe_forward_routed")
        assert int(ws[:4096].count_nonzero()) == 0
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    assert L.pe_moe_forward_routed(
        x.data_ptr(), _lib.PE_DTYPE_F16, t, h, i, e, k, lg.data_ptr(), 1, 0, None, 0, 0,
        layer.w13_codes.data_ptr(), 3, _layout(layer.w13_packed, layer.w13_tiled),
        layer.w13_norms.data_ptr(), layer.w13_ct_scaled.data_ptr(), 8,
        layer.w2_codes.data_ptr(), 4, _layout(layer.w2_packed, layer.w2_tiled),
        layer.w2_norms.data_ptr(), layer.w2_ct_scaled.data_ptr(), 16,
        outs[0].data_ptr(), ws.data_ptr(), wsb - 256,
        _lib.stream_ptr(torch.device(DEV))) == _lib.PE_ERR_WORKSPACE


def test_graph_replay_matches_eager():
    """The MoE call at the C5 shapes (64 experts, I = 1408, top-8), captured
    in a HIP graph and replayed with eager work in between: every replay
    equals the eager call bit for bit (the routing counter block is reset by
    each call, the bench replays this graph)."""
    say("moe graph replay")
    rng = np.random.default_rng(940)
    meth, layer, _ = _layer(rng, 64, 2048, 1408, 3, 4)
    x = to_dev(O.seeded_normal((128, 2048), 1.0, 941))
    logits = to_dev(O.seeded_normal((128, 64), 1.0, 942, np.float32))
    want = meth.apply(layer, x, logits, 8, True)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        meth.apply(layer, x, logits, 8, True)  # workspace at full size before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        y = meth.apply(layer, x, logits, 8, True)
    for rep in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {rep} differs"
        junk = torch.randn(1 << 20, device=DEV).sum()  # eager work between replays
        torch.cuda.synchronize()
        del junk
