"""Benchmark of the PolarEngine quantized-linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Headline (BASELINE.json metric): the Q4 12288x4096 M=1 decode linear --
FWHT-128 of x fused into the nibble GEMV, fp16 in / fp16 out -- as HBM GB/s
(algorithmic bytes / time) and us/call. One "step" is one call. Weights
rotate over 16 independent copies (416 MB > the 256 MB Infinity Cache) so
reads come from HBM; calls are captured in a HIP graph and replayed so the
host does not gate the ~4 us kernels. Also measured: the same call with one
weight copy (cache-hot), the M=2048 prefill GEMM (TFLOP/s vs dense fp16 MFMA
peak), M=4/8/16 decode, the gate/up Q3 12288x4096 and down Q4 4096x12288 decode
shapes at M=1 and 16, the Q3 4096x12288 prefill, KV-cache quantize / dequantize,
the grouped MoE experts, and the oracle's CPU time for the headline call
(cpu_baseline, numpy, 1 thread) on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "polarengine-vllm_amd"))

from polarengine_vllm import _lib  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
N_COPIES = 16


def algo_bytes(m, n, k, bits):
    """codes + fp16 norms + fp16 x + fp16 y + fp32 codebook, each once."""
    s = 4 if bits <= 4 else 8
    return n * k * s // 8 + n * (k // 128) * 2 + m * k * 2 + m * n * 2 + (1 << bits) * 4


def make_layer(n, k, bits, dev, seed):
    """Random codes in the runtime layout, |N| norms and the real codebook
    (timing does not depend on code values)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    from polarengine_vllm.utils import get_centroids
    if bits <= 4:
        codes = torch.randint(0, 256 if bits == 4 else 1 << 8, (n, k // 2), generator=g,
                              dtype=torch.int32).to(torch.uint8)
        if bits < 4:
            m = ((1 << bits) - 1) * 0x11
            codes &= m
    else:
        codes = torch.randint(0, 1 << bits, (n, k), generator=g, dtype=torch.int32).to(torch.uint8)
    norms = (torch.randn(n, k // 128, generator=g).abs() * 0.2 + 0.05).half()
    ct = (get_centroids(bits) / np.sqrt(128.0)).float()
    return codes.to(dev), norms.to(dev), ct.to(dev)


class Linear:
    """Direct C-ABI call with preallocated buffers and the tiled-16 weight
    layout (what apply() launches)."""

    def __init__(self, n, k, bits, m, dev, seed, x=None):
        from polarengine_vllm.packing import tile_weights_16
        self.n, self.k, self.bits, self.m = n, k, bits, m
        codes, norms, self.ct = make_layer(n, k, bits, dev, seed)
        # the runtime layout process_weights_after_loading produces
        self.codes, self.norms = tile_weights_16(codes, norms)
        del codes, norms
        self.ct_host = np.ascontiguousarray(self.ct.cpu().numpy(), dtype=np.float32)
        self.packed = (_lib.PE_PACK_NIBBLE if bits <= 4 else 0) | _lib.PE_LAYOUT_TILE16
        self.x = x if x is not None else torch.randn(m, k, device=dev, dtype=torch.float16)
        self.y = torch.empty(m, n, device=dev, dtype=torch.float16)
        L = _lib.lib()
        self.wsb = L.pe_linear_workspace_size(m, k, n, bits, self.packed)
        self.ws = torch.zeros(max(self.wsb, 256), device=dev, dtype=torch.uint8)
        self.dev = dev

    def __call__(self):
        L = _lib.lib()
        rc = L.pe_linear_forward(self.x.data_ptr(), 0, self.m, self.k, self.k,
                                 self.codes.data_ptr(), self.bits, self.packed,
                                 self.norms.data_ptr(), self.ct.data_ptr(),
                                 self.ct_host.ctypes.data, 1 << self.bits, None,
                                 self.y.data_ptr(), self.n, self.ws.data_ptr(), self.wsb,
                                 _lib.stream_ptr(self.dev))
        if rc:
            _lib.check(rc, "pe_linear_forward")


def time_graph(calls, reps_per_graph, warmup, steps, dev):
    """Capture `reps_per_graph` rounds over `calls` in one graph; replay.
    Returns seconds per call."""
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for c in calls:  # eager warm-up (attribute setup, first launches)
            c()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(reps_per_graph):
            for c in calls:
                c()
    per_graph = reps_per_graph * len(calls)
    n_replays = max(1, steps // per_graph)
    for _ in range(max(1, warmup // per_graph)):
        g.replay()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n_replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize(dev)
    return e0.elapsed_time(e1) * 1e-3 / (n_replays * per_graph), n_replays * per_graph


def time_eager(fn, warmup, steps, dev):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize(dev)
    return e0.elapsed_time(e1) * 1e-3 / steps


def kv_extra(dev, n_vec=1 << 21, d=128, bits=3):
    """KV-cache compression of 2M vectors (256K tokens x 8 KV heads) of
    head_dim 128 at 3 bits: quantize (bf16 in; codes + bf16 norms out) and
    dequantize (back to bf16), as HBM GB/s of algorithmic bytes."""
    from polarengine_vllm.kv_cache import PolarKVQuantizer
    qz = PolarKVQuantizer(d, bits, str(dev))
    x = torch.randn(n_vec, d, device=dev, dtype=torch.bfloat16)
    packed, norms = qz.quantize(x)
    out = torch.empty_like(x)
    t_q = time_eager(lambda: qz.quantize(x), 3, 20, dev)
    t_d = time_eager(lambda: qz.dequantize(packed, norms, (n_vec, d), out=out), 3, 20, dev)
    b = n_vec * (d * 2 + d * bits // 8 + 2)  # bf16 vectors + codes + bf16 norms
    res = {}
    for name, t in (("kv_quantize", t_q), ("kv_dequantize", t_d)):
        res[name] = {"us_per_call": round(t * 1e6, 1), "GB/s": round(b / t / 1e9, 1),
                     "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4),
                     "vectors": n_vec, "head_dim": d, "bits": bits}
    return res


def moe_extra(dev, t=128, e=64, h=2048, inter=1408, k=8, b13=3, b2=4):
    """Grouped quantized experts (routing, SwiGLU w13, w2, weighted combine)
    through PolarQuantMoEMethod.apply: 64 experts, top-8, H=2048, I=1408,
    w13 Q3 and w2 Q4 nibbles, 128 tokens (1024 token-expert pairs). The
    stored expert bytes over the call time, as HBM GB/s."""
    from polarengine_vllm.moe_method import PolarQuantMoEMethod
    meth = PolarQuantMoEMethod(128, b13, b2)
    g = torch.Generator(device=dev).manual_seed(11)
    layers = []
    for _ in range(2):  # two weight copies in turn: 571 MB > the 256 MB Infinity Cache
        layer = torch.nn.Module()
        meth.create_weights(layer, e, h, inter, torch.float16)
        layer.to(dev)
        layer.w13_codes.copy_(torch.randint(0, 1 << b13, layer.w13_codes.shape, generator=g, device=dev))
        layer.w2_codes.copy_(torch.randint(0, 1 << b2, layer.w2_codes.shape, generator=g, device=dev))
        layer.w13_norms.copy_(torch.rand(layer.w13_norms.shape, generator=g, device=dev) * 0.3 + 0.05)
        layer.w2_norms.copy_(torch.rand(layer.w2_norms.shape, generator=g, device=dev) * 0.3 + 0.05)
        meth.process_weights_after_loading(layer)
        layers.append(layer)
    x = torch.randn(t, h, generator=g, device=dev).half()
    logits = torch.randn(t, e, generator=g, device=dev)
    wbytes = sum(b.numel() * b.element_size() for b in
                 (layers[0].w13_codes, layers[0].w13_norms, layers[0].w2_codes, layers[0].w2_norms))
    _, ids = meth.select_experts(logits, k, True)
    active = int(torch.unique(ids).numel())
    # replayed from a HIP graph, the two copies in turn, so the host does not
    # gate the ~60 us call
    calls = [lambda ly=ly: meth.apply(ly, x, logits, k, True) for ly in layers]
    tm, _ = time_graph(calls, 4, 16, 64, dev)
    return {"moe_t128_e64_top8": {"us_per_call": round(tm * 1e6, 1),
                                  "GB/s": round(wbytes * active / e / tm / 1e9, 1),
                                  "hbm_frac": round(wbytes * active / e / tm / 1e9 / HBM_PEAK_GBS, 4),
                                  "expert_bytes": wbytes, "active_experts": active,
                                  "includes": "routing + x FWHT with expert bucketing + w13 SwiGLU (FWHT of h fused) + w2 + combine"}}


def cpu_baseline(budget_s=15.0):
    """Oracle per-call path of the headline config on the host, 1 thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import polar_oracle as O
    try:
        from threadpoolctl import threadpool_limits
        limiter = threadpool_limits(limits=1)
    except Exception:
        limiter = None
    n, k, bits = 12288, 4096, 4
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (n, k)).astype(np.int8)
    norms = (np.abs(rng.standard_normal((n, k // 128))) * 0.2 + 0.05).astype(np.float16)
    ct = O.ct_scaled(bits)
    x = O.seeded_normal((1, k), 1.0, 1)
    O.linear_apply(x, codes, norms, ct, k)  # warm-up
    t0 = time.perf_counter()
    calls = 0
    while time.perf_counter() - t0 < budget_s:
        O.linear_apply(x, codes, norms, ct, k)
        calls += 1
    dt = (time.perf_counter() - t0) / calls
    if limiter is not None:
        limiter.unregister()
    return {"value": round(algo_bytes(1, n, k, bits) / dt / 1e9, 4), "unit": "GB/s",
            "us_per_call": round(dt * 1e6, 1), "cores": 1, "kind": "port",
            "sample": f"oracle linear_apply (numpy fp32: FWHT, Hadamard-domain GEMV, fp16 cast) "
                      f"Q4 {n}x{k} M=1, {calls} calls in {budget_s:.0f} s"}


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic_gemv_q4_12288x4096_m1.json")
COPY_BYTES = 256 << 20


def profile_traffic(dev):
    """Workload for the two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE):
    the headline call over the rotating copies, then a plain device copy of
    COPY_BYTES whose counter reading calibrates the KiB units."""
    n, k, bits, m = 12288, 4096, 4, 1
    x = torch.randn(m, k, device=dev, dtype=torch.float16)
    layers = [Linear(n, k, bits, m, dev, seed=100 + i, x=x) for i in range(N_COPIES)]
    for _ in range(4):
        for c in layers:
            c()
    # plain copy kernel of known traffic: reads and writes COPY_BYTES once
    src = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.neg(src, out=dst)
    torch.cuda.synchronize(dev)


def summarize_pmc(fetch_csv, write_csv):
    """HBM bytes per launch of the headline kernel from the two pmc passes,
    each counter scaled by (known copy bytes / the copy kernel's reading)."""
    import csv

    def per_kernel(path, counter):
        vals = {}
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] != counter:
                continue
            vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return vals

    out = {}
    for path, counter in ((fetch_csv, "FETCH_SIZE"), (write_csv, "WRITE_SIZE")):
        v = per_kernel(path, counter)
        gemv = [k for k in v if "gemv_mfma_kernel" in k or "gemv1_kernel" in k]
        copy = [k for k in v if "neg_kernel" in k]
        if not gemv or not copy:
            raise SystemExit(f"{path}: kernels not found: {list(v)[:6]}")
        kg, kc = gemv[0], copy[0]
        scale = COPY_BYTES / (np.median(v[kc]) * 1024.0)
        out[counter] = {"kernel": kg, "kib_per_launch": float(np.median(v[kg])),
                        "copy_kernel": kc, "copy_kib": float(np.median(v[kc])),
                        "scale": float(scale),
                        "bytes_per_launch": float(np.median(v[kg]) * 1024.0 * scale)}
    out["traffic_bytes"] = out["FETCH_SIZE"]["bytes_per_launch"] + out["WRITE_SIZE"]["bytes_per_launch"]
    return out


def prefill_extra(dev):
    """Prefill linear at M=2048 (FWHT-128 of x into pair f16, then the MFMA
    GEMM): Q4 12288x4096 and the Q3 4096x12288 down projection; and the Q4
    down projection at M=128 / 512 (K split over workgroups)."""
    out = {}
    flops = 2.0 * 2048 * 12288 * 4096
    for name, (nn, kk, bb, seed) in (("prefill_m2048", (12288, 4096, 4, 300)),
                                     ("prefill_down_q3_m2048", (4096, 12288, 3, 301))):
        pf = Linear(nn, kk, bb, 2048, dev, seed=seed)
        t_pf = time_eager(pf, 3, 20, dev)
        out[name] = {"us_per_call": round(t_pf * 1e6, 1),
                     "TFLOP/s": round(flops / t_pf / 1e12, 1),
                     "mfma_frac": round(flops / t_pf / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                     "includes": "FWHT-128 of x (pair f16) + MFMA GEMM"}
        del pf
    # chunked-prefill sizes on the down projection (few output tiles: K split)
    for mm in (128, 512):
        lay = [Linear(4096, 12288, 4, mm, dev, seed=310 + i) for i in range(4)]
        t, _ = time_graph(lay, 4, 32, 256, dev)
        fl = 2.0 * mm * 4096 * 12288
        out[f"prefill_down_q4_m{mm}"] = {"us_per_call": round(t * 1e6, 1),
                                         "TFLOP/s": round(fl / t / 1e12, 1),
                                         "GB/s": round(algo_bytes(mm, 4096, 12288, 4) / t / 1e9, 1)}
        del lay
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--profile-traffic", action="store_true",
                    help="run only the workload of the FETCH_SIZE / WRITE_SIZE pmc passes")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the headline call (for a rocprofv3 kernel trace whose "
                         "average covers exactly the headline dispatches)")
    ap.add_argument("--only-extra", choices=("moe", "prefill", "kv"),
                    help="time only one of the extra workloads and print its JSON (for a "
                         "rocprofv3 kernel trace of that path alone)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the traffic JSON from the two pmc passes and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc), indent=1))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build's hot path is a single-GPU kernel "
              "(multi-GPU sharding is design-only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.lib()
    if args.profile_traffic:
        profile_traffic(dev)
        return
    if args.only_extra:
        fn = {"moe": moe_extra, "prefill": prefill_extra, "kv": kv_extra}[args.only_extra]
        print(json.dumps(fn(dev)))
        return

    n, k, bits, m = 12288, 4096, 4, 1
    x = torch.randn(m, k, device=dev, dtype=torch.float16)
    layers = [Linear(n, k, bits, m, dev, seed=100 + i, x=x) for i in range(N_COPIES)]
    t_call, calls_timed = time_graph(layers, 8, args.warmup, args.steps, dev)
    B = algo_bytes(m, n, k, bits)
    gbs = B / t_call / 1e9
    if args.headline_only:
        print(json.dumps({"workload": "headline only", "us_per_call": round(t_call * 1e6, 3),
                          "GB/s": round(gbs, 1), "calls_timed": calls_timed}))
        return
    t_hot, _ = time_graph(layers[:1], 128, args.warmup, args.steps, dev)

    extra = {}
    for mm in (4, 8, 16, 32, 64):
        lay = [Linear(n, k, bits, mm, dev, seed=200 + i) for i in range(N_COPIES)]
        t, _ = time_graph(lay, 4, 64, 512, dev)
        extra[f"decode_m{mm}"] = {"us_per_call": round(t * 1e6, 2),
                                  "GB/s": round(algo_bytes(mm, n, k, bits) / t / 1e9, 1)}
        del lay
    # the MLP's other shapes: gate/up Q3 12288x4096 and down Q4 4096x12288
    for name, (nn, kk, bb) in (("gateup_q3", (12288, 4096, 3)), ("down_q4", (4096, 12288, 4))):
        for mm in (1, 16):
            lay = [Linear(nn, kk, bb, mm, dev, seed=400 + i) for i in range(N_COPIES)]
            t, _ = time_graph(lay, 4, 64, 512, dev)
            gb = algo_bytes(mm, nn, kk, bb) / t / 1e9
            extra[f"decode_{name}_m{mm}"] = {"us_per_call": round(t * 1e6, 2), "GB/s": round(gb, 1),
                                             "hbm_frac": round(gb / HBM_PEAK_GBS, 4)}
            del lay
    extra.update(prefill_extra(dev))
    extra["cache_hot_m1"] = {"us_per_call": round(t_hot * 1e6, 2),
                             "GB/s": round(B / t_hot / 1e9, 1),
                             "note": "one weight copy, Infinity-Cache resident"}
    extra.update(kv_extra(dev))
    extra.update(moe_extra(dev))

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    traffic = None  # HBM bytes per launch from the committed pmc summary, if any
    if os.path.exists(TRAFFIC_JSON):
        with open(TRAFFIC_JSON) as f:
            traffic = round(json.load(f)["traffic_bytes"])
    out = {
        "metric": "HBM GB/s + us/call, Q4 GEMV 12288x4096 M=1; prefill GEMM TFLOPS M=2048",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": calls_timed,
        "warmup": args.warmup,
        "ms_per_step": round(t_call * 1e3, 6),
        "us_per_call": round(t_call * 1e6, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: random nibble codes, |N| fp16 norms, Lloyd-Max Q4 codebook, "
                "x ~ N(0,1) fp16; f16 MFMA operands, fp32 accumulate",
        "config": {"workload": "decode linear Q4 12288x4096 M=1 (FWHT fused + nibble GEMV), "
                               f"{N_COPIES} rotating weight copies",
                   "M": m, "N": n, "K": k, "bits": bits, "algorithmic_bytes": B},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
