"""Benchmark of the PolarEngine quantized-linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--repeats R]

Headline (BASELINE.json metric): the Q4 12288x4096 M=1 decode linear --
FWHT-128 of x fused into the nibble GEMV, fp16 in / fp16 out -- as HBM GB/s
(algorithmic bytes / time) and us/call. One "step" is one call. Weights
rotate over 16 independent copies (416 MB > the 256 MB Infinity Cache) so
reads come from HBM. W untimed calls first; then R samples, each exactly K
calls captured in one HIP graph and replayed between two synchronizes, HIP
events on the replay stream; the line reports the median sample. Also
measured (under "extra"): the same call with one weight copy (cache-hot),
batched decode on the headline and MLP shapes, C1 (Q5 4096x4096 M=1), the
prefill GEMMs (TFLOP/s vs dense fp16 MFMA peak), the C4 decoder layer's
linears at M=1 and M=512, KV-cache quantize / dequantize, the grouped MoE
experts; and the oracle's CPU time on the host's cores (cpu_baseline).
"""

from __future__ import annotations

import argparse
import json
import math
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


def time_steps(calls, steps, warmup, dev, repeats=1, steady=False, settle_s=0.0):
    """Exactly `steps` calls per timed sample (cycling through `calls`),
    captured in one HIP graph and replayed on the current stream; `warmup`
    untimed eager calls (at least one per call object) and one untimed replay
    first. Each sample is bracketed by synchronize, with HIP events on the
    replay stream. Cold samples: synchronize, start event, replay, end event
    (the replay's launch latency falls inside the sample). Steady samples
    (steady=True): synchronize, an untimed replay, start event, the timed
    replay, end event -- the timed replay is queued while the untimed one
    runs, as in a serving loop, so the sample holds the calls alone; it still
    holds exactly `steps` calls. settle_s > 0 (the extras, not the headline):
    before the samples, untimed replays worth about that much GPU time, so
    that the clock has settled under the load. Returns (median seconds per
    call, per-sample list)."""
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        for i in range(max(warmup, len(calls))):
            calls[i % len(calls)]()
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize(dev)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for i in range(steps):
            calls[i % len(calls)]()
    t_first = time.perf_counter()
    g.replay()
    torch.cuda.synchronize(dev)
    if settle_s > 0:
        per_replay = max(time.perf_counter() - t_first, 1e-6)
        for _ in range(int(math.ceil(settle_s / per_replay))):
            g.replay()
        torch.cuda.synchronize(dev)
    samples = []
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(repeats):
        torch.cuda.synchronize(dev)
        if steady:
            g.replay()
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize(dev)
        samples.append(e0.elapsed_time(e1) * 1e-3 / steps)
    return float(np.median(samples)), samples


def time_graph(calls, reps_per_graph, warmup, steps, dev):
    """Extras: about `steps` calls per sample in whole rounds over `calls`,
    replayed until the clock has settled (about 80 ms of GPU time), then the
    median of five samples. Returns (seconds per call, calls per sample)."""
    n = max(len(calls), (steps // len(calls)) * len(calls))
    t, _ = time_steps(calls, n, warmup, dev, repeats=5, settle_s=0.08)
    return t, n


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
    t_q, _, _ = time_settled(lambda: qz.quantize(x), dev)
    t_d, _, _ = time_settled(lambda: qz.dequantize(packed, norms, (n_vec, d), out=out), dev)
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
    w13 Q3 and w2 Q4 nibbles, 128 tokens (1024 token-expert pairs; C5) or
    `t` tokens. The stored expert bytes over the call time, as HBM GB/s, and
    the expert FLOPs over the call time."""
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
    return {f"moe_t{t}_e{e}_top{k}": {"us_per_call": round(tm * 1e6, 1),
                                  "GB/s": round(wbytes * active / e / tm / 1e9, 1),
                                  "hbm_frac": round(wbytes * active / e / tm / 1e9 / HBM_PEAK_GBS, 4),
                                  "TFLOP/s": round(2.0 * t * k * 3 * h * inter / tm / 1e12, 1),
                                  "expert_bytes": wbytes, "active_experts": active,
                                  "includes": "routing + x FWHT with expert bucketing + w13 SwiGLU (FWHT of h fused) + w2 + combine"}}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_time(fn, budget_s, min_runs=20):
    """Median seconds per call over at least `min_runs` runs (or as many as
    fit in budget_s), after 3 warm-up calls."""
    for _ in range(3):
        fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= min_runs and time.perf_counter() >= t_end:
            break
        if len(times) >= 4 * min_runs:
            break
    return float(np.median(times)), len(times)


def cpu_baseline(budget_s=20.0):
    """The oracle (numpy restatement of the reference's CPU-capable path) on
    the host's affinity cores, two lines per config: (i) the reference
    per-call path (x.float() -> FWHT -> Hadamard-domain product -> .half()),
    (ii) dense dequantize-then-matmul with W materialised once (only x @ W.T
    timed); on the headline config (Q4 12288x4096 M=1) and C1 (Q5 4096x4096
    M=1). `value` is line (i) on the headline config."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import polar_oracle as O
    from threadpoolctl import threadpool_limits
    cores = len(os.sched_getaffinity(0))
    lines = {}
    with threadpool_limits(limits=cores):
        for name, (n, k, bits), share in (("headline_q4_12288x4096_m1", (12288, 4096, 4), 0.4),
                                          ("c1_q5_4096x4096_m1", (4096, 4096, 5), 0.3)):
            rng = np.random.default_rng(0)
            codes = rng.integers(0, 1 << bits, (n, k)).astype(np.int8)
            norms = (np.abs(rng.standard_normal((n, k // 128))) * 0.2 + 0.05).astype(np.float16)
            ct = O.ct_scaled(bits)
            x = O.seeded_normal((1, k), 1.0, 1)
            B = algo_bytes(1, n, k, bits)
            t1, r1 = _cpu_time(lambda: O.linear_apply(x, codes, norms, ct, k), budget_s * share)
            w = O.dequant_weight(codes, norms, ct)  # materialised once, not timed
            t2, r2 = _cpu_time(lambda: O.dequant_matmul(x, w), budget_s * share / 3)
            lines[name] = {
                "per_call_path": {"us_per_call": round(t1 * 1e6, 1),
                                  "GB/s": round(B / t1 / 1e9, 4), "runs": r1},
                "dense_dequant_matmul": {"us_per_call": round(t2 * 1e6, 1),
                                         "GB/s": round(B / t2 / 1e9, 4), "runs": r2},
            }
            del w
    head = lines["headline_q4_12288x4096_m1"]["per_call_path"]
    return {"value": head["GB/s"], "unit": "GB/s", "us_per_call": head["us_per_call"],
            "cores": cores, "cpu": _cpu_model(), "kind": "port",
            "sample": f"oracle on {cores} host threads (numpy/OpenBLAS, fp32): line (i) "
                      "linear_apply per call (FWHT, Hadamard-domain GEMV, fp16 cast) and line (ii) "
                      "x @ W.T with W dequantised once, median of >= 20 runs after 3 warm-ups, on "
                      "the headline config (Q4 12288x4096 M=1) and C1 (Q5 4096x4096 M=1); value = "
                      "line (i), headline",
            "lines": lines}


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
    GEMM): Q4 12288x4096 and the Q3 4096x12288 down projection; the same two
    at the other C3 sizes, M=256 (from HIP graphs over rotating weight
    copies) and M=8192; and the Q4 down projection at M=128 / 512 (K split
    over workgroups)."""
    out = {}
    for mm, reps in ((8192, 8),):
        for name, (nn, kk, bb, seed) in ((f"prefill_m{mm}", (12288, 4096, 4, 320)),
                                         (f"prefill_down_q3_m{mm}", (4096, 12288, 3, 321))):
            pf = Linear(nn, kk, bb, mm, dev, seed=seed)
            t_pf, _, _ = time_settled(pf, dev, steps=reps)
            fl = 2.0 * mm * nn * kk
            out[name] = {"us_per_call": round(t_pf * 1e6, 1),
                         "TFLOP/s": round(fl / t_pf / 1e12, 1),
                         "mfma_frac": round(fl / t_pf / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                         "includes": "FWHT-128 of x (pair f16) + MFMA GEMM"}
            del pf
    for name, (nn, kk, bb, seed) in (("prefill_m256", (12288, 4096, 4, 330)),
                                     ("prefill_down_q3_m256", (4096, 12288, 3, 331))):
        lay = [Linear(nn, kk, bb, 256, dev, seed=seed + 2 * i) for i in range(4)]
        t, _ = time_graph(lay, 4, 32, 256, dev)
        fl = 2.0 * 256 * nn * kk
        out[name] = {"us_per_call": round(t * 1e6, 1), "TFLOP/s": round(fl / t / 1e12, 1),
                     "mfma_frac": round(fl / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                     "GB/s": round(algo_bytes(256, nn, kk, bb) / t / 1e9, 1),
                     "includes": "FWHT-128 of x (pair f16) + MFMA GEMM (K split where the tiles are few)"}
        del lay
    out.update(prefill_m2048_extra(dev))
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


PREFILL_TRACE_JSON = os.path.join(ROOT, "profiles", "trace_gemm4_prefill_m2048.json")
PREFILL_PMC_JSON = os.path.join(ROOT, "profiles", "pmc_gemm4_prefill_m2048.json")


def _time_each(fn, calls, dev):
    """Per-call times of `calls` back-to-back calls (HIP events around each
    call, one synchronize at the end): the first calls run at full clock,
    later ones at the clock the card holds under sustained load."""
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(calls + 1)]
    torch.cuda.synchronize(dev)
    ev[0].record()
    for i in range(calls):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize(dev)
    return [ev[i].elapsed_time(ev[i + 1]) * 1e-3 for i in range(calls)]


def time_settled(fn, dev, steps=20, settle_s=0.08):
    """Back-to-back calls timed one by one after warm-up calls worth about
    settle_s of GPU time. Under a sustained MFMA load the card's clock dips
    for a few tens of milliseconds (the M=2048 GEMM goes from 214 to ~270 us
    per call around calls 10-20, and back to ~212 us after ~80 calls); the
    timed calls come after that. Returns (mean seconds per call, per-call
    seconds, warm-up calls)."""
    t0 = time_eager(fn, 1, 3, dev)
    n = int(math.ceil(settle_s / max(t0, 1e-6)))
    for _ in range(n):
        fn()
    ts = _time_each(fn, steps, dev)
    return float(np.mean(ts)), ts, n


def prefill_m2048_extra(dev, trace_only=False):
    """The metric's second half: the prefill linear at M=2048 (FWHT-128 of x
    into pair f16, then the MFMA GEMM) on Q4 12288x4096 and the Q3 4096x12288
    down projection. us_per_call: the mean of 20 back-to-back calls timed
    one by one once the clock has settled under the sustained load
    (time_settled); min_us / max_us: their spread. The dense fp16 GEMM of
    the same shape (torch.matmul: hipBLASLt) is timed the same way beside it.
    roofline: the GEMM kernel alone, its duration the larger of the committed
    rocprofv3 trace mean (same settled calls) and the event-timed call minus
    the traced FWHT (profiles/), 2*M*N*K flops over it against 2.5 PFLOP/s
    dense fp16; mfma_busy from the committed counter pass."""
    out = {}
    flops = 2.0 * 2048 * 12288 * 4096
    trace = pmc = None
    if os.path.exists(PREFILL_TRACE_JSON):
        with open(PREFILL_TRACE_JSON) as f:
            trace = json.load(f)
    if os.path.exists(PREFILL_PMC_JSON):
        with open(PREFILL_PMC_JSON) as f:
            pmc = json.load(f)
    for name, (nn, kk, bb, seed) in (("prefill_m2048", (12288, 4096, 4, 300)),
                                     ("prefill_down_q3_m2048", (4096, 12288, 3, 301))):
        pf = Linear(nn, kk, bb, 2048, dev, seed=seed)
        t_pf, ts, nwarm = time_settled(pf, dev)
        if trace_only:
            out[name] = {"us_per_call": round(t_pf * 1e6, 1), "warmup_calls": nwarm}
            del pf
            continue
        ent = {"us_per_call": round(t_pf * 1e6, 1),
               "TFLOP/s": round(flops / t_pf / 1e12, 1),
               "mfma_frac": round(flops / t_pf / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
               "min_us": round(min(ts) * 1e6, 1), "max_us": round(max(ts) * 1e6, 1),
               "warmup_calls": nwarm,
               "includes": "FWHT-128 of x (pair f16) + MFMA GEMM"}
        # dense fp16 reference of the same product (not this library)
        a = torch.randn(2048, kk, device=dev, dtype=torch.float16)
        b = torch.randn(nn, kk, device=dev, dtype=torch.float16)
        c = torch.empty(2048, nn, device=dev, dtype=torch.float16)
        dense = lambda: torch.matmul(a, b.t(), out=c)  # noqa: E731
        t_d, ts_d, _ = time_settled(dense, dev)
        ent["dense_fp16_reference"] = {"us_per_call": round(t_d * 1e6, 1),
                                       "min_us": round(min(ts_d) * 1e6, 1),
                                       "max_us": round(max(ts_d) * 1e6, 1),
                                       "what": "torch.matmul fp16 (hipBLASLt), same shape, "
                                               "timed the same way"}
        del a, b, c
        tr = (trace or {}).get(name)
        if tr:
            gemm_us = max(tr["gemm_avg_us"], t_pf * 1e6 - tr["fwht_avg_us"])
            ach = flops / (gemm_us * 1e-6) / 1e12
            ent["roofline"] = {"bound": "mfma", "kernel": tr["gemm_kernel"],
                               "kernel_us": round(gemm_us, 2),
                               "kernel_us_source": "trace mean" if gemm_us == tr["gemm_avg_us"]
                               else "HIP events minus traced FWHT",
                               "achieved": round(ach, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                               "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4),
                               "fwht_us": tr["fwht_avg_us"], "trace": tr}
            if pmc and pmc.get(name):
                ent["roofline"]["mfma_busy"] = pmc[name]
        out[name] = ent
        del pf
    return out


def fwht_extra(dev):
    """FWHT-128 of the prefill activation into the GEMM's pair-f16 layout,
    M=2048 at K=4096 and K=12288, as HBM GB/s of 2*M*K*2 bytes (fp16 in,
    pair f16 out), over 8 rotating inputs from a HIP graph."""
    out = {}
    for kk in (4096, 12288):
        xs = [torch.randn(2048, kk, device=dev, dtype=torch.float16) for _ in range(8)]
        ys = [torch.empty(2048, kk // 2, device=dev, dtype=torch.int32) for _ in range(8)]
        L = _lib.lib()

        def mk(x, y):
            def f():
                rc = L.pe_fwht128(x.data_ptr(), 0, 2048, kk, kk, y.data_ptr(), _lib.PE_XTF_PAIR_F16,
                                  _lib.stream_ptr(dev))
                if rc:
                    _lib.check(rc, "pe_fwht128")
            return f
        t, n = time_graph([mk(x, y) for x, y in zip(xs, ys)], 1, 16, 256, dev)
        b = 2 * 2048 * kk * 2
        out[f"fwht_m2048_k{kk}"] = {"us_per_call": round(t * 1e6, 2), "bytes": b,
                                    "GB/s": round(b / t / 1e9, 1),
                                    "hbm_frac": round(b / t / 1e9 / HBM_PEAK_GBS, 4)}
        del xs, ys
    return out


def hbm_extra(dev, steps=20, repeats=10):
    """The part's measured HBM ceiling, timed like the headline: a plain
    streaming read of the headline's 26 MB (pe_stream_read, 16 rotating
    buffers = 416 MB, graph replays of `steps` calls, cold and steady
    samples) and a 1 GiB copy (pe_copy: 2 GiB of traffic per call)."""
    L = _lib.lib()
    nbytes = algo_bytes(1, 12288, 4096, 4) // 16 * 16
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).random_(0, 255) for _ in range(N_COPIES)]
    sink = torch.empty(L.pe_stream_read_sink_bytes(nbytes), dtype=torch.uint8, device=dev)

    def mk(b):
        def f():
            rc = L.pe_stream_read(b.data_ptr(), nbytes, sink.data_ptr(), 0x9E3779B9,
                                  _lib.stream_ptr(dev))
            if rc:
                _lib.check(rc, "pe_stream_read")
        return f
    calls = [mk(b) for b in bufs]
    t_cold, _ = time_steps(calls, steps, 32, dev, repeats=repeats)
    t_st, _ = time_steps(calls, steps, 32, dev, repeats=repeats, steady=True)
    del bufs
    cb = 1 << 30
    src = torch.empty(cb, dtype=torch.uint8, device=dev).random_(0, 255)
    dst = torch.empty_like(src)

    def cp():
        rc = L.pe_copy(dst.data_ptr(), src.data_ptr(), cb, _lib.stream_ptr(dev))
        if rc:
            _lib.check(rc, "pe_copy")
    t_cp = time_eager(cp, 3, 20, dev)
    assert torch.equal(src[:1 << 20], dst[:1 << 20])
    del src, dst
    return {"hbm_read_26MB": {"us_per_call": round(t_st * 1e6, 3), "bytes": nbytes,
                              "GB/s": round(nbytes / t_st / 1e9, 1),
                              "hbm_frac": round(nbytes / t_st / 1e9 / HBM_PEAK_GBS, 4),
                              "cold_us_per_call": round(t_cold * 1e6, 3),
                              "cold_GB/s": round(nbytes / t_cold / 1e9, 1),
                              "what": "pe_stream_read of the headline's byte count, 16 rotating "
                                      "buffers, steady and cold graph samples like the headline"},
            "hbm_copy_1GiB": {"us_per_call": round(t_cp * 1e6, 1), "bytes_moved": 2 * cb,
                              "GB/s": round(2 * cb / t_cp / 1e9, 1),
                              "hbm_frac": round(2 * cb / t_cp / 1e9 / HBM_PEAK_GBS, 4)}}


class DecoderLayerLinears:
    """The linears of the C4 decoder layer (hidden 4096, 32 q / 8 kv heads of
    128, intermediate 12288): q/k/v Q5 sharing one transform of the normed
    hidden state, o Q6, gate/up Q3 sharing one transform, down Q4; tiled-16
    weights. `merged`: vLLM's form, q/k/v one qkv_proj (6144 rows) and
    gate/up one gate_up_proj (24576 rows), as PolarQuantLinearMethod sees
    them (create_weights sums output_partition_sizes); otherwise seven
    separate modules (the transformers form). As PolarQuantLinearMethod.apply
    runs them: M <= 32, one pe_linear_forward per linear (transform fused into
    each decode GEMV); M > 32, pe_fwht128 once for q/k/v and once for gate/up,
    pe_linear_forward_xtf for those, pe_linear_forward for o and down (their
    inputs are new activations)."""
    FUSED_MAX_M = 32

    SEPARATE = [("q", 4096, 4096, 5, "qkv"), ("k", 1024, 4096, 5, "qkv"),
                ("v", 1024, 4096, 5, "qkv"), ("o", 4096, 4096, 6, "o"),
                ("gate", 12288, 4096, 3, "gu"), ("up", 12288, 4096, 3, "gu"),
                ("down", 4096, 12288, 4, "down")]
    MERGED = [("qkv", 6144, 4096, 5, "qkv"), ("o", 4096, 4096, 6, "o"),
              ("gate_up", 24576, 4096, 3, "gu"), ("down", 4096, 12288, 4, "down")]

    def __init__(self, m, dev, seed, merged=True):
        self.SPECS = self.MERGED if merged else self.SEPARATE
        from polarengine_vllm.packing import tile_weights_16
        self.m, self.dev = m, dev
        L = _lib.lib()
        self.x = {g: torch.randn(m, 12288 if g == "down" else 4096, device=dev,
                                 dtype=torch.float16) for g in ("qkv", "o", "gu", "down")}
        self.xtf = {g: torch.empty(m, 2048, dtype=torch.int32, device=dev) for g in ("qkv", "gu")}
        self.lin = []
        wsb = 0
        for i, (name, n, k, bits, grp) in enumerate(self.SPECS):
            codes, norms, ct = make_layer(n, k, bits, dev, seed + i)
            codes, norms = tile_weights_16(codes, norms)
            fmt = (_lib.PE_PACK_NIBBLE if bits <= 4 else 0) | _lib.PE_LAYOUT_TILE16
            ct_host = np.ascontiguousarray(ct.cpu().numpy(), dtype=np.float32)
            y = torch.empty(m, n, dtype=torch.float16, device=dev)
            self.lin.append((name, n, k, bits, grp, codes, norms, ct, ct_host, fmt, y))
            wsb = max(wsb, L.pe_linear_workspace_size(m, k, n, bits, fmt),
                      L.pe_linear_xtf_workspace_size(m, k, n, bits, fmt))
        self.wsb = wsb
        self.ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)

    def __call__(self):
        L = _lib.lib()
        st = _lib.stream_ptr(self.dev)
        m = self.m
        shared = m > self.FUSED_MAX_M
        if shared:
            for g in ("qkv", "gu"):
                _lib.check(L.pe_fwht128(self.x[g].data_ptr(), 0, m, 4096, 4096, self.xtf[g].data_ptr(),
                                        _lib.PE_XTF_PAIR_F16, st), "pe_fwht128")
        for (name, n, k, bits, grp, codes, norms, ct, ct_host, fmt, y) in self.lin:
            if shared and grp in ("qkv", "gu"):
                rc = L.pe_linear_forward_xtf(self.xtf[grp].data_ptr(), m, k, codes.data_ptr(), bits,
                                             fmt, norms.data_ptr(), ct.data_ptr(), ct_host.ctypes.data,
                                             1 << bits, None, 0, y.data_ptr(), n, self.ws.data_ptr(),
                                             self.wsb, st)
            else:
                rc = L.pe_linear_forward(self.x[grp].data_ptr(), 0, m, k, k, codes.data_ptr(), bits,
                                         fmt, norms.data_ptr(), ct.data_ptr(), ct_host.ctypes.data,
                                         1 << bits, None, y.data_ptr(), n, self.ws.data_ptr(),
                                         self.wsb, st)
            if rc:
                _lib.check(rc, f"decoder layer {name}")


def decoder_layer_extra(dev):
    """C4: the decoder layer's quantized linears at M = 1 (GB/s of its
    algorithmic bytes: 120.6 MB for the seven separate linears), at a decode
    batch of M = 16, and at M = 512 (TFLOP/s of 197.6 GFLOP); four layer
    copies in turn (482 MB > the 256 MB Infinity Cache). decoder_layer_m*:
    vLLM's merged qkv / gate_up form; decoder_layer_separate_m*: seven
    separate modules."""
    out = {}
    for merged, tag in ((True, "decoder_layer"), (False, "decoder_layer_separate")):
        specs = DecoderLayerLinears.MERGED if merged else DecoderLayerLinears.SEPARATE
        for m in (1, 16, 512):
            layers = [DecoderLayerLinears(m, dev, seed=500 + 10 * i, merged=merged)
                      for i in range(4)]
            t, _ = time_graph(layers, 1, 8, 64 if m <= 32 else 16, dev)
            B = sum(algo_bytes(m, n, k, b) for _, n, k, b, _ in specs)
            fl = sum(2.0 * m * n * k for _, n, k, _, _ in specs)
            ent = {"us_per_layer": round(t * 1e6, 2), "algorithmic_bytes": B,
                   "GB/s": round(B / t / 1e9, 1),
                   "hbm_frac": round(B / t / 1e9 / HBM_PEAK_GBS, 4),
                   "TFLOP/s": round(fl / t / 1e12, 2),
                   "launches": len(specs) + (2 if m > DecoderLayerLinears.FUSED_MAX_M else 0),
                   "includes": ("qkv Q5, o Q6, gate_up Q3, down Q4 (vLLM merged modules)" if merged
                                else "q/k/v Q5, o Q6, gate/up Q3, down Q4 (separate modules)")
                   + "; the transform fused into each decode GEMV up to M = 32, "
                   "shared per input above; linears only"}
            if m > DecoderLayerLinears.FUSED_MAX_M:
                ent["mfma_frac"] = round(fl / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 4)
            out[f"{tag}_m{m}"] = ent
            del layers
            torch.cuda.empty_cache()
    return out


def e2e_extra(dev, context=1024, steps=32):
    """End-to-end greedy decode through polarengine_vllm.decode_runner (the
    model runner vLLM would provide; vLLM is not in this image): a model of
    Qwen3-8B's shapes (36 layers, hidden 4096, 32 / 8 heads of 128,
    intermediate 12288, vocabulary 151936) with random codes at the C4 bits
    (qkv Q5, o Q6, gate_up Q3, down Q4), bf16 embeddings / lm_head, a static
    bf16 KV cache of context + 64 positions, attention over it in torch. The
    step (all 36 layers, the lm_head and the argmax) is one HIP graph replay;
    tokens/s for the batch from `context`. quantized_linears_ms: the step's
    144 quantized linears alone (one graph replay of all of them); the rest
    of the step is torch (norms, rotary, cache writes, attention, SiLU,
    residual, lm_head)."""
    from polarengine_vllm.decode_runner import DecodeRunner, qwen3_8b_shapes
    cfg = qwen3_8b_shapes()
    out = {}
    for batch in (1, 16):
        run = DecodeRunner(cfg, batch, context + 64, dev, seed=7)
        r = run.greedy_tokens_per_s(context, steps, warmup=2)
        # the step's quantized linears alone (all layers, same inputs shapes)
        ins = {"qkv_proj": torch.randn(batch, cfg.hidden, device=dev, dtype=torch.bfloat16),
               "o_proj": torch.randn(batch, cfg.heads * cfg.head_dim, device=dev,
                                     dtype=torch.bfloat16),
               "gate_up_proj": torch.randn(batch, cfg.hidden, device=dev, dtype=torch.bfloat16),
               "down_proj": torch.randn(batch, cfg.intermediate, device=dev, dtype=torch.bfloat16)}

        def linears(run=run, ins=ins):
            for ly in run.layers:
                for nm in ("qkv_proj", "o_proj", "gate_up_proj", "down_proj"):
                    ly[nm](ins[nm])
        t_lin, _ = time_graph([linears], 1, 2, 4, dev)
        lin_bytes = sum(ly[nm].codes_packed.numel() if ly[nm].packed else ly[nm].codes.numel()
                        for ly in run.layers for nm in ("qkv_proj", "o_proj", "gate_up_proj",
                                                        "down_proj"))
        out[f"e2e_decode_b{batch}"] = {
            "tok_per_s": round(r["tok_per_s"], 1), "ms_per_step": round(r["ms_per_step"], 3),
            "quantized_linears_ms": round(t_lin * 1e3, 3),
            "context": context, "steps": steps, "layers": cfg.layers,
            "quantized_code_bytes": int(lin_bytes),
            "model": "Qwen3-8B shapes, random codes (qkv Q5, o Q6, gate_up Q3, down Q4), bf16 lm_head"}
        del run
        torch.cuda.empty_cache()
    return out


TRACE_JSON = os.path.join(ROOT, "profiles", "trace_gemv_q4_12288x4096_m1.json")


def summarize_trace(trace_csv, kernel_substr="gemv_mfma_kernel"):
    """Headline dispatches in a rocprofv3 kernel-trace CSV: mean / median
    kernel duration, and per timed replay (dispatches less than 50 us apart)
    the span (last end - first start) / dispatches; the median over replays
    of at least 100 dispatches."""
    import csv
    rows = []
    for r in csv.DictReader(open(trace_csv)):
        if kernel_substr in r["Kernel_Name"]:
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    if not rows:
        raise SystemExit(f"{trace_csv}: no {kernel_substr} dispatches")
    rows.sort()
    dur = np.array([(e - b) * 1e-3 for b, e, _ in rows])
    runs, cur = [], [rows[0]]
    for r in rows[1:]:
        if r[0] - cur[-1][1] > 50_000:
            runs.append(cur)
            cur = [r]
        else:
            cur.append(r)
    runs.append(cur)
    spans = [((run[-1][1] - run[0][0]) * 1e-3 / len(run), len(run)) for run in runs
             if len(run) >= 100]
    return {"kernel": rows[0][2], "dispatches": len(rows), "avg_us": round(float(dur.mean()), 3),
            "median_us": round(float(np.median(dur)), 3),
            "span_us_per_call": round(float(np.median([s for s, _ in spans])), 3) if spans else None,
            "replays": len(spans), "calls_per_replay": int(np.median([c for _, c in spans]))
            if spans else 0}


def summarize_prefill(trace_csv, pmc_csv=None, timed=20):
    """The M=2048 prefill dispatches of `bench.py --only-extra prefill2048`
    (per shape: warm-up calls until the clock settles, then `timed` calls,
    each an fwht128_kernel then the GEMM; Q4 12288x4096 first, then Q3
    4096x12288; the two GEMMs are different kernel instantiations and the two
    transforms different grid sizes): per shape the GEMM's and the
    transform's mean / median / min duration over the last `timed` calls;
    with the counter pass, per-dispatch means of every counter over the same
    calls and the MFMA figures derived from them."""
    import csv
    names = ("prefill_m2048", "prefill_down_q3_m2048")
    gemm, fw = {}, {}
    for r in csv.DictReader(open(trace_csv)):
        kn = r["Kernel_Name"]
        d = (int(r["Start_Timestamp"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
        if "gemm" in kn:
            gemm.setdefault(kn.split("(")[0], []).append(d)
        elif "fwht128_kernel" in kn:
            fw.setdefault(r.get("Grid_Size_X", r.get("Grid_Size")), []).append(d)
    if len(gemm) != 2 or len(fw) != 2:
        raise SystemExit(f"{trace_csv}: expected two GEMM kernels and two transform sizes, got "
                         f"{list(gemm)} / {list(fw)}")
    gk = sorted(gemm, key=lambda k: min(gemm[k])[0])   # in call order
    fk = sorted(fw, key=lambda k: min(fw[k])[0])
    out = {}
    for name, g, f in zip(names, gk, fk):
        gm = [x for _, x in sorted(gemm[g])][-timed:]
        fwv = [x for _, x in sorted(fw[f])][-timed:]
        out[name] = {"gemm_kernel": g.replace("void ", ""), "gemm_avg_us": round(float(np.mean(gm)), 2),
                     "gemm_median_us": round(float(np.median(gm)), 2),
                     "gemm_min_us": round(float(np.min(gm)), 2),
                     "gemm_max_us": round(float(np.max(gm)), 2),
                     "fwht_avg_us": round(float(np.mean(fwv)), 2),
                     "fwht_median_us": round(float(np.median(fwv)), 2), "timed_calls": len(gm),
                     "dispatches": len(gemm[g])}
    if pmc_csv:
        disp = {}
        for r in csv.DictReader(open(pmc_csv)):
            if "gemm" not in r["Kernel_Name"]:
                continue
            d = disp.setdefault(int(r["Dispatch_Id"]), {"kernel": r["Kernel_Name"].split("(")[0]})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        pm = {}
        for name, g in zip(names, gk):
            sel = [disp[i] for i in sorted(disp) if disp[i]["kernel"] == g][-timed:]
            if not sel:
                raise SystemExit(f"{pmc_csv}: no dispatches of {g}")
            keys = [k for k in sel[0] if k != "kernel"]
            mean = {k: float(np.mean([x[k] for x in sel])) for k in keys}
            ent = {"kernel": g.replace("void ", ""), "counters_mean": {k: round(v) for k, v in mean.items()}}
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and "SQ_BUSY_CU_CYCLES" in mean:
                ent["mfma_busy_of_cu_busy"] = round(
                    mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * mean["SQ_BUSY_CU_CYCLES"]), 4)
            if "SQ_INSTS_MFMA" in mean:
                ent["mfma_flops"] = mean["SQ_INSTS_MFMA"] * 32768.0  # 32x32x16 f16: 2*32*32*16
            if "GRBM_GUI_ACTIVE" in mean and "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
                ent["mfma_busy_of_elapsed"] = round(
                    mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (4.0 * 256 * mean["GRBM_GUI_ACTIVE"] / 8.0), 4)
            pm[name] = ent
        return out, pm
    return out, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="headline calls per timed sample")
    ap.add_argument("--warmup", type=int, default=200, help="untimed headline calls first")
    ap.add_argument("--repeats", type=int, default=10,
                    help="timed samples of --steps calls each (the line reports their median)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--profile-traffic", action="store_true",
                    help="run only the workload of the FETCH_SIZE / WRITE_SIZE pmc passes")
    ap.add_argument("--headline-only", action="store_true",
                    help="time only the headline call (for a rocprofv3 kernel trace whose "
                         "dispatches are exactly the headline's)")
    ap.add_argument("--only-extra", choices=("moe", "moe2048", "prefill", "prefill2048", "kv", "layer",
                                             "decode", "e2e", "fwht", "hbm"),
                    help="time only one of the extra workloads and print its JSON (for a "
                         "rocprofv3 kernel trace of that path alone)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the traffic JSON from the two pmc passes and exit")
    ap.add_argument("--summarize-trace", metavar="KERNEL_TRACE_CSV",
                    help="print the headline kernel's trace summary JSON and exit")
    ap.add_argument("--summarize-prefill", nargs="+", metavar="CSV",
                    help="KERNEL_TRACE_CSV [PMC_CSV] of --only-extra prefill2048: write "
                         "profiles/trace_gemm4_prefill_m2048.json (and pmc_...json) and exit")
    args = ap.parse_args()
    if args.summarize_pmc:
        print(json.dumps(summarize_pmc(*args.summarize_pmc), indent=1))
        return
    if args.summarize_trace:
        print(json.dumps(summarize_trace(args.summarize_trace), indent=1))
        return
    if args.summarize_prefill:
        tr, pm = summarize_prefill(*args.summarize_prefill[:2])
        with open(PREFILL_TRACE_JSON, "w") as f:
            json.dump(tr, f, indent=1)
        if pm:
            with open(PREFILL_PMC_JSON, "w") as f:
                json.dump(pm, f, indent=1)
        print(json.dumps({"trace": tr, "pmc": pm}, indent=1))
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
        fn = {"moe": moe_extra, "moe2048": lambda d: moe_extra(d, t=2048),
              "prefill": prefill_extra, "kv": kv_extra,
              "prefill2048": lambda d: prefill_m2048_extra(d, trace_only=True),
              "layer": decoder_layer_extra, "decode": decode_extra, "e2e": e2e_extra,
              "fwht": fwht_extra, "hbm": hbm_extra}[args.only_extra]
        print(json.dumps(fn(dev)))
        return

    n, k, bits, m = 12288, 4096, 4, 1
    x = torch.randn(m, k, device=dev, dtype=torch.float16)
    layers = [Linear(n, k, bits, m, dev, seed=100 + i, x=x) for i in range(N_COPIES)]
    t_call, samples = time_steps(layers, args.steps, args.warmup, dev, repeats=args.repeats,
                                 steady=True)
    t_cold, samples_cold = time_steps(layers, args.steps, args.warmup, dev, repeats=args.repeats)
    B = algo_bytes(m, n, k, bits)
    if args.headline_only:
        print(json.dumps({"workload": "headline only", "us_per_call": round(t_call * 1e6, 3),
                          "GB/s": round(B / t_call / 1e9, 1), "steps": args.steps,
                          "repeats": args.repeats,
                          "samples_us": [round(v * 1e6, 3) for v in samples],
                          "cold_us_per_call": round(t_cold * 1e6, 3),
                          "cold_samples_us": [round(v * 1e6, 3) for v in samples_cold]}))
        return
    t_hot, _ = time_graph(layers[:1], 1, args.warmup, 1024, dev)
    del layers

    extra = decode_extra(dev)
    extra.update(hbm_extra(dev, args.steps, args.repeats))
    extra.update(fwht_extra(dev))
    extra.update(prefill_extra(dev))
    extra.update(decoder_layer_extra(dev))
    extra["cache_hot_m1"] = {"us_per_call": round(t_hot * 1e6, 2),
                             "GB/s": round(B / t_hot / 1e9, 1),
                             "note": "one weight copy, Infinity-Cache resident"}
    extra.update(kv_extra(dev))
    extra.update(moe_extra(dev))
    # the same experts in the prefill regime (about 256 rows per expert)
    extra.update(moe_extra(dev, t=2048))
    extra.update(e2e_extra(dev))

    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    traffic = None  # HBM bytes per launch from the committed pmc summary, if any
    if os.path.exists(TRAFFIC_JSON):
        with open(TRAFFIC_JSON) as f:
            traffic = round(json.load(f)["traffic_bytes"])
    trace = None  # the committed kernel trace of `bench.py --headline-only`
    if os.path.exists(TRACE_JSON):
        with open(TRACE_JSON) as f:
            trace = json.load(f)
    # the kernel's launch duration: the event-timed period, or the traced mean
    # kernel duration when that is longer (the conservative of the two)
    us_event = t_call * 1e6
    us_kernel = max(us_event, trace["avg_us"]) if trace else us_event
    achieved = B / (us_kernel * 1e-6) / 1e9
    gbs = B / t_call / 1e9
    out = {
        "metric": "HBM GB/s + us/call, Q4 GEMV 12288x4096 M=1; prefill GEMM TFLOPS M=2048",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
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
        "timing": {"method": f"{args.repeats} steady samples of exactly {args.steps} calls (one "
                             "HIP graph replay each, queued behind an untimed replay of the same "
                             "graph so the timed one holds the calls alone; HIP events on the "
                             "replay stream); median",
                   "samples": args.repeats,
                   "min_us": round(min(samples) * 1e6, 3), "max_us": round(max(samples) * 1e6, 3),
                   "cold_us_per_call": round(t_cold * 1e6, 3),
                   "cold_GB/s": round(B / t_cold / 1e9, 1),
                   "cold_method": "the same samples without the untimed replay in front: the "
                                  "replay's launch latency falls inside the sample"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel_us": round(us_kernel, 3),
                     "kernel_us_source": "trace mean" if us_kernel > us_event else "HIP events",
                     "trace": trace},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out))


def decode_extra(dev):
    """Decode at M = 4..64 on the headline shape, the MLP's gate/up Q3
    12288x4096 and down Q4 4096x12288 at M = 1 / 4 / 16, and C1 (Q5
    4096x4096 M = 1)."""
    n, k, bits = 12288, 4096, 4
    extra = {}
    for mm in (4, 8, 16, 32, 64):
        lay = [Linear(n, k, bits, mm, dev, seed=200 + i) for i in range(N_COPIES)]
        t, _ = time_graph(lay, 4, 64, 512, dev)
        extra[f"decode_m{mm}"] = {"us_per_call": round(t * 1e6, 2),
                                  "GB/s": round(algo_bytes(mm, n, k, bits) / t / 1e9, 1)}
        del lay
    for name, (nn, kk, bb), ms in (("gateup_q3", (12288, 4096, 3), (1, 4, 16)),
                                   ("down_q4", (4096, 12288, 4), (1, 4, 16)),
                                   ("c1_q5_4096x4096", (4096, 4096, 5), (1,))):
        for mm in ms:
            lay = [Linear(nn, kk, bb, mm, dev, seed=400 + i) for i in range(N_COPIES)]
            t, _ = time_graph(lay, 4, 64, 512, dev)
            gb = algo_bytes(mm, nn, kk, bb) / t / 1e9
            extra[f"decode_{name}_m{mm}"] = {"us_per_call": round(t * 1e6, 2), "GB/s": round(gb, 1),
                                             "hbm_frac": round(gb / HBM_PEAK_GBS, 4)}
            del lay
    return extra


if __name__ == "__main__":
    main()
