#!/usr/bin/env python3
"""Benchmark of the MI355X low-bit projection path (one JSON line on stdout).

Headline (``value``): the Marlin-layout W4A16 decode GEMV of BASELINE.json
configs[1] at M=1 -- K=5120, N=17408, group 128 -- in GB/s of algorithmic
bytes (K*N/2 + (K/128)*N*2 + M*K*2 + M*N*2 per call).  Inputs are resident in
HBM before timing.  A *step* is one call on each of the ``sets`` independent
weight sets (> 2x the 256 MB Infinity Cache together, so the cache cannot
serve the weights): the calls of one step are captured once in a HIP graph,
and ``--steps`` replays of it are timed with HIP events on the launch stream
(``--warmup`` untimed replays first), so the timed region is
``steps x sets`` back-to-back kernels.

Extra fields report the other BASELINE.json configs: M=4/16 decode, the M=2048
prefill GEMM in TFLOP/s (both shapes), the rowwise fallback sweep, the
64-layer decode-step projection sweep, and the streaming-read ceiling of the
device (a kernel that only reads the same bytes).  ``cpu_baseline`` times a
vectorised torch-CPU restatement of the dequantise-then-matmul arithmetic on
the host's physical cores, on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor spec
TRAFFIC_FILE = "profiles/marlin_gemv_m1_k5120_n17408_traffic.txt"
FP16_DENSE_PEAK_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 flop/clk, vendor spec
MALL_BYTES = 256 * 1024 * 1024


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def marlin_bytes(m, k, n, g=128):
    groups = 1 if g <= 0 else k // g
    return k * n // 2 + groups * n * 2 + m * k * 2 + m * n * 2


def rowwise_bytes(m, k, n, bits, g):
    return n * ((k * bits + 7) // 8) + n * math.ceil(k / g) * 2 + m * k * 2 + m * n * 2


class MarlinProblem:
    """`sets` independent random Marlin weight sets of one shape (codes uniform in [0,16))."""

    def __init__(self, torch, dev, m, k, n, sets, seed):
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        self.m, self.k, self.n = m, k, n
        self.q = [torch.randint(-2 ** 31, 2 ** 31, (k // 16, 2 * n), dtype=torch.int32, device=dev, generator=gen)
                  for _ in range(sets)]
        self.s = [(torch.randn((k // 128, n), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
                  for _ in range(sets)]
        self.x = torch.randn((m, k), device=dev, generator=gen).half()
        self.out = [torch.empty((m, n), dtype=torch.float16, device=dev) for _ in range(sets)]
        self.ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)

    def call(self, lc, i):
        lc.lowbit_marlin_gemm_out(self.q[i], self.s[i], self.x, self.out[i], self.ws, self.k, 128)


class RowwiseProblem:
    def __init__(self, torch, dev, k, n, bits, g, sets, seed):
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        self.k, self.n, self.bits, self.g = k, n, bits, g
        pc = (k * bits + 7) // 8
        self.q = [torch.randint(0, 256, (n, pc), dtype=torch.uint8, device=dev, generator=gen) for _ in range(sets)]
        self.s = [(torch.randn((n, math.ceil(k / g)), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
                  for _ in range(sets)]
        self.x = torch.randn((k,), device=dev, generator=gen).half()

    def call(self, lc, i):
        lc.lowbit_gemv(self.q[i], self.s[i], self.x, self.k, self.g, self.bits)


WARM_MS = 30.0  # minimum untimed work before a timed region (graph replays)


def time_calls(torch, fn, n_sets, steps, warmup, use_graph=True):
    """Times `steps` steps of one call per weight set (`n_sets` calls each);
    returns (elapsed_ms, steps, calls).

    With use_graph the calls of `chunk` consecutive steps (the largest divisor
    of `steps` up to 100) are captured once in a HIP graph, as a serving loop
    captures its launches, and the graph is replayed steps / chunk times, so
    the timed region holds exactly `steps` steps and the host-side cost of a
    graph launch falls once per chunk rather than once per step; events
    bracket the replays on the launch stream.  At least `warmup` untimed steps
    (whole replays) and at least WARM_MS of untimed work run first."""
    steps = max(1, int(steps))
    stream = torch.cuda.current_stream()
    if use_graph:
        chunk = max(d for d in range(1, min(steps, 100) + 1) if steps % d == 0)
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for i in range(n_sets):  # eager warm-up before capture
                fn(i)
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        # capture on the warmed-up stream: its per-stream buffers already exist
        with torch.cuda.graph(graph, stream=side):
            for _ in range(chunk):
                for i in range(n_sets):
                    fn(i)
        replays = steps // chunk
        # warm-up: at least `warmup` steps and at least WARM_MS of work, so the
        # timed region starts at the engine clock a continuous decode loop runs
        # at (the clock rises over the first ~10-20 ms of back-to-back launches)
        warm_replays = max(1, math.ceil(max(1, int(warmup)) / chunk))
        t0 = time.perf_counter()
        for _ in range(warm_replays):
            graph.replay()
        torch.cuda.synchronize()
        per_replay = (time.perf_counter() - t0) / warm_replays
        extra = max(0, math.ceil(WARM_MS * 1e-3 / max(per_replay, 1e-6)) - warm_replays)
        for _ in range(min(extra, 10000)):
            graph.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(stop), steps, steps * n_sets

    def run_step():
        for i in range(n_sets):
            fn(i)
    for _ in range(max(1, int(warmup))):
        run_step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        run_step()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop), steps, steps * n_sets


def calls_per_step_for(n_sets, calls):
    """Steps (of `n_sets` calls) covering at least `calls` calls."""
    return max(1, math.ceil(calls / n_sets))


class DecodeStep:
    """the projections of a 64-layer 27B-class decode step.

    Per layer: QKV 5120->7168, O 5120->5120, gate/up 5120->2x17408 (one fused
    Marlin tensor whose output is the [gate | up] `mixed` row) and down
    17408->5120 through the SiLU-gated op on that `mixed` row -- the
    production call sequence (langburst/model.py:1414-1482).  W4 g128 random
    packed weights, all resident (about 10.9 GB).  fused_mlp: gate/up, SiLU
    and down as one lb_marlin_mlp_fused call (at M = 16 and 32 its gate/up
    launch stores fp16(silu(g) * u) and the down launch reads those
    activations, instead of the [gate | up] row and the gated op's own
    pre-pass), whose output is bit-identical to the two calls.  A call is one
    op of the C ABI; the SiLU-gated down projection at M >= 5 is two kernel
    launches (the gated activations first)."""

    HIDDEN, INTER, QKV, O_IN = 5120, 17408, 7168, 5120

    def __init__(self, torch, dev, m, layers, seed, fused_mlp=False):
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        h, it = self.HIDDEN, self.INTER

        def tensor(k, n):
            q = torch.randint(-2 ** 31, 2 ** 31, (k // 16, 2 * n), dtype=torch.int32, device=dev, generator=gen)
            s = (torch.randn((k // 128, n), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
            return q, s

        self.m, self.layers = m, []
        for _ in range(layers):
            self.layers.append({"qkv": tensor(h, self.QKV), "o": tensor(self.O_IN, h), "gate_up": tensor(h, 2 * it),
                                "down": tensor(it, h)})
        self.x = torch.randn((m, h), device=dev, generator=gen).half()
        self.qkv_out = torch.empty((m, self.QKV), dtype=torch.float16, device=dev)
        self.o_out = torch.empty((m, h), dtype=torch.float16, device=dev)
        self.mixed = torch.randn((m, 2 * it), device=dev, generator=gen).half()  # overwritten by gate/up
        self.down_out = torch.empty((m, h), dtype=torch.float16, device=dev)
        self.ws = torch.zeros((2 * it // 128 * 16,), dtype=torch.int32, device=dev)
        self.fused_mlp = fused_mlp
        self.calls_per_layer = 4
        if fused_mlp:
            from neurova_amd import capi

            self.capi = capi
            self.fws = torch.zeros((capi.marlin_mlp_fused_workspace_len(m, h, it),), dtype=torch.int32, device=dev)
            self.fscratch = torch.empty((capi.marlin_mlp_fused_scratch_bytes(m, h, it),), dtype=torch.uint8,
                                        device=dev)
            self.calls_per_layer = 3
        per_layer = (marlin_bytes(m, h, self.QKV) + marlin_bytes(m, self.O_IN, h) + marlin_bytes(m, h, 2 * it)
                     + marlin_bytes(m, it, h) + m * it * 2)  # the gated op reads [gate | up]: 2K halves per row
        self.bytes_per_step = per_layer * layers
        self.weight_bytes = sum(q.numel() * 4 + s.numel() * 2 for L in self.layers for (q, s) in L.values())

    def step(self, lc):
        h, it = self.HIDDEN, self.INTER
        for L in self.layers:
            lc.lowbit_marlin_gemm_out(*L["qkv"], self.x, self.qkv_out, self.ws, h, 128)
            lc.lowbit_marlin_gemm_out(*L["o"], self.x, self.o_out, self.ws, self.O_IN, 128)
            if self.fused_mlp:
                st = self.capi.marlin_mlp_fused(self.x, *L["gate_up"], *L["down"], self.down_out, h, it, 128, 128,
                                                self.fws, self.fscratch)
                assert st == 0, self.capi.status_string(st)
            else:
                lc.lowbit_marlin_gemm_out(*L["gate_up"], self.x, self.mixed, self.ws, h, 128)
                lc.lowbit_marlin_gemm_silu_packed_out(*L["down"], self.mixed, self.down_out, self.ws, it, 128)


# The projections the reference publishes M = 1 timings for
# (langburst/docs/PERFORMANCE_LOG.md:421-427, RTX 4080 16GB), K x N.  Those
# figures are another GPU's and are reported beside this device's only as
# context; vs_baseline stays null.
PUBLISHED_M1 = [
    ("mlp_gate_up", 5120, 34816, 150.87),
    ("mlp_down", 17408, 5120, 73.90),
    ("gdn_qkvz", 5120, 16384, 69.79),
    ("gdn_out", 6144, 5120, 40.00),
    ("attn_qkv", 5120, 14336, 61.92),
    ("attn_o", 6144, 5120, 39.85),
]
LM_HEAD = ("lm_head_argmax", 5120, 248320, 988.42)


def published_projections(torch, lc, dev, use_graph):
    """M = 1 calls of the reference's published projection shapes (plain
    Marlin GEMM, rotating weight sets > 2x the Infinity Cache) and the lm_head
    fused argmax (5120 -> 248320, two weight sets of 656 MB each)."""
    from neurova_amd import capi

    res = {"reference_source": "langburst/docs/PERFORMANCE_LOG.md:421-427 (RTX 4080 16GB, M = 1)"}
    done = {}
    for name, k, n, ref_us in PUBLISHED_M1:
        if (k, n) not in done:
            pc = marlin_bytes(1, k, n)
            ns = sets_for(pc)
            pr = MarlinProblem(torch, dev, 1, k, n, ns, seed=30 + k % 97 + n % 89)
            ms2, _, nc2 = time_calls(torch, lambda i: pr.call(lc, i), ns, calls_per_step_for(ns, 600), 5, use_graph)
            done[(k, n)] = (ms2 * 1e3 / nc2, pc)
            del pr
        u, pc = done[(k, n)]
        res[name] = {"k": k, "n": n, "us_per_call": round(u, 3), "GB/s": round(pc / u / 1e3, 1),
                     "frac_hbm": round(pc / u / 1e3 / HBM_PEAK_GBS, 4), "reference_rtx4080_us": ref_us}
        log(f"[bench] published {name} K={k} N={n}: {u:.2f} us, {pc / u / 1e3:.1f} GB/s")
    name, k, n, ref_us = LM_HEAD
    pc = marlin_bytes(1, k, n)
    ns = 2
    gen = torch.Generator(device=dev)
    gen.manual_seed(40)
    qs = [torch.randint(-2 ** 31, 2 ** 31, (k // 16, 2 * n), dtype=torch.int32, device=dev, generator=gen)
          for _ in range(ns)]
    ss = [(torch.randn((k // 128, n), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half() for _ in range(ns)]
    x = torch.randn((1, k), device=dev, generator=gen).half()
    ws = torch.zeros((n // 128 * 16,), dtype=torch.int32, device=dev)
    state = torch.zeros((1,), dtype=torch.int64, device=dev)
    out = torch.zeros((1,), dtype=torch.int64, device=dev)
    sync = torch.zeros((2,), dtype=torch.int32, device=dev)
    sc = torch.empty((max(1, capi.marlin_scratch_bytes(1, n, k, 128)),), dtype=torch.uint8, device=dev)

    def call(i):
        assert capi.marlin_gemm_argmax(x, qs[i], ss[i], ws, 128, state, out, sync, 1, sc) == 0

    ms2, _, nc2 = time_calls(torch, call, ns, 50, 5, use_graph)
    u = ms2 * 1e3 / nc2
    res[name] = {"k": k, "n": n, "us_per_call": round(u, 3), "GB/s": round(pc / u / 1e3, 1),
                 "frac_hbm": round(pc / u / 1e3 / HBM_PEAK_GBS, 4), "reference_rtx4080_us": ref_us,
                 "bytes_per_call": pc}
    log(f"[bench] lm_head argmax K={k} N={n}: {u:.2f} us, {pc / u / 1e3:.1f} GB/s")
    del qs, ss
    torch.cuda.empty_cache()
    return res


def decode_step_sweep(torch, lc, dev, m, layers=64, replays=5, fused_mlp=False):
    """Graph-captured decode steps (3 or 4 op calls per layer), timed with events."""
    ds = DecodeStep(torch, dev, m, layers, seed=100 + m, fused_mlp=fused_mlp)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ds.step(lc)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        ds.step(lc)
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    # untimed warm-up of at least WARM_MS, as in time_calls
    for _ in range(min(100, max(0, math.ceil(WARM_MS * 1e-3 / max(time.perf_counter() - t0, 1e-6)) - 1))):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    us = start.elapsed_time(stop) * 1e3 / replays
    res = {"layers": layers, "calls_per_step": ds.calls_per_layer * layers, "us_per_step": round(us, 1),
           "bytes_per_step": ds.bytes_per_step, "weight_bytes_resident": ds.weight_bytes,
           "GB/s": round(ds.bytes_per_step / us / 1e3, 1),
           "frac_hbm": round(ds.bytes_per_step / us / 1e3 / HBM_PEAK_GBS, 4)}
    del graph, ds
    torch.cuda.empty_cache()
    return res


def sets_for(bytes_per_set, minimum=8):
    return max(minimum, math.ceil(2.0 * MALL_BYTES / bytes_per_set))


def stream_ceiling(torch, dev, nbytes, n_sets, steps=30, wg_counts=(256, 512, 1024, 2048)):
    """The streaming-read ceiling: lb_probe_stream_read over `nbytes` per launch
    (the headline's algorithmic bytes), rotating over `n_sets` buffers like the
    headline, at several grid sizes; the best is reported."""
    from neurova_amd import capi

    nb = (nbytes + 15) // 16 * 16
    bufs = [torch.randint(0, 2 ** 31, (nb // 4,), dtype=torch.int32, device=dev) for _ in range(n_sets)]
    sink = torch.empty((max(wg_counts) * 4,), dtype=torch.int32, device=dev)
    per_wg = {}
    for wgs in wg_counts:
        def call(i, wgs=wgs):
            assert capi.probe_stream_read(bufs[i], sink, wgs) == 0
        ms, _, calls = time_calls(torch, call, n_sets, steps, 3, True)
        per_wg[wgs] = ms * 1e3 / calls
    best = min(per_wg, key=per_wg.get)
    us = per_wg[best]
    del bufs, sink
    torch.cuda.empty_cache()
    return {"bytes_per_launch": nb, "workgroups": best, "us_per_launch": round(us, 3),
            "GB/s": round(nb / us / 1e3, 1), "frac_hbm": round(nb / us / 1e3 / HBM_PEAK_GBS, 4),
            "us_by_workgroups": {str(w): round(v, 3) for w, v in per_wg.items()}}


def host_cpu():
    """CPU model, physical cores and the cores this process may run on."""
    model, sockets, per_socket = platform.processor() or platform.machine(), 1, 0
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "Model name":
                model = val
            elif key == "Socket(s)":
                sockets = int(val)
            elif key == "Core(s) per socket":
                per_socket = int(val)
    except (OSError, ValueError):
        pass
    physical = sockets * per_socket or (os.cpu_count() or 1)
    allowed = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"model": model, "physical_cores": physical, "allowed_cpus": allowed}


def _timed(fn, budget_s, min_calls=3):
    fn()
    ts, t_end = [], time.perf_counter() + budget_s
    while len(ts) < min_calls or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sum(ts) / len(ts), len(ts)


def cpu_baseline(m, k, n, budget_s=12.0):
    """The headline's dequantise-then-matmul arithmetic in vectorised torch-CPU
    (oracle/torch_cpu.py: fp16 (q - 8) * s weights, fp32 matmul) on the host's
    physical cores, timed for about `budget_s` seconds.  The reference itself
    has no CPU Marlin path (ops.py:65-79 raises): this is a stated port of the
    same arithmetic, not the reference's code."""
    import numpy as np
    import torch

    from oracle import torch_cpu as T

    cpu = host_cpu()
    threads = max(1, min(cpu["physical_cores"], cpu["allowed_cpus"]))
    torch.set_num_threads(threads)
    rng = np.random.default_rng(0)
    qw = torch.from_numpy(rng.integers(-2 ** 31, 2 ** 31, size=(k // 16, 2 * n), dtype=np.int64).astype(np.int32))
    s = torch.from_numpy((np.abs(rng.normal(0, 0.01, (k // 128, n))) + 1e-3).astype(np.float16))
    x = torch.from_numpy(rng.normal(0, 1, (m, k)).astype(np.float16))
    sec, calls = _timed(lambda: T.marlin_gemm(x, qw, s, 128), budget_s)
    return {
        "value": round(marlin_bytes(m, k, n) / sec / 1e9, 4),
        "unit": "GB/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"{calls} full calls of the headline M={m} K={k} N={n} g128 ({sec * 1e3:.1f} ms/call): Marlin unpack, "
                  "fp16 dequant and fp32 matmul in torch-CPU; the reference has no CPU Marlin path, this ports "
                  "its arithmetic",
        "cpu": cpu["model"], "physical_cores": cpu["physical_cores"], "allowed_cpus": cpu["allowed_cpus"],
    }


def cpu_rowwise_cfg1(budget_s=6.0):
    """the reference's CPU rowwise path (LowBitTensor.gemv's
    CPU branch, loader.py:170-171 over dequantize_lowbit_rows, :427-465) in
    vectorised torch-CPU on the physical cores, x [4096], W [4096, 4096] b4
    g128, seed 0: (a) dequant + fp16 matmul per call, (b) the matmul alone on
    the pre-dequantised fp16 matrix."""
    import torch

    from oracle import lowbit_oracle as O
    from oracle import torch_cpu as T

    cpu = host_cpu()
    threads = max(1, min(cpu["physical_cores"], cpu["allowed_cpus"]))
    torch.set_num_threads(threads)
    _, packed, scales, x = O.make_rowwise_inputs(4096, 4096, 4, 128, batch=1, seed=0)
    q, s, xv = torch.from_numpy(packed), torch.from_numpy(scales), torch.from_numpy(x[0])
    nbytes = rowwise_bytes(1, 4096, 4096, 4, 128)
    sec_a, na = _timed(lambda: T.rowwise_gemv(q, s, xv, 4096, 128, 4), budget_s / 2)
    dense = T.rowwise_dequant_rows(q, s, 4096, 128, 4)
    sec_b, nb = _timed(lambda: torch.matmul(dense, xv), budget_s / 2)
    return {"dequant_matmul": {"us_per_call": round(sec_a * 1e6, 1), "GB/s": round(nbytes / sec_a / 1e9, 4),
                               "calls": na},
            "matmul_only_predequantised": {"us_per_call": round(sec_b * 1e6, 1),
                                           "GB/s": round(nbytes / sec_b / 1e9, 4), "calls": nb},
            "cores": int(threads), "kind": "port", "impl": "torch-CPU (oracle/torch_cpu.py)", "cpu": cpu["model"]}


def read_traffic(path):
    """HBM bytes per headline launch from the committed counter summary, if any."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def pmc_probe(torch, lc, dev, shapes=((1, 5120, 17408),), calls=24):
    """Eager calls of each shape (the headline by default) plus a plain
    elementwise copy of known size, for the counter runs (the copy calibrates
    FETCH_SIZE / WRITE_SIZE).  A shape is (M, K, N) for the Marlin GEMV/GEMM or
    ("rowwise", bits, group, K, N) for the rowwise GEMV."""
    for sh in shapes:
        if sh[0] == "rowwise":
            _, bits, g, k, n = sh
            ns = sets_for(rowwise_bytes(1, k, n, bits, g))
            prob = RowwiseProblem(torch, dev, k, n, bits, g, ns, seed=1)
            what = f"rowwise b{bits} g{g} K={k} N={n}"
        else:
            m, k, n = sh
            ns = sets_for(marlin_bytes(m, k, n))
            prob = MarlinProblem(torch, dev, m, k, n, ns, seed=1)
            what = f"M={m} K={k} N={n}"
        torch.cuda.synchronize()
        for i in range(calls):
            prob.call(lc, i % ns)
        torch.cuda.synchronize()
        del prob
        log(f"[pmc-probe] {calls} calls of {what}")
    src = torch.ones((128 * 2 ** 20,), dtype=torch.float16, device=dev)  # 256 MiB read, 256 MiB written
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.add(src, 0, out=dst)
    torch.cuda.synchronize()
    log("[pmc-probe] 4 copies of 256 MiB")


def parse_pmc_shape(sh):
    """'MxKxN' -> (M, K, N); 'rBITSgGROUPxKxN' -> ("rowwise", BITS, GROUP, K, N)."""
    if sh.startswith("r"):
        head, k, n = sh[1:].split("x")
        bits, g = head.split("g")
        return ("rowwise", int(bits), int(g), int(k), int(n))
    return tuple(int(v) for v in sh.split("x"))


def gemm_probe(torch, lc, dev, calls=6):
    """Eager prefill GEMM calls of both BASELINE.json configs[2] shapes, for the
    MFMA / clock counter runs (a few warm-up calls first)."""
    for (k, n) in ((5120, 17408), (17408, 5120)):
        prob = MarlinProblem(torch, dev, 2048, k, n, 1, seed=11)
        for _ in range(calls):
            prob.call(lc, 0)
        torch.cuda.synchronize()
        del prob
        torch.cuda.empty_cache()
    log(f"[gemm-probe] {calls} calls of each M=2048 shape")


def mlp_probe(torch, dev, calls=40):
    """The production MLP at the model's shape (hidden 5120, intermediate
    17408, W4 g128) for M = 1, 4, 16, 32: `calls` graph-replayed calls of the
    two reference ops and of lb_marlin_mlp_fused (from M = 5 its gate_up launch
    stores the gated activations), over 4 rotating weight sets, for the
    kernel-trace runs."""
    from neurova_amd import capi

    h, it, sets = DecodeStep.HIDDEN, DecodeStep.INTER, 4
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)

    def tensor(k, n):
        q = torch.randint(-2 ** 31, 2 ** 31, (k // 16, 2 * n), dtype=torch.int32, device=dev, generator=gen)
        s = (torch.randn((k // 128, n), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
        return q, s

    w = [(tensor(h, 2 * it), tensor(it, h)) for _ in range(sets)]
    for m in (1, 4, 16, 32):
        x = torch.randn((m, h), device=dev, generator=gen).half()
        mixed = torch.empty((m, 2 * it), dtype=torch.float16, device=dev)
        out = torch.empty((m, h), dtype=torch.float16, device=dev)
        ws = torch.zeros((max(2 * it // 128 * 16, capi.marlin_mlp_fused_workspace_len(m, h, it)),), dtype=torch.int32,
                         device=dev)
        sc1 = torch.empty((capi.marlin_scratch_bytes(m, 2 * it, h, 128),), dtype=torch.uint8, device=dev)
        sc2 = torch.empty((capi.marlin_scratch_bytes(m, h, it, 128),), dtype=torch.uint8, device=dev)
        fsc = torch.empty((capi.marlin_mlp_fused_scratch_bytes(m, h, it),), dtype=torch.uint8, device=dev)

        def pair(i):
            (gq, gs), (dq, ds) = w[i % sets]
            assert capi.marlin_gemm(x, gq, mixed, gs, ws, 128, sc1) == 0
            assert capi.marlin_gemm_silu_packed(mixed, dq, out, ds, ws, 128, sc2) == 0

        def fused(i):
            (gq, gs), (dq, ds) = w[i % sets]
            assert capi.marlin_mlp_fused(x, gq, gs, dq, ds, out, h, it, 128, 128, ws, fsc) == 0

        accum = torch.empty((m, h), dtype=torch.float32, device=dev)
        sync = torch.zeros((2 * m,), dtype=torch.int32, device=dev)
        ssc = torch.empty((capi.marlin_mlp_scratch_bytes(m, h, it),), dtype=torch.uint8, device=dev)

        def streaming(i):
            (gq, gs), (dq, ds) = w[i % sets]
            assert capi.marlin_mlp_streaming(gq, gs, dq, ds, x, out, accum, sync, h, it, 128, 128, ssc) == 0

        for name, fn, n_calls in (("two reference ops", pair, calls), ("lb_marlin_mlp_fused", fused, calls),
                                  ("streaming (fp32 numerics)", streaming, sets)):
            ms, _, nc = time_calls(torch, fn, sets, calls_per_step_for(sets, n_calls), 1, True)
            log(f"[mlp-probe] M={m:2d} {name}: {ms * 1e3 / nc:.2f} us per MLP")
        assert int(ws.abs().sum()) == 0
    del w
    torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300, help="timed steps (one call on each weight set per step)")
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--sets", type=int, default=0, help="weight sets to rotate (0 = enough to exceed 2x MALL)")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-extra", action="store_true")
    ap.add_argument("--pmc-probe", action="store_true", help="run the counter-calibration probe and exit")
    ap.add_argument("--pmc-shapes", default="1x5120x17408",
                    help="comma-separated shapes for --pmc-probe: MxKxN (Marlin) or rBITSgGROUPxKxN "
                         "(rowwise GEMV, e.g. r2g128x17408x5120); default: the headline")
    ap.add_argument("--gemm-probe", action="store_true", help="run the prefill GEMM counter probe and exit")
    ap.add_argument("--mlp-probe", action="store_true", help="time the decode MLP (the reference op pair / lb_marlin_mlp_fused) and exit")
    ap.add_argument("--stream-probe", action="store_true",
                    help="time the streaming-read ceiling over the headline's bytes (or --stream-mb) and exit")
    ap.add_argument("--stream-mb", default="", help="comma-separated MB (1e6 bytes) for --stream-probe")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import neurova_amd  # noqa: F401  (registers langburst_cuda)
    import langburst_cuda as lc

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.pmc_probe:
        pmc_probe(torch, lc, dev, [parse_pmc_shape(sh) for sh in args.pmc_shapes.split(",")])
        return
    if args.gemm_probe:
        gemm_probe(torch, lc, dev)
        return
    if args.mlp_probe:
        mlp_probe(torch, dev)
        return
    if args.stream_probe:
        sizes = [int(float(v) * 1e6) for v in args.stream_mb.split(",")] if args.stream_mb else \
            [marlin_bytes(1, 5120, 17408)]
        for pc in sizes:
            r = stream_ceiling(torch, dev, pc, sets_for(pc), steps=max(1, args.steps // 10),
                               wg_counts=(256, 512, 1024, 2048, 4096))
            log(f"[stream-probe] {json.dumps(r)}")
        return
    use_graph = not args.no_graph
    log(f"[bench] device {torch.cuda.get_device_name(dev)}; graph={use_graph}")

    # ---- headline: Marlin decode GEMV, M=1 ----
    m, k, n = 1, 5120, 17408
    per_call = marlin_bytes(m, k, n)
    n_sets = args.sets or sets_for(per_call)
    prob = MarlinProblem(torch, dev, m, k, n, n_sets, seed=1)
    log(f"[bench] headline M={m} K={k} N={n}: {n_sets} weight sets ({n_sets * per_call / 2**20:.0f} MiB)")
    torch.cuda.synchronize()
    ms, steps, calls = time_calls(torch, lambda i: prob.call(lc, i), n_sets, args.steps, args.warmup, use_graph)
    us_per = ms * 1e3 / calls
    gbs = per_call / (us_per * 1e-6) / 1e9
    log(f"[bench] headline {us_per:.2f} us/call, {gbs:.1f} GB/s ({steps} steps x {n_sets} calls)")
    del prob
    torch.cuda.empty_cache()

    result = {
        "metric": "W4A16 GEMV GB/s (M=1) & GEMM TFLOP/s (M=2048), % of MI355X roofline",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / steps, 6),
        "calls_per_step": n_sets,
        "timed_calls": calls,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (int4 weights, fp32 accumulate)",
        "data": "synthetic (uniform int4 codes, |N(0,0.01)|+1e-3 fp16 scales, N(0,1) fp16 activations)",
        "config": {"workload": f"marlin_w4a16_gemv M=1 K=5120 N=17408 g128; a step is one call on each of "
                               f"{n_sets} rotating weight sets" + (", hipGraph replay" if use_graph else ", eager launches"),
                   "m": m, "k": k, "n": n, "group_size": 128, "weight_sets": n_sets},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_FILE)),
                     "traffic_source": f"{TRAFFIC_FILE} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per dispatch, "
                                       "calibrated on a copy kernel; not measured in this run)",
                     "bytes_per_launch": per_call, "us_per_launch": round(us_per, 3),
                     "timing": ("HIP events on the launch stream around the graph replays (graphs of up to 100 "
                                "steps); untimed warm-up of at least the requested steps and "
                                f"{WARM_MS:.0f} ms of work before it")},
    }

    if not args.skip_extra:
        extra = {"stream_read_ceiling": stream_ceiling(torch, dev, per_call, n_sets)}
        log(f"[bench] streaming-read ceiling over {per_call} B: {extra['stream_read_ceiling']['us_per_launch']:.2f} us, "
            f"{extra['stream_read_ceiling']['GB/s']:.1f} GB/s")
        for mm in (4, 16):
            pc = marlin_bytes(mm, k, n)
            ns = sets_for(pc)
            pr = MarlinProblem(torch, dev, mm, k, n, ns, seed=2 + mm)
            ms2, _, nc2 = time_calls(torch, lambda i: pr.call(lc, i), ns, calls_per_step_for(ns, 600), 5, use_graph)
            u = ms2 * 1e3 / nc2
            extra[f"marlin_gemv_m{mm}"] = {"us_per_call": round(u, 3), "GB/s": round(pc / u / 1e3, 1),
                                           "frac_hbm": round(pc / u / 1e3 / HBM_PEAK_GBS, 4)}
            log(f"[bench] M={mm}: {u:.2f} us, {pc / u / 1e3:.1f} GB/s")
            del pr
        extra["published_projections_m1"] = published_projections(torch, lc, dev, use_graph)
        for (kk, nn) in ((5120, 17408), (17408, 5120)):
            mm = 2048
            pr = MarlinProblem(torch, dev, mm, kk, nn, 2, seed=11)
            # 40 untimed calls (about 14 ms) first: the engine clock settles
            # under sustained MFMA load; the first few calls run faster or slower
            ms2, _, nc2 = time_calls(torch, lambda i: pr.call(lc, i), 2, 20, 20, use_graph)
            u = ms2 * 1e3 / nc2
            tf = 2.0 * mm * kk * nn / (u * 1e-6) / 1e12
            extra[f"marlin_gemm_m2048_k{kk}_n{nn}"] = {"us_per_call": round(u, 2), "TFLOP/s": round(tf, 1),
                                                       "frac_fp16_peak": round(tf / FP16_DENSE_PEAK_TFLOPS, 4)}
            log(f"[bench] GEMM M=2048 K={kk} N={nn}: {u:.1f} us, {tf:.1f} TFLOP/s")
            del pr
        for bits in (2, 3, 8):
            for g in (64, 128):
                pc = rowwise_bytes(1, 17408, 5120, bits, g)
                ns = sets_for(pc)
                pr = RowwiseProblem(torch, dev, 17408, 5120, bits, g, ns, seed=bits * g)
                ms2, _, nc2 = time_calls(torch, lambda i: pr.call(lc, i), ns, calls_per_step_for(ns, 400), 5, use_graph)
                u = ms2 * 1e3 / nc2
                extra[f"rowwise_b{bits}_g{g}"] = {"us_per_call": round(u, 3), "GB/s": round(pc / u / 1e3, 1),
                                                  "frac_hbm": round(pc / u / 1e3 / HBM_PEAK_GBS, 4)}
                log(f"[bench] rowwise b{bits} g{g}: {u:.2f} us, {pc / u / 1e3:.1f} GB/s")
                del pr
        pc = rowwise_bytes(1, 4096, 4096, 4, 128)
        ns = sets_for(pc)
        pr = RowwiseProblem(torch, dev, 4096, 4096, 4, 128, ns, seed=5)
        ms2, _, nc2 = time_calls(torch, lambda i: pr.call(lc, i), ns, calls_per_step_for(ns, 400), 5, use_graph)
        u = ms2 * 1e3 / nc2
        extra["rowwise_cfg1_b4_4096"] = {"us_per_call": round(u, 3), "GB/s": round(pc / u / 1e3, 1),
                                         "frac_hbm": round(pc / u / 1e3 / HBM_PEAK_GBS, 4)}
        del pr
        torch.cuda.empty_cache()
        # rowwise callers at their model shapes: the fused GDN in_proj_ba (96 rows,
        # K = 5120) and the embedding lookup (one row of 248320 x 5120 per token)
        pc = rowwise_bytes(1, 5120, 96, 4, 128)
        ns = sets_for(pc, minimum=64)
        pr = RowwiseProblem(torch, dev, 5120, 96, 4, 128, ns, seed=96)
        ms2, _, nc2 = time_calls(torch, lambda i: pr.call(lc, i), ns, calls_per_step_for(ns, 640), 2, use_graph)
        u = ms2 * 1e3 / nc2
        extra["rowwise_in_proj_ba_b4_g128_96x5120"] = {"us_per_call": round(u, 3), "GB/s": round(pc / u / 1e3, 1),
                                                       "frac_hbm": round(pc / u / 1e3 / HBM_PEAK_GBS, 4)}
        del pr
        emb_rows, emb_cols = 248320, 5120
        gen = torch.Generator(device=dev)
        gen.manual_seed(7)
        emb_q = torch.randint(0, 256, (emb_rows, emb_cols // 2), dtype=torch.uint8, device=dev, generator=gen)
        emb_s = (torch.randn((emb_rows, emb_cols // 128), device=dev, generator=gen) * 0.01).abs_().add_(1e-3).half()
        tokens = [torch.randint(0, emb_rows, (1,), device=dev, generator=gen) for _ in range(64)]
        ms2, _, nc2 = time_calls(torch, lambda i: lc.lowbit_row_dequant(emb_q, emb_s, tokens[i], emb_cols, 128, 4),
                              64, 10, 1, use_graph)
        u = ms2 * 1e3 / nc2
        pc = emb_cols // 2 + emb_cols // 128 * 2 + emb_cols * 2 + 8
        extra["row_dequant_embedding_b4_248320x5120"] = {"us_per_call": round(u, 3), "bytes_per_call": pc}
        log(f"[bench] in_proj_ba {extra['rowwise_in_proj_ba_b4_g128_96x5120']['us_per_call']:.2f} us, "
            f"embedding row {u:.2f} us")
        del emb_q, emb_s, tokens
        torch.cuda.empty_cache()
        for mm in (1, 4, 16, 32):
            extra[f"decode_step_64_layers_m{mm}"] = r = decode_step_sweep(torch, lc, dev, mm)
            log(f"[bench] 64-layer decode step M={mm}: {r['us_per_step']:.1f} us, {r['GB/s']:.1f} GB/s")
        for mm in (16, 32):
            extra[f"decode_step_64_layers_m{mm}_fused_mlp"] = r = decode_step_sweep(torch, lc, dev, mm, fused_mlp=True)
            log(f"[bench] 64-layer decode step M={mm}, lb_marlin_mlp_fused: {r['us_per_step']:.1f} us, "
                f"{r['calls_per_step']} calls")
        result["extra"] = extra

    if not args.skip_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(m, k, n)
            result["cpu_baseline"]["cfg1_rowwise_reference_cpu_path"] = cpu_rowwise_cfg1()
        except Exception as exc:  # the baseline is reported, never required
            result["cpu_baseline"] = {"value": None, "unit": "GB/s", "cores": 0, "kind": "port",
                                      "sample": f"failed: {exc}"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
