#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

Metric: "GPTQ-int4 decode matvec GB/s (% HBM peak) + prefill
GEMM TFLOP/s (% MFMA)".

A step is one batch-1 decode token through the Llama-7B-shaped GPTQ int4
linears of BASELINE.json configs[1] (group 128, f32 activations):
  q_proj   4096 x 4096                      st_gptq_i4_matvec
  gate/up  4096 x (2 x 11008), h = silu(g) * u   st_gptq_i4_gate_up_silu
  down     11008 x 4096 on h                st_gptq_i4_matvec
(the fused gate/up emits the down projection's input, so down reads one
vector; the reference-shaped down, st_gptq_i4_silu_matvec on separate gate
and up outputs, is timed alongside as `down_silu_ab`).
`value` = algorithmic bytes of the step / step time (GB/s), inputs resident
in HBM, the step replayed as a HIP graph (gaps between launches included).
Cold cache: the weights are replicated `--copies` times (default: enough for
> 512 MB, twice the MALL) and step i uses copy i % copies.

Also reported: each kernel's duration as a profiler sees it (HIP events that
hipExtLaunchKernel stamps with the kernel's own start and end, a fixed 5 x 200
calls whatever --steps says), the roofline of the dominant kernel (gate/up),
configs[0] (K = N = 2048, 256 cold copies), the prefill GEMM, the
INT8 legs, the lm_heads and the 36-layer stack, and
the CPU baseline (the oracle's WGSL-order gptq_matvec_4t restatement on the
host cores, on configs[0]'s seeded inputs; the reference WGSL cannot run
here: no wgpu/lavapipe).

Usage: python bench.py [--gpus 1] [--steps 200] [--warmup 20]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GPTQ-int4 decode matvec GB/s (% HBM peak) + prefill GEMM TFLOP/s (% MFMA)"
HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0
GS = 128


def decode_bytes(K, N, x_bytes, y_n, n_inputs=1):
    """qweight K*N/2 + f16 scales 2*(K/g)*N + activations + f32 outputs."""
    return K * N // 2 + 2 * (K // GS) * N + n_inputs * K * x_bytes + 4 * y_n


def make_gptq(torch, dev, K, N, gen, gpu=None):
    """Random GPTQ int4 weight (uniform nibbles, |N(0,0.02)| f16 scales); with
    `gpu`, repacked into the decode kernels' tiled layout as an upload does."""
    qw = torch.randint(-(2**31), 2**31 - 1, (K // 8, N), dtype=torch.int32, device=dev, generator=gen)
    sc = (torch.randn(K // GS, N, device=dev, generator=gen) * 0.02).abs().half()
    if gpu is not None:
        from shady_thinker_amd._lib import call, lib

        t = torch.empty(lib().st_gptq_i4_tiled_words(K, N, GS), dtype=torch.int32, device=dev)
        gpu.sync_stream()
        call("st_gptq_i4_repack", gpu.handle, qw.data_ptr(), t.data_ptr(), K, N, GS)
        qw = t
    return qw, sc


def time_loop(torch, fn, iters, warmup):
    """Average ms per call of fn(i), launched eagerly from Python."""
    for i in range(warmup):
        fn(i)
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    for i in range(iters):
        fn(i)
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters  # ms


class Replayer:
    """Steps fn(0..period-1) captured as one HIP graph (plus shorter tail
    graphs on demand), so that timing sees GPU time, not Python launch cost.
    Decode loops are launch-bound; a serving loop replays a captured graph
    the same way. Step i uses weight copy i % period (cold-cache rotation)."""

    def __init__(self, torch, fn, period):
        self.torch, self.fn, self.period = torch, fn, period
        self.stream = torch.cuda.Stream()
        self.graphs = {}
        with torch.cuda.stream(self.stream):
            for i in range(period):
                fn(i)  # warm: first-call set-up happens outside capture
        torch.cuda.synchronize()
        self._graph(period)

    def _graph(self, n):
        if n not in self.graphs:
            torch = self.torch
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(self.stream):
                with torch.cuda.graph(g, stream=self.stream):
                    for i in range(n):
                        self.fn(i)
            torch.cuda.synchronize()
            self.graphs[n] = g
        return self.graphs[n]

    def _steps(self, n):
        full, tail = divmod(n, self.period)
        for _ in range(full):
            self._graph(self.period).replay()
        if tail:
            self._graph(tail).replay()

    def run(self, iters, warmup):
        """`warmup` untimed steps, then exactly `iters` timed steps; returns
        ms per step."""
        torch = self.torch
        if iters % self.period:
            self._graph(iters % self.period)  # capture outside the timed region
        with torch.cuda.stream(self.stream):
            self._steps(warmup)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(self.stream)
            self._steps(iters)
            e1.record(self.stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters


def time_replays(torch, g, iters, warmup):
    """ms per replay of a captured graph (a StackGraph), events on the
    current stream around exactly `iters` replays."""
    for _ in range(warmup):
        g.replay()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(s)
    for _ in range(iters):
        g.replay()
    e1.record(s)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


class KernelTimer:
    """Kernel durations as a profiler reports them (rocprofv3 --kernel-trace),
    measured live with HIP events: before each call the context's timing
    events are armed (st_context_set_timing_events), so the library launches
    that call's kernels through hipExtLaunchKernel, which stamps the events
    with the first kernel's start and the last kernel's end. Calls are issued
    eagerly, `launches` per window; the figure is the median over `windows`
    of each window's mean, a fixed count that does not depend on --steps."""

    def __init__(self, torch, gpu, launches=200):
        self.torch, self.gpu, self.launches = torch, gpu, launches
        self.ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(launches)]
        s = torch.cuda.current_stream()
        for a, b in self.ev:  # creates the events
            a.record(s)
            b.record(s)
        torch.cuda.synchronize()

    def _arm(self, a, b):
        from shady_thinker_amd._lib import call

        call("st_context_set_timing_events", self.gpu.handle, a, b)

    def run(self, fn, windows=5, warmup=10, launches=None, arm=None):
        """ms per call of fn(i); `arm(start, stop)` arms the events for the
        next call (default: this context's timing events)."""
        torch = self.torch
        n = min(launches or self.launches, self.launches)
        arm = arm or self._arm
        for i in range(warmup):
            fn(i)
        means, i = [], warmup
        for _ in range(windows):
            torch.cuda.synchronize()
            for a, b in self.ev[:n]:
                arm(a.cuda_event, b.cuda_event)
                fn(i)
                i += 1
            arm(None, None)
            torch.cuda.synchronize()
            means.append(sum(a.elapsed_time(b) for a, b in self.ev[:n]) / n)
        means.sort()
        return means[len(means) // 2]


def cpu_baseline(seconds=10.0):
    """Oracle restatement of gptq_matvec_4t (src/shaders/gptq_matvec_4t.wgsl)
    on the host cores, OpenMP over columns, on configs[0]'s seeded inputs
    (K = N = 2048, group 128, seed 0: the CPU-runnable case BASELINE.md plans
    the reference's lavapipe run on), repeated for about `seconds`; the
    q_proj shape (4096 x 4096) beside it for half as long. Reported beside
    the GPU figures; not the optimisation target."""
    import oracle as O

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 16))

    def run(K, N, secs):
        c = O.gptq_case(0, K, N, GS)
        _, used = O.gptq_matvec_4t_omp(c["x"], c["qweight"], c["scales"], K, N, GS, cores)
        reps, t0 = 0, time.perf_counter()
        while True:
            O.gptq_matvec_4t_omp(c["x"], c["qweight"], c["scales"], K, N, GS, cores)
            reps += 1
            el = time.perf_counter() - t0
            if el >= secs:
                break
        per = el / reps
        return decode_bytes(K, N, 4, N) / per / 1e9, used, reps, el, per

    v, used, reps, el, per = run(2048, 2048, seconds)
    vq, _, rq, elq, perq = run(4096, 4096, seconds / 2)
    return {"value": round(v, 3), "unit": "GB/s", "cores": int(used), "kind": "port",
            "sample": f"oracle gptq_matvec_4t restatement (WGSL order, OpenMP over columns), configs[0] "
                      f"2048x2048 seed-0 inputs, f32 x, {reps} calls in {el:.1f} s ({per * 1e3:.3f} ms/call)",
            "q_proj_4096": {"value": round(vq, 3), "unit": "GB/s",
                            "sample": f"{rq} calls in {elq:.1f} s ({perq * 1e3:.2f} ms/call)"}}


# The kernel template that runs configs[1]'s gate/up (st_gptq_i4_gate_up_silu,
# one token, tiled weights, f32 x): the streaming kernel with 8-wave
# workgroups; `roofline.traffic` is reported only when the committed counter
# run measured this same template.
GATE_UP_KERNEL = "qmv_stream_kernel<1, 2, 0, 2, false, false, 8>"


def load_traffic():
    """(HBM bytes per launch, kernel template) of the dominant kernel from the
    committed rocprofv3 --pmc runs (profiles/qmv_gate_up_llama7b_traffic.json),
    or (None, None)."""
    p = os.path.join(ROOT, "profiles", "qmv_gate_up_llama7b_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            d = json.load(f)
        return d.get("traffic_bytes_per_launch"), d.get("kernel_template")
    return None, None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=0, help="weight copies for cold-cache rotation (0 = auto)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-stack", action="store_true", help="skip the configs[4] 36-layer linear stack")
    ap.add_argument("--copy-calibrate", action="store_true",
                    help="profiling helper: 10 plain 64 MiB device copies (calibrates FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--only", default="", help="profiling helper: launch only this kernel, eagerly "
                                               "(q|gate_up|down|gemm|gemm512|int8gemm|lm_int4), or replay one configs[4] "
                                               "stack step per step (stack1|stack16|stack32), or its 512-token prefill (prefill512)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU; multi-GPU runs are not part of it "
              "(the decode matvec would shard column-parallel over N, with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibrate:
        a = torch.ones(16 << 20, device="cuda")  # 64 MiB
        b = torch.empty_like(a)
        for _ in range(10):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibrate_bytes": a.numel() * 4, "calls": 10}))
        return

    import shady_thinker_amd as sta
    from shady_thinker_amd import model as Mdl

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gpu = sta.GpuContext(0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    if args.only in ("gemm", "gemm512"):  # eager GEMM loop for the profiler
        K, N, Mr = 4096, 14336, (2048 if args.only == "gemm" else 512)
        qw, sc = make_gptq(torch, dev, K, N, gen, gpu)
        perm = torch.randperm(K, device=dev, generator=gen).to(torch.int32)
        A = torch.randn(Mr, K, device=dev, generator=gen).half()
        C = torch.empty(Mr, N, device=dev, dtype=torch.float16)
        ms = time_loop(torch, lambda i: Mdl.gptq_gemm(gpu, A, qw, sc, C, K, N, GS, None, perm, sta.ST_FLAG_TILED),
                       args.steps, args.warmup)
        print(json.dumps({"only": args.only, "M": Mr, "steps": args.steps, "ms_eager": round(ms, 5),
                          "TFLOP/s": round(2.0 * Mr * K * N / (ms * 1e-3) / 1e12, 1)}))
        return

    if args.only == "int8gemm":  # eager INT8 prefill GEMM loop (configs[2] weight, M = 2048) for the profiler
        K, N, Mr = 5120, 13824, 2048
        w = torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=gen)
        wt = torch.empty(sta._lib.lib().st_int8_tiled_bytes(K, N), dtype=torch.int8, device=dev)
        gpu.sync_stream()
        sta._lib.call("st_int8_repack", gpu.handle, w.data_ptr(), wt.data_ptr(), K, N)
        sc = (torch.randn(N, device=dev, generator=gen) * 0.01).abs()
        A = torch.randn(Mr, K, device=dev, generator=gen).half()
        C = torch.empty(Mr, N, device=dev, dtype=torch.float16)
        ms = time_loop(torch, lambda i: Mdl.int8_gemm(gpu, A, wt, sc, C, K, N, sta.ST_FLAG_TILED), args.steps,
                       args.warmup)
        print(json.dumps({"only": args.only, "M": Mr, "steps": args.steps, "ms_eager": round(ms, 5),
                          "TFLOP/s": round(2.0 * Mr * K * N / (ms * 1e-3) / 1e12, 1)}))
        return

    if args.only == "lm_int4":  # eager int4 lm_head calls, 4 cold copies (for the profiler)
        K, N = 2560, 151936
        W = [make_gptq(torch, dev, K, N, gen, gpu) for _ in range(4)]
        x = torch.randn(1, K, device=dev, generator=gen)
        y = torch.empty(1, N, device=dev)
        ms = time_loop(torch, lambda i: Mdl.gptq_matvec(gpu, "lm_head", x, W[i % 4][0], W[i % 4][1], y, K, N, GS,
                                                        flags=sta._lib.ST_FLAG_TILED), args.steps, args.warmup)
        print(json.dumps({"only": args.only, "steps": args.steps, "ms_eager": round(ms, 5)}))
        return
    if args.only in ("stack1", "stack16", "stack32"):  # configs[4] stack: graph replays (per-linear kernel times in the profile)
        out = bench_stack(torch, dev, gpu, Mdl, gen, args, batches=(int(args.only[5:]),), prefill=False)
        print(json.dumps({"only": args.only, **out}))
        return
    if args.only == "prefill512":  # configs[4] 512-token prefill only (per-GEMM times in the profile)
        out = bench_stack(torch, dev, gpu, Mdl, gen, args, batches=(), prefill=True)
        print(json.dumps({"only": args.only, **out}))
        return

    H, I = 4096, 11008
    shapes = {"q": (H, H), "gate_up": (H, I), "down": (I, H)}
    b_q = decode_bytes(H, H, 4, H)
    b_gu = decode_bytes(H, 2 * I, 4, I)  # two weights of 4096 x 11008, one f32 output per column pair
    b_dn = decode_bytes(I, H, 4, H)  # h = silu(g) * u from the gate/up kernel
    b_dn_ab = decode_bytes(I, H, 4, H, n_inputs=2)  # reference shape: a and b
    step_bytes = b_q + b_gu + b_dn
    copies = args.copies or max(2, -(-2 * 256 * 2**20 // step_bytes) + 1)

    W = []
    for _ in range(copies):
        W.append({
            "q": make_gptq(torch, dev, H, H, gen, gpu),
            "g": make_gptq(torch, dev, H, I, gen, gpu),
            "u": make_gptq(torch, dev, H, I, gen, gpu),
            "d": make_gptq(torch, dev, I, H, gen, gpu),
        })
    TF = sta._lib.ST_FLAG_TILED
    x = torch.randn(1, H, device=dev, generator=gen)
    yq = torch.empty(1, H, device=dev)
    a = torch.randn(1, I, device=dev, generator=gen)
    b = torch.randn(1, I, device=dev, generator=gen)
    ygu = torch.empty(1, I, device=dev)
    ydn = torch.empty(1, H, device=dev)

    def k_q(i):
        w = W[i % copies]["q"]
        Mdl.gptq_matvec(gpu, "q_proj", x, w[0], w[1], yq, H, H, GS, flags=TF)

    def k_gu(i):
        w = W[i % copies]
        Mdl.fused_gate_up_silu(gpu, x, w["g"][0], w["g"][1], w["u"][0], w["u"][1], ygu, H, I, GS, flags=TF)

    def k_dn(i):
        w = W[i % copies]["d"]
        Mdl.gptq_matvec(gpu, "down_proj", ygu, w[0], w[1], ydn, I, H, GS, flags=TF)

    def k_dn_ab(i):
        w = W[i % copies]["d"]
        Mdl.fused_silu_gptq_down(gpu, a, b, w[0], w[1], ydn, I, H, GS, flags=TF)

    def step(i):
        k_q(i)
        k_gu(i)
        k_dn(i)

    if args.only:
        fn = {"q": k_q, "gate_up": k_gu, "down": k_dn}.get(args.only)
        if fn is not None:
            ms = time_loop(torch, fn, args.steps, args.warmup)  # eager: one dispatch per call (for counters)
            print(json.dumps({"only": args.only, "steps": args.steps, "ms_eager": round(ms, 5)}))
            return

    ms_step = Replayer(torch, step, copies).run(args.steps, args.warmup)
    ms_eager = time_loop(torch, step, args.steps, args.warmup)
    kt = KernelTimer(torch, gpu)
    ms_k = {n: kt.run(f) for n, f in (("q_proj", k_q), ("gate_up", k_gu), ("down", k_dn), ("down_silu_ab", k_dn_ab))}
    # the same launches back to back in a graph: kernel time plus the gap
    # between launches
    ms_g = {n: Replayer(torch, f, copies).run(max(args.steps, 100), args.warmup)
            for n, f in (("q_proj", k_q), ("gate_up", k_gu), ("down", k_dn))}
    value = step_bytes / (ms_step * 1e-3) / 1e9
    ms_gu = ms_k["gate_up"]
    gu_gbs = b_gu / (ms_gu * 1e-3) / 1e9
    kbytes = {"q_proj": b_q, "gate_up": b_gu, "down": b_dn, "down_silu_ab": b_dn_ab}
    kernels = {}
    for n, ms in ms_k.items():
        kernels[n] = {"ms": round(ms, 5), "bytes": kbytes[n], "GB/s": round(kbytes[n] / ms / 1e6, 1),
                      "hbm_frac": round(kbytes[n] / ms / 1e6 / HBM_PEAK_GBS, 4)}
        if n in ms_g:
            kernels[n]["ms_graph_per_launch"] = round(ms_g[n], 5)
    traffic, traffic_kernel = load_traffic()

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xf32",
        "data": "synthetic (torch RNG: uniform nibbles, |N(0,0.02)| f16 scales, N(0,1) f32 activations)",
        "config": {
            "workload": "configs[1]: Llama-7B decode linears, GPTQ int4 g128, batch 1: q_proj 4096x4096 + "
                        "fused gate/up 4096x(2x11008) emitting silu(g)*u + down 11008x4096 on it",
            "batch": 1, "group_size": GS, "cold_cache_copies": copies,
            "step_bytes": step_bytes, "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        },
        "ms_per_step_eager_python": round(ms_eager, 5),
        "timing": "value / ms_per_step: HIP-graph replay of exactly `steps` steps (one graph = one step per weight "
                  "copy), events on the replay stream; kernels.*: kernel durations (hipExtLaunchKernel events on "
                  "each call's kernels, median of 5 windows of 200 eager calls, cold weight copies), "
                  "ms_graph_per_launch: the same kernel back to back in a graph, gap included",
        "kernels": kernels,
        "roofline": {"bound": "hbm", "kernel": GATE_UP_KERNEL + " (st_gptq_i4_gate_up_silu)",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic if traffic_kernel == GATE_UP_KERNEL else None},
    }

    sc = bench_stream_ceiling(torch, dev, kt, {"q_proj": b_q, "gate_up": b_gu, "down": b_dn,
                                               "lm_head_int4": decode_bytes(2560, 151936, 4, 151936),
                                               "cfg0": decode_bytes(2048, 2048, 4, 2048)})
    out["stream_ceiling"] = sc
    if "gate_up" in sc:
        for k in ("q_proj", "gate_up", "down"):
            out["kernels"][k]["frac_of_stream"] = round(sc[k]["ms"] / out["kernels"][k]["ms"], 4)
        out["roofline"]["stream_ceiling_GB/s"] = sc["gate_up"]["GB/s"]
        out["roofline"]["frac_of_stream"] = out["kernels"]["gate_up"]["frac_of_stream"]
    out["cfg0"] = bench_cfg0(torch, dev, gpu, Mdl, gen, kt)
    if "cfg0" in sc:
        out["cfg0"]["frac_of_stream"] = round(sc["cfg0"]["ms"] / out["cfg0"]["ms"], 4)

    if not args.no_gemm:
        out["gemm"] = bench_gemm(torch, dev, gpu, Mdl, gen, kt)
    out["lm_head_bf16"] = bench_lm_head(torch, dev, gpu, Mdl, gen, kt)
    out["lm_head_int4"] = bench_lm_head_int4(torch, dev, gpu, Mdl, gen, kt)
    if "lm_head_int4" in sc:
        out["lm_head_int4"]["M1"]["frac_of_stream"] = round(sc["lm_head_int4"]["ms"] / out["lm_head_int4"]["M1"]["ms"], 4)
    out["int8_cfg2"] = bench_int8(torch, dev, gpu, Mdl, gen, kt)
    if not args.no_stack:
        out["stack_cfg4"] = bench_stack(torch, dev, gpu, Mdl, gen, args)

    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    gpu.close()
    print(json.dumps(out))


def bench_stream_ceiling(torch, dev, kt, sizes):
    """The plain-stream ceiling of each decode launch: a kernel that only
    reads the same number of bytes (bench_probe/libstream_probe.so, 16-byte
    nontemporal loads, eight in flight per lane, no compute), timed like the
    kernels (kernel durations from hipExtLaunchKernel events, each call on its
    own window of a 1 GiB buffer, so every read comes from HBM), best over
    four grid sizes. What a launch of that size can reach on this box; the
    kernels' `frac_of_stream` is measured against it. A measuring stick, not
    the roofline (that is the fraction of 8 TB/s)."""
    import ctypes

    path = os.path.join(ROOT, "bench_probe", "libstream_probe.so")
    if not os.path.exists(path):
        return {"status": "bench_probe/libstream_probe.so not built"}
    lib = ctypes.CDLL(path)
    lib.stp_read.restype = ctypes.c_int
    lib.stp_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                             ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    total = 1 << 30
    buf = torch.randint(-(2**31), 2**31 - 1, (total // 4,), dtype=torch.int32, device=dev)
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    out = {"probe": "stream_read_kernel (bench_probe/libstream_probe.so): read-only, 16-byte nontemporal loads, 256 "
                    "threads per workgroup, best of grids 256/512/1024/2048; kernel durations, cold windows of a "
                    "1 GiB buffer"}
    armed = [None, None]

    def arm(a, b):
        armed[0], armed[1] = a, b

    for name, nbytes in sizes.items():
        nb = (nbytes + 255) // 256 * 256
        if 2 * nb > total:
            raise ValueError(f"stream ceiling: {nb} bytes needs a buffer above {total} bytes for two cold windows")
        period = min(64, total // nb)
        best = None
        for grid in (256, 512, 1024, 2048):
            def rd(i, grid=grid):
                r = lib.stp_read(buf.data_ptr() + (i % period) * nb, nb, sink.data_ptr(), grid, 256, 0,
                                 torch.cuda.current_stream().cuda_stream, armed[0], armed[1])
                if r:
                    raise RuntimeError(f"stp_read -> {r}")
            ms = kt.run(rd, windows=3, launches=100, arm=arm)
            if best is None or ms < best[0]:
                best = (ms, grid)
        gbs = nb / (best[0] * 1e-3) / 1e9
        out[name] = {"bytes": nb, "ms": round(best[0], 5), "GB/s": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "grid": best[1]}
    del buf
    return out


def bench_cfg0(torch, dev, gpu, Mdl, gen, kt):
    """one GPTQ int4 linear, K = N = 2048, group 128, batch 1,
    f32 x (2,179,072 algorithmic bytes). Cold cache as BASELINE.md sets it:
    256 rotated weight copies (558 MB, above twice the MALL), kernel
    durations over 5 windows of 200 calls."""
    K = N = 2048
    copies = 256
    W = [make_gptq(torch, dev, K, N, gen, gpu) for _ in range(copies)]
    TF = sta_flags_tiled()
    x = torch.randn(1, K, device=dev, generator=gen)
    y = torch.empty(1, N, device=dev)
    ms = kt.run(lambda i: Mdl.gptq_matvec(gpu, "cfg0", x, W[i % copies][0], W[i % copies][1], y, K, N, GS, flags=TF))
    b = decode_bytes(K, N, 4, N)
    del W
    return {"K": K, "N": N, "cold_cache_copies": copies, "ms": round(ms, 5), "bytes": b,
            "GB/s": round(b / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_gemm(torch, dev, gpu, Mdl, gen, kt):
    """int4 prefill GEMM with act-order, M in {512, 2048},
    K = 4096, N = 14336, f16 A, f16 C (the act-order gather + A pre-pass is
    inside the timed call). Next to it, for scale: torch's f16 GEMM of the
    same shape (hipBLASLt, dense f16 B, no dequant)."""
    import shady_thinker_amd as sta

    K, N = 4096, 14336
    qw, sc = make_gptq(torch, dev, K, N, gen, gpu)  # tiled, as an upload stores it
    perm = torch.randperm(K, device=dev, generator=gen).to(torch.int32)
    out = {"K": K, "N": N, "group_size": GS, "act_order": True, "peak_TFLOP/s": F16_MFMA_PEAK_TFLOPS}
    for Mr in (512, 2048):
        A = torch.randn(Mr, K, device=dev, generator=gen).half()
        C = torch.empty(Mr, N, device=dev, dtype=torch.float16)
        try:
            Mdl.gptq_gemm(gpu, A, qw, sc, C, K, N, GS, None, perm, sta.ST_FLAG_TILED)
        except sta.ShadyHipError as e:
            return {"status": "not available", "error": str(e)}
        ms = kt.run(lambda i: Mdl.gptq_gemm(gpu, A, qw, sc, C, K, N, GS, None, perm, sta.ST_FLAG_TILED), windows=3,
                    launches=50)
        tf = 2.0 * Mr * K * N / (ms * 1e-3) / 1e12
        B16 = torch.randn(N, K, device=dev, generator=gen).half()
        ms_ref = Replayer(torch, lambda i: torch.matmul(A, B16.t()), 1).run(30, 3)
        del B16
        out[f"M{Mr}"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1), "mfma_frac": round(tf / F16_MFMA_PEAK_TFLOPS, 4),
                         "torch_f16_gemm_TFLOP/s": round(2.0 * Mr * K * N / (ms_ref * 1e-3) / 1e12, 1)}
    return out


def bench_stack(torch, dev, gpu, Mdl, gen, args, batches=(1, 16, 32), prefill=True):
    """the quantized linear stack of a 36-layer decoder
    (hidden 2560, 32 q / 8 kv heads of 128, intermediate 9728, vocab 151936),
    every linear GPTQ int4 g128 (lm_head included), random-init packed
    weights (2.27 GB: each token streams them from HBM). q is the reference's
    gated width, 2 * 32 * 128 = 8192 columns (src/model.rs:696: the query and
    its output gate); o reads 32 * 128 = 4096. A token = one
    DecoderStack step (per layer q|k|v as one concatenated linear, o, fused
    gate/up emitting silu(g)*u, down on it; then the lm_head), captured once
    with DecoderStack.capture and replayed; batch 1 and 16 (the config), and
    32 (every linear in one 32-token launch). Attention and
    norms are outside the path (no hooks), so activations are synthetic."""
    H, Q, QG, KV, I, V, L = 2560, 4096, 8192, 1024, 9728, 151936, 36
    TF = sta_flags_tiled()
    import shady_thinker_amd as sta

    def gw(k, n):
        qw, sc = make_gptq(torch, dev, k, n, gen, gpu)
        return sta.GptqWeight(qw, sc, None, None, k, n, GS, TF)

    # One DecoderLinears per layer (q, k and v concatenated at construction:
    # GptqWeight.cat, values unchanged, one launch instead of three).
    layers = [sta.DecoderLinears(gw(H, QG), gw(H, KV), gw(H, KV), gw(Q, H), gw(H, I), gw(H, I), gw(I, H))
              for _ in range(L)]
    lm = make_gptq(torch, dev, H, V, gen, gpu)
    per_layer = (decode_bytes(H, QG, 4, QG) + 2 * decode_bytes(H, KV, 4, KV) + decode_bytes(Q, H, 4, H) +
                 decode_bytes(H, 2 * I, 4, I) + decode_bytes(I, H, 4, H))
    out = {"layers": L, "weights_GB": None, "api": "DecoderStack.capture (one HIP graph per token step)",
           "q_width": QG, "q_width_note": "gated q, 2 * heads * head_dim (src/model.rs:696)"}
    stack = sta.DecoderStack(layers, sta.GptqWeight(lm[0], lm[1], None, None, H, V, GS, TF))
    wbytes = 0
    for Mb in batches:
        b = stack.buffers(gpu, Mb)
        for t in (b.x, b.attn, b.xm):
            t.normal_(generator=gen)
        g = stack.capture(gpu, b)
        ms = time_replays(torch, g, 30, 3)
        # algorithmic bytes of one step: the weights (read once for all Mb
        # tokens) plus batch-1 activation terms (Mb - 1 more rows are < 0.1%)
        tok_bytes = L * per_layer + decode_bytes(H, V, 4, V)
        wbytes = tok_bytes
        out[f"batch{Mb}"] = {"ms_per_token_step": round(ms, 4), "tokens_per_s": round(Mb / (ms * 1e-3), 1),
                             "GB/s": round(tok_bytes / (ms * 1e-3) / 1e9, 1),
                             "hbm_frac": round(tok_bytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "linear_calls_per_step": 4 * L + 1, "qkv": "one concatenated linear"}
        del g, b
    out["weights_GB"] = round(wbytes / 1e9, 3)
    if not prefill:
        del layers, lm, stack
        torch.cuda.empty_cache()
        return out
    # Prefill of a 512-token prompt through the same weights with the GEMM
    # (DecoderLinears.prefill: f16 activations and outputs; q|k|v, o, gate
    # and up in one call, and down on silu(gate) * up fused into the GEMM's A
    # pass), then the lm_head for the last token only, as a prefill does.
    P = 512
    xa = torch.randn(P, H, device=dev, generator=gen).half()
    aa = torch.randn(P, Q, device=dev, generator=gen).half()
    cq = torch.empty(P, QG + 2 * KV, device=dev, dtype=torch.float16)
    co = torch.empty(P, H, device=dev, dtype=torch.float16)
    cg = torch.empty(P, I, device=dev, dtype=torch.float16)
    cu = torch.empty(P, I, device=dev, dtype=torch.float16)
    cd = torch.empty(P, H, device=dev, dtype=torch.float16)
    xl = torch.randn(1, H, device=dev, generator=gen)
    logits1 = torch.empty(1, V, device=dev)

    def prefill(i):
        for layer in layers:
            layer.prefill(gpu, xa, aa, cq, co, cg, cu, cd)
        Mdl.gptq_matvec(gpu, "lm_head", xl, lm[0], lm[1], logits1, H, V, GS, flags=TF)

    ms = Replayer(torch, prefill, 1).run(5, 1)
    flops = 2.0 * P * L * (H * QG + 2 * H * KV + Q * H + 2 * H * I + I * H)
    out[f"prefill{P}"] = {"ms": round(ms, 3), "tokens_per_s": round(P / (ms * 1e-3), 1),
                          "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1), "gemm_calls": 4 * L}
    out["weights_GB"] = round(wbytes / 1e9, 3)
    del layers, lm
    torch.cuda.empty_cache()
    return out


def sta_flags_tiled():
    from shady_thinker_amd._lib import ST_FLAG_TILED

    return ST_FLAG_TILED


def bench_int8(torch, dev, gpu, Mdl, gen, kt):
    """INT8 per-channel weights [13824, 5120] (70.8 MB), f16
    activations, M = 1 / 8 / 32 (matvec to skinny GEMM), 4 cold copies."""
    K, N, copies = 5120, 13824, 4
    ws = [torch.randint(-127, 128, (N, K), device=dev, dtype=torch.int8, generator=gen) for _ in range(copies)]
    from shady_thinker_amd._lib import ST_FLAG_TILED, call, lib

    def tile8(w):  # the upload-time layout (Int8Weight.upload)
        t = torch.empty(lib().st_int8_tiled_bytes(K, N), dtype=torch.int8, device=dev)
        gpu.sync_stream()
        call("st_int8_repack", gpu.handle, w.data_ptr(), t.data_ptr(), K, N)
        return t

    ws = [tile8(w) for w in ws]
    sc = (torch.randn(N, device=dev, generator=gen) * 0.01).abs()
    out = {"K": K, "N": N}
    for Mr in (1, 8, 32):
        x = torch.randn(Mr, K, device=dev, generator=gen).half()
        y = torch.empty(Mr, N, device=dev)
        ms = kt.run(lambda i: Mdl.int8_matvec(gpu, x, ws[i % copies], sc, y, K, N, ST_FLAG_TILED))
        b = K * N + 4 * N + 2 * Mr * K + 4 * Mr * N
        out[f"M{Mr}"] = {"ms": round(ms, 5), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "TOPS": round(2.0 * Mr * K * N / (ms * 1e-3) / 1e12, 2)}
    # Prefill on the same weight (st_int8_gemm, f16 A and C), M in {512, 2048},
    # next to torch's f16 GEMM of the same shape (hipBLASLt, dense f16 B).
    out["prefill"] = {"kernel": "gemm_kernel INT8 (st_int8_gemm)", "peak_TFLOP/s": F16_MFMA_PEAK_TFLOPS}
    for Mr in (512, 2048):
        A = torch.randn(Mr, K, device=dev, generator=gen).half()
        C = torch.empty(Mr, N, device=dev, dtype=torch.float16)
        ms = kt.run(lambda i: Mdl.int8_gemm(gpu, A, ws[0], sc, C, K, N, ST_FLAG_TILED), windows=3, launches=50)
        tf = 2.0 * Mr * K * N / (ms * 1e-3) / 1e12
        B16 = torch.randn(N, K, device=dev, generator=gen).half()
        ms_ref = Replayer(torch, lambda i: torch.matmul(A, B16.t()), 1).run(30, 3)
        del B16
        out["prefill"][f"M{Mr}"] = {"ms": round(ms, 4), "TFLOP/s": round(tf, 1),
                                    "mfma_frac": round(tf / F16_MFMA_PEAK_TFLOPS, 4),
                                    "torch_f16_gemm_TFLOP/s": round(2.0 * Mr * K * N / (ms_ref * 1e-3) / 1e12, 1)}
    del ws
    return out


def bench_lm_head(torch, dev, gpu, Mdl, gen, kt):
    """configs[4]'s lm_head: bf16 [151936, 2560] x f32 hidden, batch 1
    (st_bf16_matvec; 778 MB, more than twice the MALL, so every call is cold)."""
    K, N = 2560, 151936
    w = (torch.randn(N, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16).view(torch.int16)
    x = torch.randn(1, K, device=dev, generator=gen)
    y = torch.empty(1, N, device=dev)
    ms = kt.run(lambda i: Mdl.bf16_matvec(gpu, x, w, y, K, N), windows=3, launches=100)
    b = N * K * 2 + K * 4 + N * 4
    del w
    return {"N": N, "K": K, "ms": round(ms, 4), "bytes": b, "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_lm_head_int4(torch, dev, gpu, Mdl, gen, kt):
    """configs[4]'s lm_head as GPTQ int4 g128 (2560 -> 151936, 200 MB;
    st_gptq_i4_matvec, the streaming kernel at 1-4 tokens), 4 cold copies
    (800 MB, three times the MALL), batch 1 and 4."""
    K, N = 2560, 151936
    TF = sta_flags_tiled()
    copies = 4
    W = [make_gptq(torch, dev, K, N, gen, gpu) for _ in range(copies)]
    out = {"N": N, "K": K}
    for Mr in (1, 4):
        x = torch.randn(Mr, K, device=dev, generator=gen)
        y = torch.empty(Mr, N, device=dev)
        ms = kt.run(lambda i: Mdl.gptq_matvec(gpu, "lm_head", x, W[i % copies][0], W[i % copies][1], y, K, N, GS,
                                              flags=TF))
        b = decode_bytes(K, N, 4, N) + (Mr - 1) * (K * 4 + N * 4)
        out[f"M{Mr}"] = {"ms": round(ms, 5), "bytes": b, "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del W
    return out


if __name__ == "__main__":
    main()
