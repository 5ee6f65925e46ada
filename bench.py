#!/usr/bin/env python3
"""Benchmark of the snnk hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads: ``lif`` (config 0).  A step is one pass of
the operator over one batch of synthetic, seeded input that is resident in HBM
before timing starts.  Buffers rotate over several sets (> 512 MiB in total)
so that the 256 MiB MALL cannot serve a step from the previous step's data.

Two timed passes per workload:
  * whole job: K steps captured in a HIP graph and replayed, bracketed by
    torch.cuda.synchronize() -> ms_per_step and ``value``;
  * per kernel: K eager launches, each bracketed by a pair of HIP events on
    the launch stream -> the dominant kernel's average duration, from which
    ``roofline.achieved`` = algorithmic bytes (or ops) per launch / duration.
The CPU baseline times the oracle (a restatement of the reference's PyTorch CPU
path) on the host cores on a bounded sample and reports it beside the GPU
figure.  One JSON line is printed.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "triton-pass-analysis_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import torch  # noqa: E402

METRIC = "VGG16-SNN (T=4,B=32) images/sec; LIF HBM GB/s; binary GEMM TOPS vs peak"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 640 << 20


def cpu_threads() -> int:
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def time_cpu(fn, budget_s: float = 8.0, min_runs: int = 3) -> float:
    """Median seconds of fn() after one warm-up run, within a time budget."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 4 * budget_s:
            break
    return statistics.median(times)


def time_gpu(step, nsets: int, steps: int, warmup: int):
    """(wall seconds per step via graph replay, mean per-launch event ms)."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        step(i % nsets)
    torch.cuda.synchronize()
    # per-launch kernel durations (eager, HIP events on the launch stream)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        step(i % nsets)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    kern_ms = [a.elapsed_time(b) for a, b in ev]
    # whole job: the K steps captured once, replayed
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        step(0)  # one eager launch on the capture stream before capture
        with torch.cuda.graph(graph, stream=cap):
            for i in range(steps):
                step(i % nsets)
    stream.wait_stream(cap)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    return wall, statistics.mean(kern_ms), statistics.median(kern_ms)


# --------------------------------------------------------------------------
# LIF
# --------------------------------------------------------------------------
def bench_lif(args, dev):
    from snnk.kernels.neurons import launch_lif, THR_SCALAR
    from oracle import neurons as on

    T, B, C, H, W = 4, 32, 64, 32, 32
    NCL = B * C * H * W
    g = torch.Generator().manual_seed(0)
    x_cpu = torch.randn(T, B, C, H, W, generator=g) * 1.5
    bytes_per = T * NCL * 4 + T * NCL * 4 + NCL * 4        # x in, fp32 spikes out, final v
    nsets = max(2, math.ceil(ROTATE_BYTES / bytes_per))
    xs = [x_cpu.to(dev) for _ in range(nsets)]
    ss = [torch.empty_like(xs[0]) for _ in range(nsets)]
    vs = [torch.empty(B, C, H, W, device=dev) for _ in range(nsets)]

    def step(i):
        launch_lif(xs[i], thr=(THR_SCALAR, None, 1.0), spikes=ss[i], v_out=vs[i],
                   C=C, HW=H * W, decay=0.5, in_scale=0.5, v_reset=0.0)

    wall, kern_mean, kern_med = time_gpu(step, nsets, args.steps, args.warmup)
    # parity of what the timed graph wrote
    s_ref, v_ref, _ = on.lif_multistep(x_cpu, neuron="lif", tau=2.0)
    ok = torch.equal(ss[0].cpu(), s_ref) and torch.equal(vs[0].cpu(), v_ref)

    rec = {
        "workload": "lif", "value": bytes_per / wall / 1e9, "unit": "GB/s",
        "ms_per_step": wall * 1e3, "dtype": "f32",
        "config": {"workload": "lif_multistep_T4_B32_C64_H32_W32", "T": T,
                   "shape": [T, B, C, H, W], "tau": 2.0, "v_threshold": 1.0,
                   "reset": "hard0", "spike_dtype": "f32", "final_v": True,
                   "rotating_sets": nsets},
        "roofline": {"bound": "hbm", "kernel": "lif_kernel",
                     "achieved": bytes_per / (kern_mean * 1e-3) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": bytes_per / (kern_mean * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "traffic": None, "algorithmic_bytes": bytes_per,
                     "kernel_ms_mean": kern_mean, "kernel_ms_median": kern_med},
        "parity": ok,
    }
    if not args.no_cpu_baseline:
        nth = cpu_threads()
        torch.set_num_threads(nth)
        sec = time_cpu(lambda: on.lif_multistep(x_cpu, neuron="lif", tau=2.0))
        rec["cpu_baseline"] = {"value": bytes_per / sec / 1e9, "unit": "GB/s",
                               "cores": torch.get_num_threads(), "kind": "port",
                               "sample": "oracle.neurons.lif_multistep (torch CPU restatement "
                                         "of naive_if_lif + final v) on the full LIF config",
                               "seconds_per_call": sec}
    return rec


WORKLOADS = {"lif": bench_lif}
HEADLINE_ORDER = ["lif"]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="all", choices=["all", *WORKLOADS])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every path here runs on a single MI355X "
              f"(asked for --gpus {args.gpus}); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    names = HEADLINE_ORDER if args.workload == "all" else [args.workload]
    recs = {}
    for n in names:
        print(f"[bench] {n} ...", file=sys.stderr, flush=True)
        recs[n] = WORKLOADS[n](args, dev)
        print(f"[bench] {n}: {recs[n]['value']:.3f} {recs[n]['unit']}", file=sys.stderr,
              flush=True)
    head = recs[names[0]]
    out = {
        "metric": METRIC, "value": head["value"], "unit": head["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": head["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded torch CPU generator), random-init weights",
        "config": {**head["config"], "parallelism": "none (1 GPU)"},
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "parity": head["parity"],
        "components": {n: {k: r[k] for k in ("value", "unit", "ms_per_step", "roofline",
                                             "parity", "cpu_baseline") if k in r}
                       for n, r in recs.items() if n != names[0]},
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
