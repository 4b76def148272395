#!/usr/bin/env python3
"""Throughput of the first-order LPV scan, forward + backward, on one MI355X.

Workload (the metric's config): a[B,T]~U(-0.99,0.99),
x[B,T]~N(0,1), y0[B]~N(0,1), upstream grad g[B,T]~N(0,1), B=64, T=65536,
fp32, generated on the CPU with torch.Generator().manual_seed(1) and copied to
the GPU before timing.

One step = the hot path over that batch: the forward scan
``torch.ops.philtorch.recur`` and the fused adjoint pass
``torch.ops.philtorch.recur_backward`` (grad w.r.t. a, x and y0).  Before
every step a 512 MiB buffer is read end to end so the 256 MB Infinity Cache
holds none of the step's operands (a read sweep, not a write: a write would
leave dirty lines whose write-back then competes with the step); the sweep
is outside the timed events.

Output: one JSON line (the driver's contract) with
  value        GSamples/s = B*T / t_step, whole job (one GPU); t_step is the
               mean over the K timed steps of one HIP-event pair around the
               forward and backward launches
  roofline     the dominant kernel (the backward scan): algorithmic bytes per
               launch (20 B/sample: read a, g, y; write grad_x, grad_a) over
               its mean HIP-event duration from a second pass that puts an
               event between the two launches, against 8 TB/s
  cpu_baseline the oracle (a C restatement of the reference CPU extension and
               its composite backward, OpenMP over the batch) on a bounded
               sample of the same workload, on this host's cores
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_HBM_GBS = 8000.0
CONFIGS = {
    # name: (B, T, dtype)
    "c1": (64, 65536, "float32"),
    "c5": (8, 1 << 24, "float32"),
    "c5_f64": (8, 1 << 24, "float64"),
}


def make_inputs(B, T, dtype, seed=1):
    import torch

    g = torch.Generator().manual_seed(seed)
    dt = getattr(torch, dtype)
    a = (torch.rand(B, T, generator=g, dtype=torch.float64) * 1.98 - 0.99).to(dt)
    x = torch.randn(B, T, generator=g, dtype=torch.float64).to(dt)
    y0 = torch.randn(B, generator=g, dtype=torch.float64).to(dt)
    gy = torch.randn(B, T, generator=g, dtype=torch.float64).to(dt)
    return a, x, y0, gy


def cpu_baseline(a, x, y0, gy, budget_s=10.0):
    """Time the oracle's forward + backward on a bounded sample of rows."""
    import numpy as np
    import oracle

    cores = len(os.sched_getaffinity(0))
    B, T = a.shape
    a_n, x_n, y0_n, g_n = (t.numpy() for t in (a, x, y0, gy))
    rows = min(B, max(cores, 1))
    # one probe on the sample to size the timed repetitions
    t0 = time.perf_counter()
    y = oracle.recur(a_n[:rows], y0_n[:rows], x_n[:rows], nthreads=cores)
    oracle.recur_bwd(a_n[:rows], y0_n[:rows], y, g_n[:rows], nthreads=cores)
    probe = time.perf_counter() - t0
    reps = int(max(1, min(50, budget_s / max(probe, 1e-6))))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        y = oracle.recur(a_n[:rows], y0_n[:rows], x_n[:rows], nthreads=cores)
        oracle.recur_bwd(a_n[:rows], y0_n[:rows], y, g_n[:rows], nthreads=cores)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {
        "value": rows * T / med / 1e9,
        "unit": "GSamples/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{rows} of {B} rows x T={T}, fwd+bwd, median of {reps} reps "
        f"(oracle/phs_oracle.c, OpenMP over rows, {cores} threads)",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c1", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-evict", action="store_true", help="keep operands cache-resident (diagnostic)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py measures one GPU only: the linear-recurrence path shards over batch rows "
            "with no communication, and this build runs and reports a single MI355X.",
            file=sys.stderr,
        )
        return 2

    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import philtorch_amd

    philtorch_amd.require_extension()
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2

    B, T, dtype = CONFIGS[args.config]
    a_c, x_c, y0_c, g_c = make_inputs(B, T, dtype)
    dev = torch.device("cuda", 0)
    a, x, y0, gy = (t.to(dev) for t in (a_c, x_c, y0_c, g_c))
    evict = None if args.no_evict else torch.ones(128 << 20, dtype=torch.float32, device=dev)
    evict_sink = torch.empty((), dtype=torch.float32, device=dev)
    recur = torch.ops.philtorch.recur
    recur_bwd = torch.ops.philtorch.recur_backward

    def evict_caches():
        if evict is not None:
            torch.sum(evict, dim=0, out=evict_sink)

    def step():
        y = recur(a, y0, x)
        return recur_bwd(a, y0, y, gy)

    for _ in range(args.warmup):
        evict_caches()
        step()
    torch.cuda.synchronize()

    # timed region: K steps, each bracketed by one event pair (the cache
    # eviction before each step stays outside the events)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for i in range(args.steps):
        evict_caches()
        ev[i][0].record()
        step()
        ev[i][1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = sum(e[0].elapsed_time(e[1]) for e in ev) / args.steps

    # roofline pass: the same steps with an event between the two kernels,
    # giving each kernel's mean launch duration on the stream it runs on
    kev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    for i in range(args.steps):
        evict_caches()
        kev[i][0].record()
        y = recur(a, y0, x)
        kev[i][1].record()
        recur_bwd(a, y0, y, gy)
        kev[i][2].record()
    torch.cuda.synchronize()
    mean_fwd = sum(e[0].elapsed_time(e[1]) for e in kev) / args.steps
    mean_bwd = sum(e[1].elapsed_time(e[2]) for e in kev) / args.steps
    samples = B * T
    esize = 4 if dtype == "float32" else 8
    bwd_bytes = 5 * esize * samples  # read a, g, y; write grad_x, grad_a
    fwd_bytes = 3 * esize * samples  # read a, x; write y
    dominant = ("backward", bwd_bytes, mean_bwd) if mean_bwd >= mean_fwd else ("forward", fwd_bytes, mean_fwd)
    achieved = dominant[1] / (dominant[2] * 1e-3) / 1e9

    result = {
        "metric": "GSamples/s fwd+bwd and % of HBM peak, 1st-order LPV scan B=64 T=65536 fp32",
        "value": round(samples / (ms_per_step * 1e-3) / 1e9, 3),
        "unit": "GSamples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if dtype == "float32" else "f64",
        "data": "synthetic (seeded torch.Generator, CPU-generated, copied to HBM before timing)",
        "config": {
            "workload": f"lpv_scan_fwd_bwd_{args.config}",
            "B": B,
            "T": T,
            "op": "philtorch::recur + philtorch::recur_backward",
            "cache_evicted_between_steps": evict is not None,
        },
        "detail": {
            "ms_fwd_kernel": round(mean_fwd, 5),
            "ms_bwd_kernel": round(mean_bwd, 5),
            "fwd_GBs_algorithmic": round(fwd_bytes / (mean_fwd * 1e-3) / 1e9, 1),
            "bwd_GBs_algorithmic": round(bwd_bytes / (mean_bwd * 1e-3) / 1e9, 1),
            "wall_s_timed_region": round(wall, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": f"scan_kernel ({dominant[0]})",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": None,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(a_c, x_c, y0_c, g_c)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
