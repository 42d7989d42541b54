#!/usr/bin/env python3
"""Benchmark of the north-star path on one MI355X.

Workload (config C2): ``d2p_amd.soft_sw(scores, gap=-1.0, temperature=1.0)``
followed by ``value.sum().backward()`` on a fresh ``requires_grad`` leaf, with
scores [256, 512, 512] ~ N(0,1) fp32 (seed 1, drawn on the CPU, copied to the
device before timing).  One step = that forward + backward; the metric is DP
cells per second (B*L1*L2 per step).

Prints one JSON line (see the keys below) with:
  * ``roofline``: the dominant kernel (largest share of the timed region),
    its algorithmic HBM bytes per launch divided by its average launch time,
    timed with HIP events recorded by the kernel library on its own stream;
  * ``step_roofline``: the whole step at 16 algorithmic bytes per cell;
  * ``cpu_baseline``: the reference's own CPU kernels (oracle/_ref, built from
    the reference sources) run in the reference's autograd call sequence on the
    host cores, on the full C2 batch.
Only one GPU is supported: ``--gpus`` above 1 exits with a message.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "DP cells/sec fwd+bwd, soft_sw B=256 512x512 fp32; achieved HBM GB/s %"
B, L1, L2 = 256, 512, 512
GAP, TEMP, SEED = -1.0, 1.0, 1

# algorithmic HBM bytes per DP cell attributed to each kernel of one step:
# the forward op must read scores (4) and write marginals (4); the autograd
# backward must read the saved marginals (4) and write grad_scores (4).  The
# scores read is attributed to sw_forward, the marginal write to sw_backward.
ALGO_BYTES_PER_CELL = {"sw_forward": 4, "sw_backward": 4, "scale_by_batch": 8}


def kernel_stats(lib):
    buf = ctypes.create_string_buffer(1 << 16)
    if lib.d2p_profile_report(buf, len(buf)) != 0:
        raise RuntimeError(lib.d2p_last_error().decode())
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, tot, mn, mx = line.split()
        out[name] = {"launches": int(cnt), "total_ms": float(tot), "avg_ms": float(tot) / int(cnt),
                     "min_ms": float(mn), "max_ms": float(mx)}
    return out


def cpu_baseline(scores_np, runs=3):
    """The reference CPU path timed on the host: per step, SoftSWRegularCPUFunction
    runs forward + backward DP in its forward and the backward DP again in its
    backward, then scales the posteriors (src/sw/torch_cpu.cpp:114-259)."""
    import numpy as np
    from oracle import oracle as O
    kind = "reference" if O.reference_available() else "port"
    k = O.get("oracle" if kind == "port" else "reference")
    cores = max(1, min(16, os.cpu_count() or 1))
    O.set_threads(cores)
    ones = np.ones((scores_np.shape[0], 1, 1), np.float32)

    def step():
        alpha, part = k.sw_forward(scores_np, None, GAP, TEMP)
        k.sw_backward(alpha, scores_np, part, None, GAP, TEMP)
        post, _, _ = k.sw_backward(alpha, scores_np, part, None, GAP, TEMP)
        return ones * post

    step()  # warm-up
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    cells = scores_np.shape[0] * scores_np.shape[1] * scores_np.shape[2]
    return {"value": cells / t, "unit": "cells/s", "cores": cores, "kind": kind,
            "sample": f"full C2 batch {list(scores_np.shape)} fwd + 2x bwd DP + scale, "
                      f"median of {runs} runs after 1 warm-up ({t:.3f} s each)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X only; --gpus {args.gpus} is not supported "
              "(the soft-DP batch would shard over B with no exchange; see DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import d2p_amd
    from d2p_amd import _ops

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(SEED)
    scores_cpu = torch.randn((B, L1, L2), generator=g, dtype=torch.float32)
    scores = scores_cpu.to(dev)

    lib = ctypes.CDLL(_ops.KERNEL_LIBRARY)
    lib.d2p_profile_report.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    lib.d2p_last_error.restype = ctypes.c_char_p

    def step():
        x = scores.detach().requires_grad_(True)
        res = d2p_amd.soft_sw(x, gap=GAP, temperature=TEMP)
        res.value.sum().backward()
        return x

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    lib.d2p_profile_reset()
    lib.d2p_profile_enable(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    lib.d2p_profile_enable(0)
    kstats = kernel_stats(lib)

    cells = B * L1 * L2
    ms_per_step = elapsed * 1e3 / args.steps
    value = cells * args.steps / elapsed
    dominant = max(kstats, key=lambda k: kstats[k]["total_ms"])
    d = kstats[dominant]
    algo_bytes = ALGO_BYTES_PER_CELL[dominant] * cells
    achieved = algo_bytes / (d["avg_ms"] * 1e-3) / 1e9
    step_gbs = 16 * cells / (ms_per_step * 1e-3) / 1e9

    out = {
        "metric": METRIC,
        "value": value,
        "unit": "cells/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) scores, generated on the CPU)",
        "config": {"workload": "C2: soft_sw linear gap, scores [256,512,512] fp32, gap=-1, "
                               "T=1, fwd (value+marginals) + value.sum().backward()",
                   "B": B, "L1": L1, "L2": L2, "gap": GAP, "temperature": TEMP,
                   "parallelism": "single GPU, one workgroup per batch element"},
        "roofline": {"bound": "hbm", "kernel": dominant, "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": None,
                     "algo_bytes_per_launch": algo_bytes,
                     "avg_launch_ms": d["avg_ms"]},
        "step_roofline": {"algo_bytes_per_step": 16 * cells, "achieved": step_gbs,
                          "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": step_gbs / HBM_PEAK_GBS},
        "kernels_ms": {k: round(v["avg_ms"], 5) for k, v in kstats.items()},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(scores_cpu.numpy())
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
