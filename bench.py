#!/usr/bin/env python3
"""Throughput of the YOLO26 inference hot path on one MI355X.

Workload (BASELINE.json metric / configs[4]): YOLO26m end-to-end forward,
batch 64, 3x640x640 U[0,1) input, seeded Kaiming-normal weights with folded
identity BN, bfloat16 activations and weights.  One "step" is one forward of
the batch: input pack -> backbone/neck/head -> raw DetectOutput (boxes
[64, 4*8400], scores [64, 80*8400], float32), replayed from a captured
hipGraph with the input already resident in HBM.

Prints ONE JSON line.  Besides the contract fields it carries:
  roofline      the dominant kernel (largest total time per forward): its
                algorithmic FLOPs (or bytes) per launch over its average
                launch time, measured here with HIP events around each launch
                on the stream the kernels run on, against the MI355X peak
  cpu_baseline  the CPU oracle (oracle/, float32, OpenMP) on a bounded sample
                of the same workload, timed on this host
  kernels       per-kernel-symbol time / work breakdown of one forward

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vision-rs_amd"))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_profile(m, iters=3):
    """Per-launch time with events between launches (same stream as the kernels)."""
    import torch
    names = m.launch_names()
    work = m.launch_work()
    L = len(names)
    stream = torch.cuda.current_stream()
    tot = [0.0] * L
    for _ in range(iters):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(L + 1)]
        evs[0].record(stream)
        for i in range(L):
            m.run_launches(i, 1, stream.cuda_stream)
            evs[i + 1].record(stream)
        torch.cuda.synchronize()
        for i in range(L):
            tot[i] += evs[i].elapsed_time(evs[i + 1]) / iters
    per_sym = {}
    for (label, (fl, by), ms) in zip(names, work, tot):
        sym = label.split(":")[-1]
        d = per_sym.setdefault(sym, {"launches": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        d["launches"] += 1
        d["ms"] += ms
        d["flops"] += fl
        d["bytes"] += by
    layers = [{"layer": lab, "us": round(ms * 1e3, 2), "gflop": round(fl / 1e9, 3), "mb": round(by / 1e6, 2)}
              for lab, (fl, by), ms in zip(names, work, tot)]
    return per_sym, layers


def roofline_of(sym, d, dtype_peak):
    sec = d["ms"] / 1e3
    ai = d["flops"] / max(d["bytes"], 1.0)
    if d["flops"] > 0 and ai > dtype_peak * 1e12 / (PEAK_HBM_GBS * 1e9):
        ach = d["flops"] / sec / 1e12
        return {"kernel": sym, "bound": "mfma", "achieved": round(ach, 2), "peak": dtype_peak, "unit": "TFLOP/s",
                "frac": round(ach / dtype_peak, 4), "traffic": None,
                "launches_per_step": d["launches"], "avg_launch_us": round(d["ms"] * 1e3 / d["launches"], 2),
                "algorithmic_gflop_per_launch": round(d["flops"] / d["launches"] / 1e9, 4)}
    ach = d["bytes"] / sec / 1e9
    return {"kernel": sym, "bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None, "launches_per_step": d["launches"],
            "avg_launch_us": round(d["ms"] * 1e3 / d["launches"], 2),
            "algorithmic_mb_per_launch": round(d["bytes"] / d["launches"] / 1e6, 3)}


def cpu_baseline(variant, size, P, budget_s=15.0):
    """CPU oracle (float32, OpenMP) on a bounded sample of the same workload."""
    import numpy as np
    import oracle
    from oracle import yolo26 as Y
    from vrs.synth import images
    net = Y.yolo26(80, variant)
    PP = Y.Params(P, eps=1e-3)
    x1 = images(1, size, size, seed=1)
    t0 = time.perf_counter()
    net(PP, x1)
    t1 = time.perf_counter() - t0
    n = int(max(1, min(64, budget_s // max(t1, 1e-3))))
    xs = images(n, size, size, seed=2)
    t0 = time.perf_counter()
    net(PP, xs)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "images/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": f"YOLO26{variant} float32 forward of {n} image(s) at {size}x{size} in one batch "
                      f"({dt:.1f} s) on the C oracle (oracle/vrs_oracle.c, OpenMP); the reference has no CPU path"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--size", type=int, default=640)
    ap.add_argument("--variant", default="m")
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "f32"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--layers", action="store_true", help="also print the per-layer table to stderr")
    a = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every box in this build has one MI355X and the path shards by "
              "batch with no collectives (see DESIGN.md); run without --gpus or with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import vrs
    from vrs.synth import images, seeded_params

    log(f"[bench] YOLO26{a.variant} {a.dtype} bs{a.batch} {a.size}x{a.size}: building")
    torch.cuda.init()
    ctx = vrs.Context(0)
    dt = vrs.BF16 if a.dtype == "bf16" else vrs.F32
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant=a.variant, one2one=True)
    m = vrs.Model(ctx, desc, a.batch, a.size, a.size, dt, 1e-3)
    P = seeded_params(m.params(), seed=0, bn="identity")
    m.load(P)
    x = torch.from_numpy(images(a.batch, a.size, a.size, seed=0)).cuda()
    outs = m.alloc_outputs()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        m.forward(x, outs, stream.cuda_stream)
        torch.cuda.synchronize()
        m.capture(x, outs, stream.cuda_stream)
        log(f"[bench] captured {len(m.launch_names())} launches; warmup {a.warmup}")
        for _ in range(a.warmup):
            m.replay(stream.cuda_stream)
        torch.cuda.synchronize()
        log(f"[bench] timing {a.steps} steps")
        t0 = time.perf_counter()
        for _ in range(a.steps):
            m.replay(stream.cuda_stream)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        log("[bench] per-kernel profile")
        per_sym, layers = kernel_profile(m)
    ms = elapsed * 1e3 / a.steps
    value = a.batch * a.steps / elapsed
    peak = PEAK_BF16_TFLOPS if dt == vrs.BF16 else PEAK_F32_TFLOPS
    dom = max(per_sym.items(), key=lambda kv: kv[1]["ms"])
    roof = roofline_of(dom[0], dom[1], peak)
    kern = {s: {"launches": d["launches"], "ms": round(d["ms"], 4),
                "tflops": round(d["flops"] / max(d["ms"], 1e-9) / 1e9, 2),
                "gbs": round(d["bytes"] / max(d["ms"], 1e-9) / 1e6, 1)} for s, d in
            sorted(per_sym.items(), key=lambda kv: -kv[1]["ms"])}
    total_flops = sum(d["flops"] for d in per_sym.values())
    if a.layers:
        for r in layers:
            log(json.dumps(r))
    cpu = None
    if not a.no_cpu:
        log("[bench] cpu baseline (oracle)")
        cpu = cpu_baseline(a.variant, a.size, P)
    line = {
        "metric": "YOLO26 images/s @640 bs64 bf16 on 1 GPU; per-kernel % of HBM/MFMA roofline",
        "value": round(value, 1), "unit": "images/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": a.dtype, "data": "synthetic",
        "config": {"workload": f"YOLO26{a.variant} end-to-end forward {a.size}x{a.size} batch {a.batch}",
                   "batch": a.batch, "size": a.size, "variant": a.variant, "classes": 80,
                   "weights": "seeded Kaiming-normal, identity BN folded", "graph": "hipGraph replay",
                   "forward_tflop": round(total_flops / 1e12, 3),
                   "achieved_tflops_e2e": round(total_flops / (ms / 1e3) / 1e12, 1)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "kernels": kern,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
