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
                (run 3 times back to back) on the stream the kernels run on,
                against the MI355X peak
  cpu_baseline  the CPU oracle (oracle/, float32, OpenMP) timed on this host
                for one warm forward of the workload's batch (64 images at
                640x640: about 12 s on 16 cores, inside the 10-30 s bound)
  kernels       per-kernel-symbol time / work breakdown of one forward
  fp8_run, fp8_forced_run
                config 5's second run (e4m3 weights and activations), each
                with `roofline_fp8`: the fp8 kernel with the largest total
                time, priced at the fp8 MFMA peak

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
PEAK_FP8_TFLOPS = 5000.0    # dense fp8 MFMA
PEAK_HBM_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


PROFILE_ITERS, PROFILE_REPS = 3, 3


def kernel_profile(m, iters=PROFILE_ITERS, reps=PROFILE_REPS):
    """Per-launch time with HIP events on the kernels' stream: each launch of
    the forward runs `reps` times back to back between two events (so the
    event records add their ~6 us once per `reps` launches), in forward
    order, `iters` times; the model's buffers hold garbage afterwards."""
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
            for _ in range(reps):
                m.run_launches(i, 1, stream.cuda_stream)
            evs[i + 1].record(stream)
        torch.cuda.synchronize()
        for i in range(L):
            tot[i] += evs[i].elapsed_time(evs[i + 1]) / iters / reps
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


TRAFFIC_MD = os.path.join(ROOT, "profiles", "yolo26m_bf16_bs64_traffic.md")
PLAN_DIR = os.path.join(ROOT, "vision-rs_amd", "plans")


def plan_path(variant, dtype_name, batch, size):
    """Committed tile plan of a workload (vrs_model_get_plan of an autotuned
    model): every run that loads it -- the bench line and each profiler pass
    -- runs the same kernels."""
    return os.path.join(PLAN_DIR, f"yolo26{variant}_{dtype_name}_bs{batch}_{size}.json")


def load_plan(path, conv_names):
    """The committed plan's tile codes, or None (then the run autotunes) when
    the file is missing or its conv names differ from the model's: a plan
    whose entries no longer line up with the convs would run valid but
    mis-tuned tiles on the wrong layers."""
    try:
        with open(path) as f:
            d = json.load(f)
    except OSError:
        return None
    rows = d.get("plan", [])
    names = [n for n, _ in rows]
    if names != list(conv_names):
        bad = next((i for i, (p, q) in enumerate(zip(names, conv_names)) if p != q), min(len(names), len(conv_names)))
        log(f"[bench] {os.path.relpath(path, ROOT)} does not match the model's convs (first difference at entry "
            f"{bad}: {len(names)} entries for {len(conv_names)} convs); autotuning instead")
        return None
    return [int(code) for _, code in rows]


def save_plan(path, m, note):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    names = [pre for pre, _, _ in m.conv_info()]
    rows = ",\n".join(f"  [{json.dumps(n)}, {c}]" for n, c in zip(names, m.get_plan()))
    with open(path, "w") as f:
        f.write(f'{{"note": {json.dumps(note)},\n "plan": [\n{rows}\n]}}\n')


def traffic_pass(a, ctx, labels_out):
    """Workload for the two rocprofv3 --pmc passes: a 1 GiB copy (counter
    calibration), model build + tile autotuning, then two eager forwards; the
    last forward's dispatches are the ones the summary reads.  --dtype fp8:
    the forced fp8 model (every eligible conv on e4m3, its committed plan),
    calibrated on the batch first."""
    import torch
    import vrs
    from vrs.synth import images, seeded_params
    src = torch.empty(2 ** 28, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    dt = {"bf16": vrs.BF16, "f32": vrs.F32, "fp8": vrs.FP8}[a.dtype]
    m = vrs.Model(ctx, vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant=a.variant, one2one=True),
                  a.batch, a.size, a.size, dt, 1e-3, autotune=2 if dt == vrs.FP8 else 1)
    # the committed tile plan, so each counter pass runs the kernels the bench line times
    dname = "fp8_forced" if dt == vrs.FP8 else a.dtype
    plan = None if a.autotune else load_plan(plan_path(a.variant, dname, a.batch, a.size),
                                              [pre for pre, _, _ in m.conv_info()])
    if plan is not None:
        m.set_plan(plan)
    log(f"[traffic] tile plan: {'committed' if plan is not None else 'autotuned'}")
    m.load(seeded_params(m.params(), seed=0, bn="identity"))
    x = torch.from_numpy(images(a.batch, a.size, a.size, seed=0)).cuda()
    outs = m.alloc_outputs()
    if dt == vrs.FP8:
        m.calibrate(x)
    m.forward(x, outs)
    m.forward(x, outs)
    torch.cuda.synchronize()
    with open(labels_out, "w") as f:
        json.dump({"labels": m.launch_names(), "work": m.launch_work(), "copy_bytes": 2 ** 30}, f)
    log(f"[traffic] {len(m.launch_names())} launches per forward -> {labels_out}")


def _pmc_rows(csv_dir, counter):
    import csv
    import glob
    rows = []
    for fn in glob.glob(os.path.join(csv_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(fn) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def traffic_summary(fetch_dir, write_dir):
    """Markdown table of HBM bytes per launch of the last forward, from the
    FETCH_SIZE and WRITE_SIZE passes (each directory holds the pass's CSV and
    the labels.json its --traffic-pass wrote), each counter scaled by what it
    read for the calibration copy.  Launches whose autotuned kernel differs
    between the two passes are left out."""
    per, labs, factors = {}, {}, {}
    for name, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        with open(os.path.join(d, "labels.json")) as f:
            meta = json.load(f)
        labels = meta["labels"]
        rows = _pmc_rows(d, name)
        cal = max(v for _, k, v in rows if "copy" in k.lower())
        factors[name] = meta["copy_bytes"] / 1024.0 / cal
        mine = [(k, v) for _, k, v in rows if k.startswith("vrs_")][-len(labels):]
        if [k for k, _ in mine] != [lab.split(":")[-1] for lab in labels]:
            raise SystemExit(f"{name}: the last {len(labels)} vrs_ dispatches do not match the forward's launches")
        per[name] = [v for _, v in mine]
        labs[name] = labels
        work = meta["work"]
    out = [f"Calibration (1 GiB device copy): FETCH_SIZE factor {factors['FETCH_SIZE']:.4f}, "
           f"WRITE_SIZE factor {factors['WRITE_SIZE']:.4f}; HBM bytes = factor x KiB x 1024.", "",
           "| launch | kernel | FETCH KiB | WRITE KiB | HBM MB | algorithmic MB | HBM / algorithmic |",
           "|---|---|---|---|---|---|---|"]
    sym_tot = {}
    skipped = 0
    for i, lab in enumerate(labs["FETCH_SIZE"]):
        if i >= len(labs["WRITE_SIZE"]) or labs["WRITE_SIZE"][i] != lab:
            skipped += 1
            continue
        fk, wk = per["FETCH_SIZE"][i], per["WRITE_SIZE"][i]
        hbm = (fk * factors["FETCH_SIZE"] + wk * factors["WRITE_SIZE"]) * 1024.0
        alg = work[i][1]
        sym = lab.split(":")[-1]
        t = sym_tot.setdefault(sym, [0, 0.0, 0.0])
        t[0] += 1
        t[1] += hbm
        t[2] += alg
        out.append(f"| {lab.rsplit(':', 1)[0]} | {sym} | {fk:.1f} | {wk:.1f} | {hbm / 1e6:.3f} | {alg / 1e6:.3f} | "
                   f"{hbm / max(alg, 1.0):.2f} |")
    out += ["", f"{skipped} launch(es) left out (different autotuned kernel in the two passes).", "",
            "| kernel | launches | HBM MB per launch | algorithmic MB per launch | HBM / algorithmic |",
            "|---|---|---|---|---|"]
    for sym, (n, hbm, alg) in sorted(sym_tot.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| {sym} | {n} | {hbm / n / 1e6:.3f} | {alg / n / 1e6:.3f} | {hbm / max(alg, 1.0):.2f} |")
    return "\n".join(out)


def mfma_summary(pmc_dir, xcds=8, simds=1024):
    """Markdown table of MFMA busy per launch of the last forward, from one
    --pmc pass of GRBM_GUI_ACTIVE and SQ_VALU_MFMA_BUSY_CYCLES over the
    --traffic-pass workload.  GRBM_GUI_ACTIVE is summed over the XCDs and
    SQ_VALU_MFMA_BUSY_CYCLES over every SIMD (one cycle per 1024 bf16 flops
    of MFMA issue), so busy = MFMA_BUSY / (GRBM_GUI_ACTIVE / xcds * simds)."""
    import csv
    import glob
    with open(os.path.join(pmc_dir, "labels.json")) as f:
        meta = json.load(f)
    labels, work = meta["labels"], meta["work"]
    disp = {}
    for fn in glob.glob(os.path.join(pmc_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(fn) as f:
            for r in csv.DictReader(f):
                d = disp.setdefault(int(r["Dispatch_Id"]), {"k": r["Kernel_Name"],
                                                             "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
                d[r["Counter_Name"]] = float(r["Counter_Value"])
    mine = [d for _, d in sorted(disp.items()) if d["k"].startswith("vrs_")][-len(labels):]
    if [d["k"] for d in mine] != [lab.split(":")[-1] for lab in labels]:
        raise SystemExit(f"the last {len(labels)} vrs_ dispatches do not match the forward's launches")
    out = [f"busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {xcds} x {simds} SIMDs); "
           "clock = GRBM_GUI_ACTIVE / XCDs / duration; TFLOP/s = algorithmic flops / duration.", "",
           "| launch | kernel | us | clock MHz | MFMA busy % | algorithmic TFLOP/s |",
           "|---|---|---|---|---|---|"]
    sym_tot = {}
    for lab, d, (fl, _) in zip(labels, mine, work):
        if fl <= 0:
            continue
        cyc = d["GRBM_GUI_ACTIVE"] / xcds
        busy = d["SQ_VALU_MFMA_BUSY_CYCLES"] / (cyc * simds)
        us = d["ns"] / 1e3
        sym = lab.split(":")[-1]
        t = sym_tot.setdefault(sym, [0, 0.0, 0.0, 0.0, 0.0])
        t[0] += 1
        t[1] += us
        t[2] += fl
        t[3] += d["SQ_VALU_MFMA_BUSY_CYCLES"] / simds
        t[4] += cyc
        out.append(f"| {lab.rsplit(':', 1)[0]} | {sym} | {us:.1f} | {cyc / us:.0f} | {100 * busy:.1f} | "
                   f"{fl / us / 1e6:.1f} |")
    out += ["", "| kernel | launches | total us | MFMA busy % (over its cycles) | algorithmic TFLOP/s |",
            "|---|---|---|---|---|"]
    for sym, (n, us, fl, bc, cyc) in sorted(sym_tot.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| {sym} | {n} | {us:.0f} | {100 * bc / cyc:.1f} | {fl / us / 1e6:.1f} |")
    return "\n".join(out)


def pmc_table(dirs, copy_bytes=2 ** 30):
    """Per (kernel, grid) medians of every counter in the given --pmc passes
    (typically over `bench.py --micro --no-cpu`), with the FETCH_SIZE and
    WRITE_SIZE passes scaled to HBM bytes by the 1 GiB calibration copy and
    MFMA busy as in mfma_summary."""
    import csv
    import glob
    import statistics
    per = {}
    for d in dirs:
        for fn in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(fn) as f:
                for r in csv.DictReader(f):
                    k = (r["Kernel_Name"], int(r["Grid_Size"]))
                    e = per.setdefault(k, {})
                    e.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
                    e.setdefault("ns:" + r["Counter_Name"], []).append(
                        int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    med = {k: {c: statistics.median(v) for c, v in e.items()} for k, e in per.items()}
    cal = {c: max(e.get(c, 0.0) for (n, _), e in med.items() if "copybuffer" in n.lower())
           for c in ("FETCH_SIZE", "WRITE_SIZE")}
    fac = {c: copy_bytes / 1024.0 / v if v else None for c, v in cal.items()}
    known = {"GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "FETCH_SIZE", "WRITE_SIZE"}
    extra = sorted({c for e in med.values() for c in e if not c.startswith("ns:") and c not in known})
    out = [f"Calibration (1 GiB device copy): FETCH_SIZE factor {fac['FETCH_SIZE'] or 0:.4f}, "
           f"WRITE_SIZE factor {fac['WRITE_SIZE'] or 0:.4f}.", "",
           "| kernel | grid | us | MFMA busy % | HBM read MB | HBM write MB | HBM GB/s |" +
           "".join(f" {c} |" for c in extra), "|---|---|---|---|---|---|---|" + "---|" * len(extra)]
    for (name, grid), e in sorted(med.items()):
        if not name.startswith("vrs_"):
            continue
        us = [e[c] / 1e3 for c in e if c.startswith("ns:")]
        us = statistics.median(us) if us else 0.0
        busy = ""
        if "SQ_VALU_MFMA_BUSY_CYCLES" in e and e.get("GRBM_GUI_ACTIVE"):
            busy = f"{100 * e['SQ_VALU_MFMA_BUSY_CYCLES'] / (e['GRBM_GUI_ACTIVE'] / 8 * 1024):.1f}"
        rd = e["FETCH_SIZE"] * fac["FETCH_SIZE"] * 1024 / 1e6 if "FETCH_SIZE" in e and fac["FETCH_SIZE"] else None
        wr = e["WRITE_SIZE"] * fac["WRITE_SIZE"] * 1024 / 1e6 if "WRITE_SIZE" in e and fac["WRITE_SIZE"] else None
        gbs = f"{(rd + wr) / us * 1e3:.0f}" if rd is not None and wr is not None and us else ""
        out.append(f"| {name} | {grid} | {us:.1f} | {busy} | {'' if rd is None else f'{rd:.2f}'} | "
                   f"{'' if wr is None else f'{wr:.2f}'} | {gbs} |" +
                   "".join(f" {e[c]:.4g} |" if c in e else " |" for c in extra))
    return "\n".join(out)


def layers_summary(path, key="layer"):
    """Markdown table of the per-layer lines `bench.py --layers` writes to
    stderr (key "layer": the bf16 run; "layer8": the forced fp8 run): each
    launch's time (HIP events around every launch of one eager forward,
    averaged over 3), its algorithmic work and the fraction of its bounding
    roofline (MFMA -- fp8 peak for the fp8 kernels, bf16 peak for the others
    -- or HBM, whichever the work's arithmetic intensity puts it under)."""
    rows = []
    with open(path) as f:
        for line in f:
            if line.startswith('{"%s"' % key):
                rows.append(json.loads(line))
    out = ["| launch | kernel | us | GFLOP | MB | bound | achieved | roofline frac |", "|---|---|---|---|---|---|---|---|"]
    tot = ideal = 0.0
    for r in rows:
        lab, sym = r[key].rsplit(":", 1)
        peak_tflops = PEAK_FP8_TFLOPS if "_fp8_" in sym else PEAK_BF16_TFLOPS
        ridge = peak_tflops * 1e12 / (PEAK_HBM_GBS * 1e9)
        fl, mb, us = r["gflop"] * 1e9, r["mb"] * 1e6, r["us"]
        if fl > 0 and fl / max(mb, 1.0) > ridge:
            ach, bound, frac = f"{fl / us / 1e6:.0f} TFLOP/s", "mfma", fl / us / 1e6 / peak_tflops
        else:
            ach, bound, frac = f"{mb / us / 1e3:.0f} GB/s", "hbm", mb / us / 1e3 / PEAK_HBM_GBS
        tot += us
        ideal += max(fl / (peak_tflops * 1e12), mb / (PEAK_HBM_GBS * 1e9)) * 1e6
        out.append(f"| {lab} | {sym} | {us:.1f} | {r['gflop']:.2f} | {r['mb']:.1f} | {bound} | {ach} | {frac:.3f} |")
    out += ["", f"{len(rows)} launches, {tot:.0f} us in sum (eager, one launch at a time; the hipGraph replay runs "
                f"the same launches, the Detect head's chains as parallel branches beside the trunk); at the MI355X "
                f"peaks the same work needs "
                f"{ideal:.0f} us."]
    return "\n".join(out)


def trace_summary(trace_dir, bench_json, steps, profile_iters=PROFILE_ITERS * PROFILE_REPS):
    """Per-kernel launch durations from a `rocprofv3 --kernel-trace` run of
    `bench.py --no-cpu --no-fp8 --steps S` against that run's own JSON line:
    the last profile_iters x launches dispatches of each kernel are bench.py's
    per-kernel profile (kernel_profile: the source of `kernels` and
    `roofline.avg_launch_us`), the steps x launches before them the timed
    hipGraph replays (the Detect head's chains as parallel branches beside the trunk)."""
    import csv
    import glob
    with open(bench_json) as f:
        d = json.loads([l for l in f if l.startswith("{")][-1])
    disp = []
    for fn in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(fn) as f:
            for r in csv.DictReader(f):
                disp.append((int(r["Start_Timestamp"]), r["Kernel_Name"],
                             (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    disp.sort()
    out = ["| kernel | launches per forward | bench.py avg us (HIP events) | rocprofv3 avg us, same launches | "
           "rocprofv3 avg us, timed graph replays |", "|---|---|---|---|---|"]
    for sym, k in d["kernels"].items():
        n = k["launches"]
        durs = [us for _, name, us in disp if name == sym]
        prof = durs[-profile_iters * n:]
        rep = durs[-(profile_iters + steps) * n:-profile_iters * n]
        out.append(f"| {sym} | {n} | {k['ms'] * 1e3 / n:.1f} | {sum(prof) / max(len(prof), 1):.1f} | "
                   f"{sum(rep) / max(len(rep), 1):.1f} |")
    r = d["roofline"]
    out += ["", f"bench.py line: {d['value']} images/s, {d['ms_per_step']} ms per forward; dominant kernel "
                f"{r['kernel']} avg_launch_us {r['avg_launch_us']}, {r['achieved']} {r['unit']} = {r['frac']:.1%} "
                f"of {r['peak']}."]
    return "\n".join(out)


def traffic_lookup(sym, names):
    """HBM bytes per launch of `sym` in this forward, from the committed
    per-launch table (launches whose layer ran the same kernel there)."""
    try:
        with open(TRAFFIC_MD) as f:
            table = {}
            for line in f:
                c = [x.strip() for x in line.strip().strip("|").split("|")]
                if len(c) == 7 and c[1].startswith("vrs_"):
                    table[(c[0], c[1])] = float(c[4]) * 1e6
    except OSError:
        return None, 0
    mine = [lab.rsplit(":", 1)[0] for lab in names if lab.split(":")[-1] == sym]
    got = [table[(l, sym)] for l in mine if (l, sym) in table]
    if not got:
        return None, 0
    return sum(got) / len(got), len(got) / len(mine)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(variant, size, batch, P, max_images=64):
    """CPU oracle (float32, OpenMP over the host's cores): one warm forward of
    the whole workload batch (the CPU baseline is one warm iteration at bs64),
    capped at max_images."""
    import oracle
    from oracle import yolo26 as Y
    from vrs.synth import images
    net = Y.yolo26(80, variant)
    PP = Y.Params(P, eps=1e-3)
    net(PP, images(1, size, size, seed=1))   # warm: page in weights, spin up the thread pool
    n = min(batch, max_images)
    xs = images(n, size, size, seed=2)
    t0 = time.perf_counter()
    net(PP, xs)
    dt = time.perf_counter() - t0
    threads = oracle.num_threads()
    return {"value": round(n / dt, 3), "unit": "images/s", "cores": threads, "kind": "port",
            "sample": f"one warm YOLO26{variant} float32 forward of a batch of {n} image(s) at {size}x{size} "
                      f"({dt:.1f} s) on the C oracle (oracle/vrs_oracle.c); the reference has no CPU path",
            "batch": n, "seconds": round(dt, 2), "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "omp_threads": threads, "compiler": oracle.build_info()}


def yolo26n_latency(ctx, iters=200):
    """The reference's own published configuration as context: YOLO26n,
    batch 1, float32, 640x640 (docs/optimisation.md:3-4,14: 9.07 ms/img
    end to end with H2D and D2H, 8.41 ms of GPU kernels, on an RTX 5070; its
    bench loop is examples/yolo26.rs:3087-3162).  GPU-only: mean of `iters`
    graph replays with the input resident.  End to end: per image, a pinned
    host input copied in, the replay, and both outputs copied back to pinned
    host memory, synchronised each time."""
    import torch
    import vrs
    from vrs.synth import images, seeded_params
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="n", one2one=True)
    m = vrs.Model(ctx, desc, 1, 640, 640, vrs.F32, 1e-3)
    m.load(seeded_params(m.params(), seed=0, bn="identity"))
    host_x = torch.from_numpy(images(1, 640, 640, seed=3)).pin_memory()
    x = host_x.cuda()
    outs = m.alloc_outputs()
    host_outs = [torch.empty(o.shape, dtype=o.dtype, pin_memory=True) for o in outs]
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        m.forward(x, outs, st.cuda_stream)
        torch.cuda.synchronize()
        m.capture(x, outs, st.cuda_stream)
        for _ in range(10):
            m.replay(st.cuda_stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            m.replay(st.cuda_stream)
        torch.cuda.synchronize()
        gpu_ms = (time.perf_counter() - t0) * 1e3 / iters
        t0 = time.perf_counter()
        for _ in range(iters):
            x.copy_(host_x, non_blocking=True)
            m.replay(st.cuda_stream)
            for h, o in zip(host_outs, outs):
                h.copy_(o, non_blocking=True)
            st.synchronize()
        e2e_ms = (time.perf_counter() - t0) * 1e3 / iters
    n_launch = len(m.launch_names())
    m.close()
    return {"workload": "YOLO26n end-to-end forward 640x640 batch 1, float32", "gpu_ms": round(gpu_ms, 3),
            "e2e_ms_with_h2d_d2h": round(e2e_ms, 3), "launches": n_launch,
            "reference": "9.07 ms/img end to end, 8.41 ms GPU kernels, RTX 5070 (docs/optimisation.md:14,24)",
            "note": "context only: the reference's one published configuration, not BASELINE's metric"}


def _time_launches(fn, n_sets, iters=20, warmup=3, queued=False):
    """Average GPU time of fn(set_index) (one kernel launch each) on the current
    stream.  queued=False: events around every launch.  queued=True (calls
    that only enqueue GPU work): the launches are queued behind a GPU spin
    longer than the host takes to issue them, then run back to back between
    one event pair -- the GPU never waits for the host and no event sits
    between two launches (per-launch event pairs add ~2 us to each)."""
    import torch
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i % n_sets)
    torch.cuda.synchronize()
    if queued:
        t0 = time.perf_counter()
        for i in range(3):
            fn(i % n_sets)
        issue_s = (time.perf_counter() - t0) / 3   # host time to issue one call
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        torch.cuda._sleep(1 << 20)
        e1.record(stream)
        torch.cuda.synchronize()
        spin_s = e0.elapsed_time(e1) / 1e3 / (1 << 20)   # seconds per spin cycle
        torch.cuda._sleep(int(min(2 * iters * issue_s + 1e-3, 0.5) / spin_s))
        e0.record(stream)
        for i in range(iters):
            fn(i % n_sets)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters  # ms
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for i, (e0, e1) in enumerate(evs):
        e0.record(stream)
        fn(i % n_sets)
        e1.record(stream)
    torch.cuda.synchronize()
    return sum(e0.elapsed_time(e1) for e0, e1 in evs) / iters  # ms


def _cpu_ms(fn, reps=1):
    """Wall time of fn() on the CPU oracle (float32 restatement, OpenMP over
    the host's cores), after one warm call: the reference has no CPU path, so
    this is the CPU baseline timed beside each GPU config."""
    fn()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    return (time.perf_counter() - t0) / reps * 1e3


def micro(ctx, emit, cpu=True):
    """BASELINE configs 2-4 as isolated kernels (bf16 unless stated), each with
    the CPU oracle's time for the same config beside it (cpu_ms; cpu=False
    skips it)."""
    import numpy as np
    import torch
    import vrs
    from vrs.synth import seeded_params
    if cpu:
        import oracle
        cores = oracle.num_threads()
    dev = "cuda"
    MALL = 256 * 2 ** 20  # Infinity Cache: rotate buffer sets beyond it for HBM-bound kernels

    def sets_for(nbytes):
        return max(1, int(np.ceil(2 * MALL / max(nbytes, 1))))

    # copy of a known size: calibrates FETCH_SIZE / WRITE_SIZE counter readings
    src = torch.empty(2 ** 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    emit({"config": "calibration copy", "bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4})
    del src, dst

    # ---- config 3: conv microbench, B=32, folded BN + SiLU epilogue ----------
    convs = [("c3a 3x3 s1 128->128 @80", 128, 128, 80, 3, 1), ("c3b 3x3 s2 256->512 @40", 256, 512, 40, 3, 2),
             ("c3d 1x1 1024->512 @20", 1024, 512, 20, 1, 1)]
    B = 32
    rng = np.random.default_rng(0)
    for name, cin, cout, hw, k, s in convs:
        ho = (hw + 2 * (k // 2) - k) // s + 1
        wt = (rng.standard_normal((cout, cin, k, k)) * np.sqrt(2.0 / (cin * k * k))).astype(np.float32)
        wp = torch.from_numpy(vrs.pack_conv_weight(wt, 1, cin, vrs.BF16)).to(dev)
        sc = torch.full((cout,), 1.0 / np.sqrt(1.001), device=dev)
        sh = torch.zeros(cout, device=dev)
        in_b, out_b = B * hw * hw * cin * 2, B * ho * ho * cout * 2
        n_sets = sets_for(in_b + out_b)
        xs = [torch.nn.functional.silu(torch.randn(B, hw, hw, cin, device=dev)).to(torch.bfloat16) for _ in range(n_sets)]
        ys = [torch.empty(B, ho, ho, cout, dtype=torch.bfloat16, device=dev) for _ in range(n_sets)]
        flops = 2.0 * B * ho * ho * cout * cin * k * k
        best = None
        for tile in [vrs.TILE_128x128, vrs.TILE_128x128 | vrs.TILE_K32, vrs.TILE_256x128, vrs.TILE_256x256, vrs.TILE_128x256,
                     vrs.TILE_64x256]:
            try:
                f = lambda i, t=tile: ctx.conv2d(vrs.nhwc(xs[i]), wp, sc, sh, vrs.nhwc(ys[i]), k, s, 1, vrs.ACT_SILU,
                                                  None, vrs.BF16, tile=t)
                ms = _time_launches(f, n_sets, queued=True)
            except vrs.VrsError:
                continue
            if best is None or ms < best[1]:
                best = (tile, ms)
        tile, ms = best
        line = {"config": name, "batch": B, "us": round(ms * 1e3, 2), "tile": tile,
                "gflop": round(flops / 1e9, 2), "tflops": round(flops / ms / 1e9, 1),
                "frac_mfma": round(flops / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
                "mb": round((in_b + out_b + cout * cin * k * k * 2) / 1e6, 1), "buffer_sets": n_sets}
        if cpu:
            xc = rng.standard_normal((B, cin, hw, hw)).astype(np.float32)
            scc = np.full(cout, 1.0 / np.sqrt(1.001), np.float32)
            line["cpu_ms"] = round(_cpu_ms(lambda: oracle.affine_act(oracle.conv2d(xc, wt, s, k // 2), scc,
                                                                       np.zeros(cout, np.float32), 1)), 1)
            line["cpu_cores"] = cores
        emit(line)
        del xs, ys

    # (c) depthwise 3x3 512 @20x20, HBM-bound; plus the YOLO26m head's largest
    # depthwise shape (256 ch @80x80, batch 64) where launch latency matters less
    for name, C, hw, bb in (("c3c dw3x3 512 @20", 512, 20, B), ("dw3x3 256 @80 (YOLO26m head, bs64)", 256, 80, 64)):
        wdw = (rng.standard_normal((C, 1, 3, 3)) * np.sqrt(2.0 / 9)).astype(np.float32)
        wp = torch.from_numpy(vrs.pack_conv_weight(wdw, C, 1, vrs.BF16)).to(dev)
        sc = torch.full((C,), 1.0 / np.sqrt(1.001), device=dev)
        sh = torch.zeros(C, device=dev)
        nb = 2 * bb * hw * hw * C * 2
        n_sets = sets_for(nb)
        xs = [torch.nn.functional.silu(torch.randn(bb, hw, hw, C, device=dev)).to(torch.bfloat16)
              for _ in range(n_sets)]
        ys = [torch.empty(bb, hw, hw, C, dtype=torch.bfloat16, device=dev) for _ in range(n_sets)]
        ms = _time_launches(lambda i: ctx.conv2d(vrs.nhwc(xs[i]), wp, sc, sh, vrs.nhwc(ys[i]), 3, 1, C,
                                                 vrs.ACT_SILU, None, vrs.BF16), n_sets, iters=60, queued=True)
        line = {"config": name, "batch": bb, "us": round(ms * 1e3, 2), "mb": round(nb / 1e6, 2),
                "gbs": round(nb / ms / 1e6, 1), "frac_hbm": round(nb / ms / 1e6 / PEAK_HBM_GBS, 4),
                "buffer_sets": n_sets}
        if cpu:
            xc = rng.standard_normal((bb, C, hw, hw)).astype(np.float32)
            scc = np.full(C, 1.0 / np.sqrt(1.001), np.float32)
            line["cpu_ms"] = round(_cpu_ms(lambda: oracle.affine_act(oracle.conv2d(xc, wdw, 1, 1, groups=C), scc,
                                                                       np.zeros(C, np.float32), 1)), 1)
            line["cpu_cores"] = cores
        emit(line)
        del xs, ys

    # ---- config 2: isolated PSA attention block, B=32, 256 ch @20x20, 4 heads --
    desc = vrs.block(vrs.BLOCK_PSA_ATTN, 256, 256, heads=4)
    m = vrs.Model(ctx, desc, 32, 20, 20, vrs.BF16, 1e-3)
    P = seeded_params(m.params(), seed=0)
    for nme in P:  # N(0, 1/sqrt(C)) weights
        if P[nme].ndim == 4:
            P[nme] = (np.random.default_rng(1).standard_normal(P[nme].shape) / 16.0).astype(np.float32)
    m.load(P)
    x = torch.randn(32, 256, 20, 20, device=dev)
    outs = m.forward(x)
    torch.cuda.synchronize()
    names = m.launch_names()
    work = m.launch_work()
    ai = [i for i, n in enumerate(names) if "psa_attn" in n][0]
    ms_core = _time_launches(lambda i: m.run_launches(ai, 1), 1, iters=50, queued=True)
    ms_blk = _time_launches(lambda i: m.run_launches(1, len(names) - 2), 1, iters=20,  # qkv..proj, no pack/unpack
                            queued=True)
    core_fl = work[ai][0]
    blk_fl = sum(w[0] for w in work[1:len(names) - 1])
    line = {"config": "c2 psa attention B32 256ch 20x20 4 heads", "core_us": round(ms_core * 1e3, 2),
            "core_gflop": round(core_fl / 1e9, 3), "core_tflops": round(core_fl / ms_core / 1e9, 1),
            "core_frac_mfma": round(core_fl / ms_core / 1e9 / PEAK_BF16_TFLOPS, 4),
            "block_us": round(ms_blk * 1e3, 2), "block_gflop": round(blk_fl / 1e9, 3),
            "block_tflops": round(blk_fl / ms_blk / 1e9, 1)}
    if cpu:  # the attention core (softmax(q k^T * kd^-0.5) v) on the oracle
        qkvc = np.random.default_rng(2).standard_normal((32, 4 * 128, 20, 20)).astype(np.float32)
        line["cpu_core_ms"] = round(_cpu_ms(lambda: oracle.psa_attention(qkvc, 4, 32, 64)), 1)
        line["cpu_cores"] = cores
    emit(line)
    m.close()

    # ---- config 4: MSDA, fp32 value, B=8, Q=300, 8 heads, 4 levels x 4 points ----
    shapes = [(80, 80), (40, 40), (20, 20), (10, 10)]
    Bq, Q, Hh, L, Pp = 8, 300, 8, 4, 4
    S = sum(h * w for h, w in shapes)
    vbytes = Bq * S * Hh * 32 * 4
    n_sets = sets_for(vbytes)
    vals = [torch.randn(Bq, S, Hh, 32, device=dev) for _ in range(n_sets)]
    ref = torch.rand(Bq, Q, 2, device=dev)
    off = torch.randn(Bq, Q, Hh, L, Pp, 2, device=dev) * 0.05
    attw = torch.softmax(torch.randn(Bq, Q, Hh, L * Pp, device=dev), -1).reshape(Bq, Q, Hh, L, Pp).contiguous()
    out = torch.empty(Bq, Q, Hh * 32, device=dev)
    ms = _time_launches(lambda i: ctx.msda(vals[i], shapes, ref, off, attw, out), n_sets, iters=60, queued=True)
    comp = vbytes + ref.numel() * 4 + off.numel() * 4 + attw.numel() * 4 + out.numel() * 4
    issued = Bq * Q * Hh * L * Pp * 4 * 32 * 4
    line = {"config": "c4 msda B8 Q300 8h 4L 4P fp32", "us": round(ms * 1e3, 2),
            "compulsory_mb": round(comp / 1e6, 2), "gbs_compulsory": round(comp / ms / 1e6, 1),
            "frac_hbm": round(comp / ms / 1e6 / PEAK_HBM_GBS, 4), "issued_gather_mb": round(issued / 1e6, 1),
            "buffer_sets": n_sets}
    if cpu:
        vc, rc_, oc, ac = (t.cpu().numpy() for t in (vals[0], ref, off, attw))
        line["cpu_ms"] = round(_cpu_ms(lambda: oracle.msda(vc, shapes, rc_, oc, ac), reps=3), 2)
        line["cpu_cores"] = cores
    emit(line)

    # ---- letterbox preprocessing: 64 RGB8 1280x720 frames -> [64,3,640,640] f32 ----
    nimg, (lw, lh), S = 64, (1280, 720), 640
    src_b = nimg * lw * lh * 3
    out_b = nimg * 3 * S * S * 4
    n_sets = sets_for(src_b + out_b)
    srcs = [torch.randint(0, 256, (src_b,), dtype=torch.uint8, device=dev) for _ in range(n_sets)]
    outs_lb = [torch.empty(nimg, 3, S, S, device=dev) for _ in range(n_sets)]
    offs = [i * lw * lh * 3 for i in range(nimg)]
    ms = _time_launches(lambda i: ctx.letterbox(srcs[i], offs, [(lw, lh)] * nimg, S, out=outs_lb[i]), n_sets, iters=30)
    line = {"config": "letterbox 64x 1280x720 RGB8 -> 640 f32 NCHW", "us": round(ms * 1e3, 2),
            "mb": round((src_b + out_b) / 1e6, 1), "gbs": round((src_b + out_b) / ms / 1e6, 1),
            "frac_hbm": round((src_b + out_b) / ms / 1e6 / PEAK_HBM_GBS, 4), "buffer_sets": n_sets}
    if cpu:  # the oracle is single-threaded per frame: 4 frames timed, scaled to 64
        frame = srcs[0][: lw * lh * 3].cpu().numpy().reshape(lh, lw, 3)
        per = _cpu_ms(lambda: oracle.letterbox(frame, S), reps=4)
        line["cpu_ms"] = round(per * nimg, 1)
        line["cpu_sample"] = "4 frames timed one at a time (1 thread), x64"
        line["cpu_cores"] = 1
    emit(line)

    # ---- Detect post-process (decode, score, stable top-k) on the bs64 640 outputs ----
    B, nc, A, max_det = 64, 80, 8400, 300
    g = torch.Generator(device=dev).manual_seed(0)
    boxes = torch.rand(B, 4 * A, device=dev, generator=g) * 8.0
    # class logits ~ N(-6, 1.5): about 4 % of the anchors have a class above the
    # 0.25 threshold, a few hundred candidates per image for the top 300
    scores = torch.randn(B, nc * A, device=dev, generator=g) * 1.5 - 6.0
    ws = torch.empty(64 * 2 ** 20, dtype=torch.uint8, device=dev)
    pp = ctx.detect_postprocess(boxes, scores, nc, 640, 640, (8, 16, 32), 0.25, max_det, workspace=ws)
    ms = _time_launches(lambda i: ctx.detect_postprocess(boxes, scores, nc, 640, 640, (8, 16, 32), 0.25, max_det,
                                                         outs=pp, workspace=ws), 1, iters=30)
    in_b = (boxes.numel() + scores.numel()) * 4
    line = {"config": "detect post-process bs64 640 (8400 anchors, 80 classes, thr 0.25, top 300)",
            "us": round(ms * 1e3, 2), "mb": round(in_b / 1e6, 1), "gbs": round(in_b / ms / 1e6, 1),
            "frac_hbm": round(in_b / ms / 1e6 / PEAK_HBM_GBS, 4),
            "detections_per_image": round(float(pp[0].float().mean()), 1)}
    if cpu:
        bc, scc = boxes.cpu().numpy(), scores.cpu().numpy()
        line["cpu_ms"] = round(_cpu_ms(lambda: oracle.detect_postprocess(bc, scc, nc, 640, 640, (8, 16, 32), 0.25,
                                                                          max_det), reps=3), 2)
        line["cpu_cores"] = cores
    emit(line)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--size", type=int, default=640)
    ap.add_argument("--variant", default="m")
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "f32", "fp8"])
    ap.add_argument("--no-fp8", action="store_true", help="skip the fp8 second run (BASELINE config 5)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--streams", type=int, default=3,
                    help="capture streams: the trunk plus side streams for the Detect head's six chains, all in "
                         "one graph whose parallel branches replay on parallel hardware queues (1 = serial)")
    ap.add_argument("--layers", action="store_true", help="also print the per-layer table to stderr")
    ap.add_argument("--autotune", action="store_true",
                    help="autotune the tiles instead of loading the committed plan (vision-rs_amd/plans/)")
    ap.add_argument("--save-plans", action="store_true",
                    help="write the tile plans this run used to vision-rs_amd/plans/ (or --plan-dir)")
    ap.add_argument("--plan-dir", default=None,
                    help="directory --save-plans writes to (e.g. a scratch folder on a remote box)")
    ap.add_argument("--no-micro", action="store_true",
                    help="skip the isolated BASELINE configs 2-4 in the default line's `micro` object")
    ap.add_argument("--micro", action="store_true",
                    help="instead: BASELINE configs 2-4 as isolated kernels, one JSON line each")
    ap.add_argument("--traffic-pass", metavar="LABELS_JSON",
                    help="instead: the workload profiled by the rocprofv3 --pmc traffic passes")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="instead (no GPU): print the per-launch HBM traffic table from the two passes")
    ap.add_argument("--mfma-summary", metavar="PMC_DIR",
                    help="instead (no GPU): print the per-launch MFMA busy table from a GRBM_GUI_ACTIVE + "
                         "SQ_VALU_MFMA_BUSY_CYCLES pass over the --traffic-pass workload")
    ap.add_argument("--layers-summary", metavar="STDERR_FILE",
                    help="instead (no GPU): per-layer roofline table from a --layers run's stderr")
    ap.add_argument("--layers-key", default="layer",
                    help="with --layers-summary: layer (the bf16 run) or layer8 (the forced fp8 run)")
    ap.add_argument("--trace-summary", nargs=2, metavar=("TRACE_DIR", "BENCH_JSON"),
                    help="instead (no GPU): per-kernel durations of a rocprofv3 --kernel-trace run of "
                         "bench.py --no-cpu --no-fp8 against its JSON line (pass the run's --steps)")
    ap.add_argument("--pmc-table", nargs="+", metavar="PMC_DIR",
                    help="instead (no GPU): per-kernel medians of the counters in these --pmc passes")
    a = ap.parse_args()
    if a.layers_summary:
        print(layers_summary(a.layers_summary, a.layers_key))
        return 0
    if a.trace_summary:
        print(trace_summary(*a.trace_summary, steps=a.steps))
        return 0
    if a.pmc_table:
        print(pmc_table(a.pmc_table))
        return 0
    if a.traffic_summary:
        print(traffic_summary(*a.traffic_summary))
        return 0
    if a.mfma_summary:
        print(mfma_summary(a.mfma_summary))
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: every box in this build has one MI355X and the path shards by "
              "batch with no collectives; run without --gpus or with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import vrs
    from vrs.synth import images, seeded_params

    torch.cuda.init()
    ctx = vrs.Context(0)
    if a.micro:
        micro(ctx, lambda d: print(json.dumps(d), flush=True), cpu=not a.no_cpu)
        return 0
    if a.traffic_pass:
        traffic_pass(a, ctx, a.traffic_pass)
        return 0
    dt = {"bf16": vrs.BF16, "f32": vrs.F32, "fp8": vrs.FP8}[a.dtype]
    desc = vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant=a.variant, one2one=True)
    x = torch.from_numpy(images(a.batch, a.size, a.size, seed=0)).cuda()
    stream = torch.cuda.Stream()

    plans_used = {}

    def run(dtype, tune_mode=1):
        """Build, (calibrate,) capture and time one forward per step; returns
        (model, elapsed seconds, per-kernel, per-layer).  Tiles: the committed
        plan of the workload if there is one (and --autotune is not given),
        else autotuned (tune_mode 2: fp8 forced on every eligible conv)."""
        dname = ["f32", "bf16", "fp8"][dtype] + ("_forced" if tune_mode == 2 else "")
        log(f"[bench] YOLO26{a.variant} {dname} bs{a.batch} {a.size}x{a.size}: building")
        m = vrs.Model(ctx, desc, a.batch, a.size, a.size, dtype, 1e-3, autotune=tune_mode)
        pp = plan_path(a.variant, dname, a.batch, a.size)
        plan = None if a.autotune else load_plan(pp, [pre for pre, _, _ in m.conv_info()])
        if plan is not None:
            m.set_plan(plan)
            plans_used[dname] = os.path.relpath(pp, ROOT)
        else:
            plans_used[dname] = "autotuned in this run"
        m.load(P)
        if a.save_plans:
            save_plan(os.path.join(a.plan_dir, os.path.basename(pp)) if a.plan_dir else pp, m, f"YOLO26{a.variant} {dname} batch {a.batch} {a.size}x{a.size}: per-conv tile codes "
                             "(vrs_model_get_plan; | 0x10000 = fp8) from an autotuned MI355X run")
        m.set_streams(a.streams)
        outs = m.alloc_outputs()
        with torch.cuda.stream(stream):
            if dtype == vrs.FP8:
                m.calibrate(x, stream.cuda_stream)   # activation scales from this batch (bf16 pass)
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
            el = time.perf_counter() - t0
            log("[bench] per-kernel profile")
            ps, ly = kernel_profile(m)
        return m, el, ps, ly

    P = seeded_params(vrs.Model(None, desc, a.batch, a.size, a.size).params(), seed=0, bn="identity")
    m, elapsed, per_sym, layers = run(dt)
    fp8_run = fp8_forced = None

    def fp8_summary(m8, el8, ps8, note):
        top = sorted(ps8.items(), key=lambda kv: -kv[1]["ms"])[:4]
        # the fp8 kernel with the largest total time per forward, priced at the
        # fp8 MFMA peak (HBM traffic: profiles/yolo26m_fp8_forced_bs64_traffic.md)
        f8k = [kv for kv in ps8.items() if "_fp8_" in kv[0]]
        roof8 = roofline_of(*max(f8k, key=lambda kv: kv[1]["ms"]), PEAK_FP8_TFLOPS) if f8k else None
        ios = [m8.conv_io(i) for i in range(len(m8.conv_info()))]
        return {"value": round(a.batch * a.steps / el8, 1), "unit": "images/s",
                "ms_per_step": round(el8 * 1e3 / a.steps, 3),
                "fp8_convs": sum(1 for _, f8, _ in m8.conv_info() if f8), "convs": len(m8.conv_info()),
                "e4m3_inputs": sum(io.x_e4m3 for io in ios), "e4m3_outputs": sum(io.y_e4m3 for io in ios),
                "note": note, "roofline_fp8": roof8,
                "kernels": {s: {"launches": d["launches"], "ms": round(d["ms"], 4),
                                "tflops": round(d["flops"] / max(d["ms"], 1e-9) / 1e9, 2)} for s, d in top}}

    if dt == vrs.BF16 and not a.no_fp8:
        m8, el8, ps8, _ = run(vrs.FP8)
        fp8_run = fp8_summary(m8, el8, ps8,
                              "e4m3 weights (per-channel absmax/448) and e4m3 activations (per-tensor power-of-two "
                              "step calibrated on this batch) on the fp8 MFMA for convs with Cin % 64 == 0 whose "
                              "fastest fp8 tile beats their fastest bf16 tile (per-layer plan); the rest bf16; "
                              "activations stored as e4m3 where every reader and writer is an fp8 conv, else bf16")
        m8.close()
        m8, el8, ps8, ly8 = run(vrs.FP8, tune_mode=2)
        if a.layers:
            for r in ly8:
                r = dict(r)
                log(json.dumps({"layer8": r.pop("layer"), **r}))
        fp8_forced = fp8_summary(m8, el8, ps8,
                                 "every conv with Cin % 64 == 0 forced onto the fp8 MFMA (fastest fp8 tile per "
                                 "layer), the rest (stem, depthwise) bf16; activations stored as e4m3 where every "
                                 "reader and writer is an fp8 conv, else bf16")
        m8.close()
    micro_summary = None
    if not a.no_micro:
        log("[bench] isolated BASELINE configs 2-4")
        rows = []
        micro(ctx, rows.append, cpu=not a.no_cpu)
        micro_summary = {}
        for r in rows:
            cfg = r.get("config", "")
            if cfg.startswith(("c2", "c3", "c4")):
                key = cfg.split()[0]
                us = r.get("us", r.get("core_us"))
                frac = r.get("frac_mfma", r.get("frac_hbm", r.get("core_frac_mfma")))
                micro_summary[key] = {"config": cfg, "us": us, "frac": frac,
                                      "bound": "hbm" if "frac_hbm" in r else "mfma",
                                      "cpu_ms": r.get("cpu_ms", r.get("cpu_core_ms"))}
                if key == "c2":
                    micro_summary[key]["block_us"] = r.get("block_us")
    context = None
    if not a.no_micro:
        log("[bench] YOLO26n bs1 float32 latency (the reference's published configuration)")
        context = {"yolo26n_bs1_fp32": yolo26n_latency(ctx)}
    ms = elapsed * 1e3 / a.steps
    value = a.batch * a.steps / elapsed
    peak = PEAK_BF16_TFLOPS if dt == vrs.BF16 else PEAK_FP8_TFLOPS if dt == vrs.FP8 else PEAK_F32_TFLOPS
    dom = max(per_sym.items(), key=lambda kv: kv[1]["ms"])
    roof = roofline_of(dom[0], dom[1], peak)
    if a.variant == "m" and a.batch == 64 and a.size == 640 and a.dtype == "bf16":
        tr, cover = traffic_lookup(dom[0], m.launch_names())
        if tr is not None:
            roof["traffic"] = round(tr)
            roof["traffic_source"] = (f"{os.path.relpath(TRAFFIC_MD, ROOT)}: rocprofv3 FETCH_SIZE/WRITE_SIZE, "
                                      f"{cover:.0%} of this run's launches of the kernel")
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
        cpu = cpu_baseline(a.variant, a.size, a.batch, P)
    line = {
        "metric": "YOLO26 images/s @640 bs64 bf16 on 1 GPU; per-kernel % of HBM/MFMA roofline",
        "value": round(value, 1), "unit": "images/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": a.dtype, "data": "synthetic",
        "config": {"workload": f"YOLO26{a.variant} end-to-end forward {a.size}x{a.size} batch {a.batch}",
                   "batch": a.batch, "size": a.size, "variant": a.variant, "classes": 80,
                   "weights": "seeded Kaiming-normal, identity BN folded", "graph": ("hipGraph replay: one graph, its dispatches in order on one hardware queue" if a.streams == 1
                             else f"hipGraph replay: one graph captured over {a.streams} streams, the Detect "
                                  "head's six chains as parallel branches beside the trunk"),
                   "forward_tflop": round(total_flops / 1e12, 3),
                   "achieved_tflops_e2e": round(total_flops / (ms / 1e3) / 1e12, 1),
                   "tile_plans": plans_used},
        "roofline": roof,
        "cpu_baseline": cpu,
        "micro": micro_summary,
        "fp8_run": fp8_run,
        "fp8_forced_run": fp8_forced,
        "context": context,
        "kernels": kern,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
