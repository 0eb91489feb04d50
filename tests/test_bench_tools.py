"""CPU tests of bench.py's profile summarisers on small synthetic inputs in the
formats rocprofv3 and `bench.py --layers` write."""
import csv
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _write_csv(path, header, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(header)
        w.writerows(rows)


def test_layers_summary_bounds(tmp_path):
    # 1 GFLOP over 1 MB: above the bf16 ridge (312 flop/B) -> MFMA bound;
    # 0.1 GFLOP over 100 MB -> HBM bound
    p = tmp_path / "layers.err"
    p.write_text("\n".join([
        "[bench] something else",
        json.dumps({"layer": "model.1:vrs_conv_x", "us": 1.0, "gflop": 1.0, "mb": 1.0}),
        json.dumps({"layer": "model.2:vrs_dw_y", "us": 50.0, "gflop": 0.1, "mb": 100.0}),
    ]) + "\n")
    out = bench.layers_summary(str(p))
    rows = [l for l in out.splitlines() if l.startswith("| model.")]
    assert len(rows) == 2
    c1 = [c.strip() for c in rows[0].strip("|").split("|")]
    c2 = [c.strip() for c in rows[1].strip("|").split("|")]
    assert c1[5] == "mfma" and c1[6] == "1000 TFLOP/s" and c1[7] == "0.400"
    assert c2[5] == "hbm" and c2[6] == "2000 GB/s" and c2[7] == "0.250"
    assert "2 launches, 51 us in sum" in out


def test_pmc_table_calibration_and_busy(tmp_path):
    hdr = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value", "Start_Timestamp",
           "End_Timestamp"]
    # calibration copy: 1 GiB read reported as 512 MiB (factor 2), 1 GiB written (factor 1)
    gib_kib = 2 ** 30 / 1024
    rows = [
        [1, "__amd_rocclr_copyBuffer", 64, "FETCH_SIZE", gib_kib / 2, 0, 1000],
        [1, "__amd_rocclr_copyBuffer", 64, "WRITE_SIZE", gib_kib, 0, 1000],
        [2, "vrs_k", 256, "FETCH_SIZE", 1000.0, 0, 10_000],
        [2, "vrs_k", 256, "WRITE_SIZE", 500.0, 0, 10_000],
        # busy = 2.048e6 / (8e5 / 8 * 1024) = 2 %
        [2, "vrs_k", 256, "GRBM_GUI_ACTIVE", 8e5, 0, 10_000],
        [2, "vrs_k", 256, "SQ_VALU_MFMA_BUSY_CYCLES", 2.048e6, 0, 10_000],
    ]
    d = tmp_path / "p"
    d.mkdir()
    _write_csv(d / "x_counter_collection.csv", hdr, rows)
    out = bench.pmc_table([str(d)])
    assert "FETCH_SIZE factor 2.0000, WRITE_SIZE factor 1.0000" in out
    row = [l for l in out.splitlines() if l.startswith("| vrs_k")][0]
    c = [x.strip() for x in row.strip("|").split("|")]
    assert c[2] == "10.0" and c[3] == "2.0"
    assert c[4] == f"{1000 * 2 * 1024 / 1e6:.2f}" and c[5] == f"{500 * 1024 / 1e6:.2f}"


def test_trace_summary_matches_profile_launches(tmp_path):
    # one kernel, 2 launches per forward, 1 timed step, 2 profile dispatches:
    # replays take 10 us, profile dispatches 20 us, earlier autotune ones 99 us
    hdr = ["Kernel_Name", "Start_Timestamp", "End_Timestamp"]
    rows, t = [], 0
    for us in [99, 99, 10, 10, 20, 20]:
        rows.append(["vrs_k", t, t + us * 1000])
        t += 1_000_000
    d = tmp_path / "tr"
    d.mkdir()
    _write_csv(d / "b_kernel_trace.csv", hdr, rows)
    bj = tmp_path / "b.json"
    bj.write_text(json.dumps({"value": 1.0, "ms_per_step": 1.0, "kernels": {"vrs_k": {"launches": 2, "ms": 0.042}},
                              "roofline": {"kernel": "vrs_k", "avg_launch_us": 21.0, "achieved": 1.0,
                                           "unit": "TFLOP/s", "frac": 0.5, "peak": 2.0}}) + "\n")
    out = bench.trace_summary(str(d), str(bj), steps=1, profile_iters=1)
    row = [l for l in out.splitlines() if l.startswith("| vrs_k")][0]
    c = [x.strip() for x in row.strip("|").split("|")]
    assert c[1] == "2" and c[2] == "21.0" and c[3] == "20.0" and c[4] == "10.0"


def test_load_plan_checks_conv_names(tmp_path):
    # a plan is applied only when its conv names are the model's, in order
    p = tmp_path / "plan.json"
    p.write_text(json.dumps({"note": "t", "plan": [["model.0", 0], ["model.1", 11], ["model.2.cv1", 1]]}))
    assert bench.load_plan(str(p), ["model.0", "model.1", "model.2.cv1"]) == [0, 11, 1]
    assert bench.load_plan(str(p), ["model.0", "model.2.cv1", "model.1"]) is None      # reordered
    assert bench.load_plan(str(p), ["model.0", "model.1"]) is None                     # count differs
    assert bench.load_plan(str(tmp_path / "missing.json"), ["model.0"]) is None


def test_committed_plans_match_the_model_builder():
    # the committed plans name the convs of the record-only YOLO26m model
    sys.path.insert(0, os.path.join(ROOT, "vision-rs_amd"))
    import vrs
    m = vrs.Model(None, vrs.block(vrs.BLOCK_YOLO26, 3, nc=80, variant="m", one2one=True), 64, 640, 640,
                  vrs.BF16, 1e-3)
    names = [pre for pre, _, _ in m.conv_info()]
    for kind in ("bf16", "fp8", "fp8_forced"):
        path = bench.plan_path("m", kind, 64, 640)
        if os.path.exists(path):
            assert bench.load_plan(path, names) is not None, path
