#!/usr/bin/env python3
"""Copy the reference's forward-pass golden vectors into tests/golden/.

The reference (spinorml/vision-rs) keeps little-endian float32 NCHW fixtures
under tests/fixtures/<family>/ (seed 42, PyTorch/ultralytics generated; see
the reference's tests/test_*_cuda.rs for how each is consumed).  Only DATA
files (*.bin) of forward-pass fixtures are copied; generator scripts,
backward-pass and training-loss fixtures are not.  The copies are committed so
the GPU box (which has no /root/reference) can run the parity tests.

Run once in the build container:  python tests/golden/copy_fixtures.py
"""
import os
import shutil
import sys

REF = os.environ.get("VRS_REFERENCE", "/root/reference")
SRC = os.path.join(REF, "tests", "fixtures")
DST = os.path.dirname(os.path.abspath(__file__))

# family -> list of sub-directories ("" = the family directory itself)
FAMILIES = {
    "c2psa_yolo26": [""],
    "c3k2_yolo26": ["", "shortcut", "deep_sf", "deep_st", "head_sf", "head_st"],
    "concat_upsample": [""],
    "conv_grouped": ["depthwise", "g4"],
    "conv_yolo26": [""],
    "detect_decode": [""],
    "detect_yolo26": [""],
    "sppf_yolo26": [""],
    "silu_4d": [""],
    "sigmoid_4d": [""],
}
# backward-only files that live next to forward data in some families
SKIP = {"dy.bin", "dyu.bin", "dx_expected.bin", "dw_expected.bin", "expected_backward.bin",
        "expected_dx0.bin", "expected_dx1.bin", "expected_dxu.bin"}


def main() -> int:
    if not os.path.isdir(SRC):
        print(f"reference fixtures not found at {SRC}", file=sys.stderr)
        return 1
    n = 0
    for fam, subs in FAMILIES.items():
        for sub in subs:
            sdir = os.path.join(SRC, fam, sub)
            ddir = os.path.join(DST, fam, sub)
            os.makedirs(ddir, exist_ok=True)
            for f in sorted(os.listdir(sdir)):
                if not f.endswith(".bin") or f in SKIP:
                    continue
                shutil.copyfile(os.path.join(sdir, f), os.path.join(ddir, f))
                n += 1
    print(f"copied {n} fixture files into {DST}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
