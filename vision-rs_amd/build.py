#!/usr/bin/env python3
"""Build the gfx950 code objects and the C-ABI host library, in-tree.

  vision-rs_amd/lib/*.hsaco   one code object per csrc/kernels/*.hip
                              (hipcc --genco --offload-arch=gfx950), loaded at
                              run time with hipModuleLoad
  vision-rs_amd/lib/libvrs.so host runtime (csrc/host/*.cpp), exports include/vrs.h

Runs on a machine without a GPU (hipcc cross-compiles).  Usage:
  python vision-rs_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "lib")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU forms are disabled for every device compile (their results
# have been unreliable on this pool); -O3 would otherwise emit them.
DEVICE_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-result",
              f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    return out


def build(jobs: int = 8, verbose: bool = False) -> None:
    os.makedirs(LIB, exist_ok=True)
    kernels = sorted(glob.glob(os.path.join(CSRC, "kernels", "*.hip")))
    # host runtime: C++ sources plus the HIP source holding the library's own
    # device array (the allocation-free entry point's workspace)
    hosts = sorted(glob.glob(os.path.join(CSRC, "host", "*.cpp"))) + \
        sorted(glob.glob(os.path.join(CSRC, "host", "*.hip")))
    cmds = []
    for k in kernels:
        name = os.path.splitext(os.path.basename(k))[0]
        out = os.path.join(LIB, f"{name}.hsaco")
        cmds.append([HIPCC, "--genco", *DEVICE_FLAGS, "-o", out + ".tmp", k])
    so = os.path.join(LIB, "libvrs.so")
    cmds.append([HIPCC, *HOST_FLAGS, *DEVICE_FLAGS[2:], "-o", so + ".tmp", *hosts])
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        for cmd, out in zip(cmds, ex.map(_run, cmds)):
            if verbose and out.strip():
                print(out)
    for cmd in cmds:
        tmp = cmd[cmd.index("-o") + 1]
        os.replace(tmp, tmp[: -len(".tmp")])


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    build(a.jobs, a.verbose)
    print(f"built {LIB}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
