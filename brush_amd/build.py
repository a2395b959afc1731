"""Builds the gfx950 shared library libbrush_hip.so in-tree with hipcc.

Usage: python -m brush_amd.build   (or __graft_entry__.build()).
"""
from __future__ import annotations

import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libbrush_hip.so")
SOURCES = ["api.hip", "sort.hip", "project.hip", "raster.hip", "backward.hip", "loss.hip", "adam.hip", "ply.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # integer outputs must be reproducible on the CPU: no FMA contraction,
    # IEEE division and square root (the HIP default, stated explicitly)
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # packed FP32 instructions are disabled for this target pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def build(verbose: bool = True) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = OUT + ".tmp"
    cmd = [HIPCC, *FLAGS, "-o", tmp, *srcs]
    t0 = time.time()
    if verbose:
        print("[build]", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed to build libbrush_hip.so")
    os.replace(tmp, OUT)
    if verbose:
        warn = [l for l in res.stderr.splitlines() if "warning" in l and "packed-fp32-ops" not in l]
        for l in warn[:20]:
            print("[build]", l)
        print(f"[build] {OUT} ({time.time() - t0:.1f} s)", flush=True)
    return OUT


if __name__ == "__main__":
    build()
