"""Builds the gfx950 shared library libbrush_hip.so in-tree with hipcc.

Usage: python -m brush_amd.build   (or __graft_entry__.build()).
"""
from __future__ import annotations

import os
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor

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
    # per-kernel VGPRs, LDS, occupancy and scratch, checked below
    "-Rpass-analysis=kernel-resource-usage",
]
# the stage ranges (roctx, recorded by rocprofv3 --marker-trace)
LINK_LIBS = ["-L/opt/rocm/lib", "-lrocprofiler-sdk-roctx", "-Wl,-rpath,/opt/rocm/lib"]


def kernel_resources(stderr: str) -> dict:
    """Parses the compiler's kernel-resource-usage remarks into
    {kernel: {field: value}} (fields as the compiler names them)."""
    out, cur = {}, None
    for line in stderr.splitlines():
        if "remark:" not in line:
            continue
        text = line.split("remark:", 1)[1].split("[-Rpass", 1)[0].strip()
        if text.startswith("Function Name:"):
            cur = out.setdefault(text.split(":", 1)[1].strip(), {})
        elif cur is not None and ":" in text:
            k, v = text.rsplit(":", 1)
            cur[k.strip()] = v.strip()
    return out


def _run(cmd):
    return subprocess.run(cmd, capture_output=True, text=True)


def build(verbose: bool = True) -> str:
    """Compiles every translation unit to an object in parallel (each one is
    self-contained: no relocatable device code), then links the library."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    jobs = []
    for src in SOURCES:
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        jobs.append((obj, [HIPCC, *compile_flags, "-c", "-o", obj, os.path.join(CSRC, src)]))
    t0 = time.time()
    if verbose:
        print("[build]", " ".join(jobs[0][1][:-4]), "-c <source>", flush=True)
    workers = max(1, min(len(jobs), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        results = list(pool.map(_run, [cmd for _, cmd in jobs]))
    stderr = []
    for (obj, cmd), res in zip(jobs, results):
        stderr.append(res.stderr)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError(f"hipcc failed to compile {cmd[-1]}")
    # A kernel that spills to scratch (private memory) runs several times
    # slower; none of this library's kernels needs scratch, so one that does
    # is a build error (a captured lambda variable that lost SROA was one).
    res = {}
    for e in stderr:
        res.update(kernel_resources(e))
    scratch = {k: v.get("ScratchSize [bytes/lane]") for k, v in res.items()
               if v.get("ScratchSize [bytes/lane]", "0") != "0"}
    if scratch:
        raise RuntimeError(f"kernels use scratch memory: {scratch}")
    with open(os.path.join(objdir, "kernel_resources.txt"), "w") as f:
        for k in sorted(res):
            f.write(k + " " + " | ".join(f"{a}={b}" for a, b in res[k].items()) + "\n")
    tmp = OUT + ".tmp"
    res = _run([HIPCC, "--offload-arch=gfx950", "-fPIC", "-shared", "-o", tmp, *[obj for obj, _ in jobs], *LINK_LIBS])
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed to link libbrush_hip.so")
    os.replace(tmp, OUT)
    if verbose:
        warn = [l for e in stderr for l in e.splitlines()
                if "warning" in l and "packed-fp32-ops" not in l and "remark" not in l]
        for l in warn[:20]:
            print("[build]", l)
        print(f"[build] {OUT} ({time.time() - t0:.1f} s)", flush=True)
    return OUT


if __name__ == "__main__":
    build()
