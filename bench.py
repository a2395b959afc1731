"""Benchmark: the rasterizer on one MI355X.

The default run is BASELINE.json's north-star workload, config 1: one step is
the differentiable render of 1M SH-degree-3 splats at 1920x1080 (f = 1100,
camera at distance 4) followed by its backward for a fixed upstream image
gradient ~ N(0, 1): project + cull, depth sort, scan, project_visible, map,
tile sort, tile offsets, blend, rasterize backward and project backward, all
through libbrush_hip.so.  Inputs are resident in HBM before the timed region.

``--workload ply`` times PLY import/export instead: decode of a resident
1M-splat SH-3 vertex element and export encode (bench_ply).

``--config 0|2`` times the same forward + backward on those workloads,
``--config 3`` the forward-only render of the eight 3840x2160 poses (one step =
eight views), ``--config 4`` one full training step (render, L1 + SSIM loss,
backward, AdamScaled on every splat parameter) at 1600x1064.

Prints one JSON line (the driver's contract).  ``roofline`` reports the kernel
with the largest share of the step: its algorithmic bytes per launch divided by
its mean launch time (HIP events on the library's stream bound to that kernel's
dispatch, in the timed region, on every fifth step by default), against 8 TB/s; ``traffic`` is the HBM bytes
per launch that rocprofv3 FETCH_SIZE / WRITE_SIZE measured for it
(profiles/cfg1_hbm_traffic.md).  ``kernels`` is a per-kernel table from a short
separate pass with every launch bracketed by events.  ``cpu_baseline`` times the
C restatement (oracle/liboracle.so) on the box's host cores over a bounded
sample of the same workload.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "cfg1_hbm_traffic.md")
PLY_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "ply_hbm_traffic.md")
METRIC_CFG1 = "fwd+bwd rasterize ms & Mpix/s, 1M Gaussians SH3 @1080p; % HBM roofline"


def measured_traffic(kernel: str, workload: str, profile: str = TRAFFIC_PROFILE):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (lines ``traffic <kernel> <bytes>``), or
    None when that summary does not cover this workload or kernel."""
    try:
        text = open(profile).read()
    except OSError:
        return None
    if f"workload: {workload}" not in text:
        return None
    for line in text.splitlines():
        f = line.split()
        if len(f) == 3 and f[0] == "traffic" and f[1] == kernel:
            return int(f[2])
    return None


VALU_PROFILE = os.path.join(ROOT, "profiles", "cfg1_valu_counters.md")
SIMDS = 1024          # 256 CUs x 4 SIMDs
CLOCK_GHZ = 2.4       # peak engine clock
CYCLES_PER_VALU = 4   # a wave64 FP32 instruction on a 16-lane SIMD (packed FP32 off)


def measured_valu(kernel: str, workload: str, profile: str = VALU_PROFILE):
    """VALU instructions per launch of ``kernel`` from the committed SQ counter
    summary (table rows `| `kernel` | busy us | VGPRs | LDS | waves | VALU (M) |`),
    or None when the summary does not cover this workload or kernel."""
    try:
        text = open(profile).read()
    except OSError:
        return None
    if f"workload: {workload}" not in text:
        return None
    for line in text.splitlines():
        f = [c.strip() for c in line.split("|")]
        if len(f) > 6 and f[1] == f"`{kernel}`":
            try:
                return float(f[6]) * 1e6
            except ValueError:
                return None
    return None


def algorithmic_bytes(name: str, n: int, v: int, m: int, m_post: int, t: int, p: int, c: int,
                      contributing: int | None = None) -> float:
    """Compulsory HBM bytes of one launch: every input read once, every output
    written once (counts per launch; sort passes are separate launches).
    ``contributing`` is the number of splats some pixel blended (the forward's
    visible mask), the ones with a gradient."""
    if name == "project_forward":
        # transforms+opac in; count, radius, depth key out; the visible
        # splats' SH rows in and their 48-B row slots out
        return 44.0 * n + 12.0 * n + v * (12 * c + 48)
    if name == "project_visible":
        # (only without intersections; otherwise map_intersects orders the rows)
        return v * (4 + 48) + v * (40 + 4)               # gid + row slot in; ordered row, depth out
    if name == "scan":
        return 12.0 * v                                  # gid + gathered count in, cum out
    if name == "depth_sort_count":
        # (key, gid, tile count) in, (gid, cum_tiles_hit) out, for every pair.  The count kernel sorts the buckets with 1 to
        # 15 key bits below the top digit and at most 8192 pairs (every
        # bucket at configs 0, 1 and 4), the LSD kernel the others (most of
        # them at configs 2 and 3); the pairs' bytes are credited here.
        return 20.0 * v
    if name == "depth_sort_buckets":
        return 0.0
    if name == "map_intersects":
        # gid + global-id row slot (48 B) + cum in; ordered row + depth out; (tile, id) pairs out,
        # the tile ids 16-bit below 2^16 tiles
        return (4.0 + 48.0 + 8.0) * v + 44.0 * v + (6.0 if t < 65536 else 8.0) * m
    if name == "tile_offsets":
        return 4.0 * m + 8.0 * t
    if name == "rasterize":
        # id+row per used isect, image, visible, offsets; its trailing workgroups zero the
        # backward's [N, 11] gradient rows (a forward with the backward's record)
        return 44.0 * m_post + 16.0 * p + 4.0 * v + 16.0 * t + 44.0 * n
    if name == "rasterize_backward":
        # id+row, image+grad image, atomics per isect; its fill workgroups zero
        # the dense gradient rows (transforms, SH, opacity, refine)
        fill = (40 + 12 * c + 8) * n if n >= FUSED_FILL_MIN_SPLATS else 0
        return 44.0 * m_post + 32.0 * p + 40.0 * m_post + fill
    if name == "project_backward":
        # gradient lanes [N, 11] in, dense rows out (transforms, SH, opacity,
        # refine); the parameters are read only for the splats with a
        # gradient, those some pixel blended.  From FUSED_FILL_MIN_SPLATS on,
        # the rasterize backward zeroes the dense rows and project backward
        # writes only the rows with a gradient.
        k = v if contributing is None else contributing
        rows = k if n >= FUSED_FILL_MIN_SPLATS else n
        return 44.0 * n + (40 + 12 * c + 4) * k + (40 + 12 * c + 8) * rows
    if name == "image_loss_forward":
        return 28.0 * p                                  # RGB + packed GT in, RGB map out
    if name == "image_loss_backward":
        return 44.0 * p                                  # RGB, GT, chain in; RGBA gradient out
    if name == "adam_step":
        # three launches per step (transforms, SH with per-row second moment,
        # opacity): the mean per launch
        return (28.0 * 10 * n + (20.0 * 3 * c + 8.0) * n + 28.0 * n) / 3.0
    return 0.0


BUCKET_SORT_MAX_SPLATS = 1 << 21  # the depth sort's bucket path (brush_amd/csrc/api.hip)
FUSED_FILL_MIN_SPLATS = 0  # dense gradients zeroed by the rasterize backward (brush_amd/csrc/api.hip)


def sort_bytes_per_launch(name: str, passes: float, n: int, m: int, t: int) -> float:
    """Algorithmic bytes of one launch of a sort kernel: every digit pass reads
    and writes (key, u32 value) once; the depth sort's first pass generates
    its values (global ids) instead of reading them; each pass's upsweep reads
    the keys (the offset scan's few counters are not counted), and the bucket
    path's one upsweep also each splat's tile count.  Below 2^16 tiles the
    tile sort's keys are 16-bit until its last pass writes the 32-bit sorted
    ids."""
    k16 = t < 65536
    if name == "depth_sort_up":
        return (8.0 if n <= BUCKET_SORT_MAX_SPLATS else 4.0) * n
    if name == "tile_sort_up":
        return (2.0 if k16 else 4.0) * m
    if name == "depth_sort_onesweep":
        if n <= BUCKET_SORT_MAX_SPLATS:
            # the top-digit pass: key in, (key, gid) out, each gid's tile
            # count in and out beside it
            return 20.0 * n
        return (16.0 * passes - 4.0) * n / max(passes, 1.0)
    if name == "tile_sort_onesweep":
        if not k16:
            return 16.0 * m
        # 12 B per pair in the earlier passes, 14 B in the last
        return (12.0 * passes + 2.0) * m / max(passes, 1.0)
    return 0.0


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(mode: str, workload, transforms, sh, opac, v_out, gt, min_seconds: float = 10.0,
                 max_reps: int = 20) -> dict:
    """Times the C restatement (oracle/liboracle.so, OpenMP over splats and
    tiles) on the same full workload on the host cores it may use, then on one
    core; each repeated until about ``min_seconds`` / 2 of CPU work (at least
    one repetition); reports the median repetition in Mpix/s.  Forward-only
    workloads time one pose per repetition."""
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))
    multi = _cpu_run(mode, workload, transforms, sh, opac, v_out, gt, threads, min_seconds / 2.0, max_reps)
    single = _cpu_run(mode, workload, transforms, sh, opac, v_out, gt, 1, min_seconds / 2.0, max_reps)
    out = dict(multi)
    out["cpu_model"] = cpu_model()
    out["single_thread"] = {"value": single["value"], "ms_per_step": single["ms_per_step"], "reps": single["reps"],
                            "cores": 1}
    return out


def _cpu_run(mode, workload, transforms, sh, opac, v_out, gt, threads, min_seconds, max_reps) -> dict:
    from brush_amd.camera import project_uniforms
    from oracle import oracle as O

    O.set_threads(threads)
    w = workload
    u = project_uniforms(w.camera(0, 8 if mode == "forward" else 1), w.img_w, w.img_h, w.n, w.sh_degree)
    h, wd = w.img_h, w.img_w
    p = [transforms.copy(), sh.copy(), opac.copy()] if mode == "train" else None
    m1 = [np.zeros_like(x) for x in p] if p else None
    m2 = [np.zeros_like(p[0]), np.zeros((w.n,), np.float32), np.zeros_like(p[2])] if p else None
    times = []
    t_start = time.perf_counter()
    while len(times) < max_reps and (time.perf_counter() - t_start < min_seconds or len(times) < 1):
        t0 = time.perf_counter()
        if mode == "forward":
            O.render_forward(u, transforms, sh, opac, 0)
        elif mode == "fwd_bwd":
            fwd = O.render_forward(u, transforms, sh, opac, O.FLAG_BWD_INFO)
            vc = O.rasterize_backward(fwd, v_out, O.FLAG_REFINE_WEIGHT)
            O.project_backward(fwd, transforms, sh, opac, vc)
        else:
            fwd = O.render_forward(u, p[0], p[1], p[2], O.FLAG_BWD_INFO)
            cfg = O.loss_config(0.8, -0.2)
            O.image_loss_forward(fwd.out_img, 3, gt, cfg)
            chain = np.full((h, wd, 3), np.float32(1.0 / (3 * h * wd)), np.float32)
            v_img = O.image_loss_backward(fwd.out_img, 3, gt, cfg, chain)
            vc = O.rasterize_backward(fwd, v_img, O.FLAG_REFINE_WEIGHT)
            vt, vcoef, vo, _ = O.project_backward(fwd, p[0], p[1], p[2], vc)
            step = len(times) + 1
            sc_t = np.array([1.6e-4] * 3 + [2e-3] * 4 + [7e-3] * 3, np.float32)
            sc_c = np.repeat(np.array([1.0] + [0.1] * (w.num_coeffs - 1), np.float32), 3)
            O.adam_scaled_step(p[0], vt, m1[0], m2[0], sc_t, False, 1.0, step)
            O.adam_scaled_step(p[1], vcoef, m1[1], m2[1], sc_c, True, 2.5e-3, step)
            O.adam_scaled_step(p[2], vo, m1[2], m2[2], None, False, 0.012, step)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    px = w.img_w * w.img_h
    what = {"forward": "forward-only render of one pose", "fwd_bwd": "fwd+bwd step",
            "train": "training step (render, loss, backward, Adam)"}[mode]
    return {"value": round(px / dt / 1e6, 4), "unit": "Mpix/s", "cores": threads, "kind": "port",
            "ms_per_step": round(dt * 1000.0, 2), "reps": len(times),
            "sample": f"the C restatement of the reference algorithm (oracle/, not the reference binary) on the "
                      f"full {w.name} {what} ({w.n} splats, {w.img_w}x{w.img_h}), median of {len(times)} repetitions"}


PLY_METRIC = "PLY import+export splats/s: decode of a resident 3DGS vertex element + export encode, 1M SH3"


def _ply_workload(n: int, seed: int = 7):
    """A 3DGS-layout PLY (x y z nx ny nz f_dc_0..2 f_rest_0..44 opacity
    scale_0..2 rot_0..3, 62 float32 properties) of n seeded splats."""
    rng = np.random.default_rng(seed)
    names = ["x", "y", "z", "nx", "ny", "nz"] + [f"f_dc_{k}" for k in range(3)] + \
        [f"f_rest_{k}" for k in range(45)] + ["opacity"] + [f"scale_{k}" for k in range(3)] + \
        [f"rot_{k}" for k in range(4)]
    rows = rng.standard_normal((n, len(names)), dtype=np.float32)
    head = "ply\nformat binary_little_endian 1.0\nelement vertex %d\n" % n
    head += "".join(f"property float {k}\n" for k in names) + "end_header\n"
    return head.encode() + rows.tobytes(), len(names) * 4


def bench_ply(args):
    """--workload ply: one step decodes the vertex element of a 1M-splat
    SH-degree-3 PLY already resident in HBM (bh_ply_decode_rows) and encodes
    the decoded splats back into export rows (bh_ply_encode_rows)."""
    import torch

    from brush_amd import _lib
    from brush_amd import serde as S

    n = 1 << 20
    dev = torch.device("cuda:0")
    if args.calibrate_copy_mib > 0:  # the first device copy of the run: rocprofv3 counter calibration
        src = torch.ones(args.calibrate_copy_mib * (1 << 18), dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    data, row_bytes = _ply_workload(n)
    header = S.parse_header(data[:1 << 16])
    layout = S.vertex_layout(header.get_element("vertex"))
    body = np.frombuffer(data, np.uint8, n * row_bytes, header.data_offset)
    rows = torch.from_numpy(body.copy()).to(dev)
    out = (torch.empty((n, 10), dtype=torch.float32, device=dev),
           torch.empty((n, layout.num_coeffs, 3), dtype=torch.float32, device=dev),
           torch.empty((n,), dtype=torch.float32, device=dev))
    export = torch.empty((n, 11 + 3 * layout.num_coeffs), dtype=torch.float32, device=dev)
    ctx = _lib.context(0)

    def step():
        d = S.decode_rows(rows, layout, n, out=out)
        ctx.check(_lib.lib().bh_ply_encode_rows(ctx.handle, _lib.ptr(d.transforms), _lib.ptr(d.sh), _lib.ptr(d.opac),
                                                n, layout.num_coeffs, _lib.ptr(export)), "ply_encode_rows")

    out_bytes = n * (10 + 3 * layout.num_coeffs + 1) * 4
    algo = {"ply_decode_rows": n * row_bytes + out_bytes,
            "ply_encode_rows": out_bytes + n * (11 + 3 * layout.num_coeffs) * 4}
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    kernels = {}
    ctx.reset_timings()
    ctx.set_timing(True)
    for _ in range(max(args.profile_steps, 1)):
        step()
    torch.cuda.synchronize()
    for name, (launches, total) in ctx.read_timings().items():
        avg = total / max(launches, 1)
        kernels[name] = {"avg_ms": round(avg, 4), "algorithmic_mb": round(algo[name] / 1e6, 2),
                         "gb_s": round(algo[name] / (avg / 1000.0) / 1e9, 1)}
    ctx.set_timing(False)
    dominant = max(kernels.items(), key=lambda kv: kv[1]["avg_ms"])[0]
    ctx.reset_timings()
    ctx.set_timing(True, only=dominant)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    launches, total = ctx.read_timings()[dominant]
    ctx.set_timing(False)
    ms = (t1 - t0) * 1000.0 / args.steps
    avg = total / max(launches, 1)
    achieved = round(algo[dominant] / (avg / 1000.0) / 1e9, 1)
    roofline = {"bound": "hbm", "kernel": dominant, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(dominant, "ply_1M_sh3", PLY_TRAFFIC_PROFILE),
                "avg_ms": round(avg, 4), "algorithmic_mb": round(algo[dominant] / 1e6, 2),
                "timed_launches": int(launches)}
    # the path a caller with a file in host memory takes (PCIe included)
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    S.load_splat_from_ply(data)
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - h0) * 1000.0
    cpu = None
    if args.cpu_seconds > 0:
        try:
            from oracle import ply_oracle as P

            sample_n = 1 << 17
            sample, _ = _ply_workload(sample_n, seed=8)
            done, c0 = 0, time.perf_counter()
            while time.perf_counter() - c0 < args.cpu_seconds:
                m = P.load_splat_from_ply(sample)
                tt, shh, oo = m.data.with_defaults()
                P.export_rows(tt, shh, oo)
                done += sample_n
            el = time.perf_counter() - c0
            cpu = {"value": round(done / el, 1), "unit": "splats/s", "cores": 1, "kind": "port",
                   "sample": f"numpy restatement (oracle/ply_oracle.py): import of a {sample_n}-splat SH3 PLY "
                             f"from host bytes plus export rows, repeated {done // sample_n}x in {el:.1f} s"}
        except Exception as e:  # reported, never required
            cpu = {"error": str(e)}
    line = {
        "metric": PLY_METRIC,
        "value": round(n / (ms / 1000.0), 1),
        "unit": "splats/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy rows in the 3DGS PLY layout)",
        "config": {"workload": "ply_1M_sh3", "splats": n, "row_bytes": row_bytes, "sh_degree": 3,
                   "host_inclusive_load_ms": round(host_ms, 2), "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line))


def _trace_dispatches(path: str) -> list:
    """(start_ns, end_ns, kernel name) of every dispatch in a rocprofv3 kernel
    trace: a rocpd database (``*_results.db``, the default output) or a csv
    kernel trace (``*_kernel_trace.csv``), in start order."""
    import re

    rows = []
    if path.endswith(".db"):
        import sqlite3

        con = sqlite3.connect(f"file:{path}?mode=ro", uri=True)
        for name, start, end in con.execute("select name, start, end from kernels"):
            rows.append((int(start), int(end), name))
        con.close()
    else:
        import csv

        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    short = lambda n: re.sub(r"[<(].*", "", n.replace("void ", "")).strip()
    typed = lambda n: re.sub(r"\(.*", "", n.replace("void ", "")).strip()
    return sorted((a, b, short(n), typed(n)) for a, b, n in rows)


def split_trace(path: str, steps: int, first_kernel: str = "bh::project_forward_kernel") -> str:
    """Split the last ``steps`` steps of a bench.py run's kernel trace into the
    time the GPU ran kernels and the time it sat idle, as a markdown summary
    (with each kernel's share of the timed steps).

    A step starts at its ``first_kernel`` dispatch and lasts until the next
    step's (the last one until its final dispatch ends); bench.py launches no
    GPU work after its timed region, so the last ``steps`` steps of the trace
    are the timed ones.  Idle time is grouped by the pair of kernels around
    each gap, which names the host work the GPU waited for."""
    rows = _trace_dispatches(path)
    starts = [i for i, r in enumerate(rows) if r[2] == first_kernel]
    if len(starts) < steps:
        raise SystemExit(f"{path}: {len(starts)} steps in the trace, fewer than {steps}")
    sel = starts[-steps:]
    spans, busys, gaps, counts, per_kernel = [], [], {}, {}, {}
    for k, s in enumerate(sel):
        e = sel[k + 1] if k + 1 < len(sel) else len(rows)
        seg = rows[s:e]
        stop = rows[e][0] if e < len(rows) else max(r[1] for r in seg)
        busy, cur = 0, seg[0][0]
        for a, b, _, name in seg:
            busy += max(0, b - max(a, cur))
            cur = max(cur, b)
            n, t = per_kernel.get(name, (0, 0))
            per_kernel[name] = (n + 1, t + (b - a))
        spans.append(stop - seg[0][0])
        busys.append(busy)
        # a gap is time with no kernel running (kernels of a second stream
        # overlap): from the latest end so far to the next start, named by
        # the kernel that ended last and the one that starts
        ends = seg[1:] + ([rows[e]] if e < len(rows) else [])
        last_end, last_name = seg[0][1], seg[0][2]
        for (a0, b0, n0, _), (a1, _, n1, _) in zip(seg, ends):
            if b0 > last_end:
                last_end, last_name = b0, n0
            if a1 > last_end:
                key = (last_name, n1)
                gaps[key] = gaps.get(key, 0) + (a1 - last_end)
                counts[key] = counts.get(key, 0) + 1
    us = lambda ns: ns / 1000.0
    span, busy = sum(spans) / steps, sum(busys) / steps
    out = [f"trace: `{os.path.basename(path)}`: {len(rows)} dispatches, {len(starts)} steps; "
           f"the last {steps} (the timed region) are split below.", "",
           "| per step | us |", "|---|---|",
           f"| step (first dispatch to the next step's first dispatch) | {us(span):.1f} |",
           f"| kernels running | {us(busy):.1f} |",
           f"| GPU idle | {us(span - busy):.1f} ({100.0 * (span - busy) / span:.1f} %) |", "",
           "Step by step (us): " + ", ".join(f"{us(a):.0f}/{us(b):.0f}" for a, b in zip(spans, busys))
           + " (span/kernels).", "",
           "| idle gap between | total us over the timed steps | gaps | us per step |", "|---|---|---|---|"]
    for key, g in sorted(gaps.items(), key=lambda kv: -kv[1])[:10]:
        out.append(f"| `{key[0]}` -> `{key[1]}` | {us(g):.1f} | {counts[key]} | {us(g) / steps:.2f} |")
    out += ["", "| kernel (timed steps) | launches per step | avg us | us per step |", "|---|---|---|---|"]
    for name, (n, t) in sorted(per_kernel.items(), key=lambda kv: -kv[1][1]):
        out.append(f"| `{name}` | {n / steps:g} | {us(t) / n:.2f} | {us(t) / steps:.2f} |")
    return "\n".join(out)


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--split-trace":
        # bench.py --split-trace RESULTS [STEPS]: summarise a rocprofv3 kernel
        # trace of a bench.py run (no GPU used)
        print(split_trace(sys.argv[2], int(sys.argv[3]) if len(sys.argv) > 3 else 20))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 200 timed steps after 20 warm-up steps: shorter runs (20 after 3) read
    # ~11 % slower at config 1, before the GPU reaches its steady clocks
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget in seconds (0 = skip)")
    ap.add_argument("--no-timing", action="store_true", help="do not bracket kernels with HIP events")
    ap.add_argument("--sample-every", type=int, default=5,
                    help="bracket the dominant kernel with events on every Nth timed step (1 = all)")
    ap.add_argument("--profile-steps", type=int, default=5,
                    help="untimed steps with every kernel bracketed by events (per-kernel table)")
    ap.add_argument("--rasterizer", choices=["legacy", "candidate"], default="legacy",
                    help="16x16 tiles (the reference's product path) or the 16x8 candidate tiles")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="before warm-up, run one plain device copy of this many MiB (the known-size reference "
                         "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes)")
    ap.add_argument("--workload", choices=["raster", "ply"], default="raster",
                    help="raster: the rasterizer (BASELINE.json's metric); ply: PLY import/export rows")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported by this build "
              "(the rasterizer path is single-GPU: several GPUs would each render their own views "
              "of a replicated scene and all-reduce the splat gradients)", file=sys.stderr)
        sys.exit(2)

    if args.workload == "ply":
        bench_ply(args)
        return

    import torch

    from brush_amd import _lib
    from brush_amd import render as R
    from brush_amd.synthetic import CONFIGS, generate_splats, generate_target, generate_v_output

    w = CONFIGS[args.config]
    mode = "train" if args.config == 4 else ("forward" if w.forward_only else "fwd_bwd")
    poses = 8 if mode == "forward" else 1
    t_gen = time.perf_counter()
    tr, sh, opac = generate_splats(w)
    v_out = generate_v_output(w) if mode == "fwd_bwd" else None
    gt = generate_target(w) if mode == "train" else None
    t_gen = time.perf_counter() - t_gen
    dev = torch.device("cuda:0")
    t = torch.from_numpy(tr).to(dev).requires_grad_(mode == "fwd_bwd")
    s = torch.from_numpy(sh).to(dev).requires_grad_(mode == "fwd_bwd")
    o = torch.from_numpy(opac).to(dev).requires_grad_(mode == "fwd_bwd")
    vo = torch.from_numpy(v_out).to(dev) if v_out is not None else None
    gt_dev = torch.from_numpy(gt.view(np.int32)).to(dev) if gt is not None else None
    splats = R.Splats(t, s, o)
    rasterizer = R.Rasterizer.Candidate if args.rasterizer == "candidate" else R.Rasterizer.Legacy
    cams = [w.camera(k, poses) for k in range(poses)]
    img_size = (w.img_w, w.img_h)
    ctx = _lib.context(0)
    trainer = None
    if mode == "train":
        from brush_amd.train import SplatTrainer

        trainer = SplatTrainer(rasterizer=rasterizer)

    stats = {"num_visible": 0, "num_intersections": 0}

    def step():
        if mode == "fwd_bwd":
            t.grad = None
            s.grad = None
            o.grad = None
            res = R.render_splats_diff(splats, cams[0], img_size, (0.0, 0.0, 0.0), rasterizer=rasterizer)
            res.img.backward(vo)
            stats["num_visible"] = res.num_visible
            stats["num_intersections"] = res.aux.num_intersections
            stats["tile_offsets"] = res.aux.tile_offsets
            stats["visible_mask"] = res.visible
        elif mode == "forward":
            vis = isect = 0
            for cam in cams:
                out = R.render(cam, img_size, t, s, o, raster_pass=R.RasterPass.Forward, rasterizer=rasterizer)
                vis += out.aux.num_visible
                isect += out.aux.num_intersections
                stats["tile_offsets"] = out.aux.tile_offsets
                out.state.release()
            stats["num_visible"] = vis / poses
            stats["num_intersections"] = isect / poses
        else:
            res = trainer.step(splats, cams[0], gt_dev)
            stats["num_visible"] = res["num_visible"]
            stats["loss"] = res["loss"]

    if args.calibrate_copy_mib > 0:
        words = args.calibrate_copy_mib * (1 << 18)
        src = torch.ones(words, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # The per-kernel pass (or, without timing, one untimed step) comes first:
    # it gives the scene's counts for the byte models and the dominant
    # kernel.  The W warm-up steps then run right before the timed region, so
    # no host work (the tables, the collector) idles the GPU between the last
    # warm-up step and the first timed one.
    # Per-kernel breakdown: a short untimed pass with every launch bracketed by
    # HIP events (events on every launch add ~0.15 ms per step, so the timed
    # region below brackets only the dominant kernel).
    profile_steps = 0 if args.no_timing else max(args.profile_steps, 0)
    if profile_steps:
        # two steps first take the first-use costs (pool blocks, the second
        # stream) out of the table
        for _ in range(2):
            step()
        ctx.reset_timings()
        ctx.set_timing(True)
        for _ in range(profile_steps):
            step()
        torch.cuda.synchronize()
        all_timings = ctx.read_timings()
        ctx.set_timing(False)
    else:
        step()
        torch.cuda.synchronize()
        all_timings = {}
    m_post = 0
    if "tile_offsets" in stats:
        to = stats.pop("tile_offsets")
        m_post = int((to[..., 1].long() - to[..., 0].long()).sum().item())
    contributing = None
    if "visible_mask" in stats:
        contributing = int((stats.pop("visible_mask") > 0).sum().item())
    if mode == "train":
        # the training step's intersection count: one forward at the current parameters
        out = R.render(cams[0], img_size, t, s, o, raster_pass=R.RasterPass.Backward, rasterizer=rasterizer)
        stats["num_intersections"] = out.aux.num_intersections
        m_post = int((out.aux.tile_offsets[..., 1].long() - out.aux.tile_offsets[..., 0].long()).sum().item())
        out.state.release()

    n, v, m = w.n, int(stats["num_visible"]), int(stats["num_intersections"])
    tiles = ((w.img_w + 15) // 16) * ((w.img_h + rasterizer.tile_height - 1) // rasterizer.tile_height)
    c = w.num_coeffs
    pixels = w.img_w * w.img_h

    def kernel_table(timings: dict, steps: int) -> dict:
        table = {}
        for name, (launches, total) in timings.items():
            per_step_launches = launches / steps
            avg = total / max(launches, 1)
            if name.endswith(("_onesweep", "_up", "_scan")):
                b = sort_bytes_per_launch(name, per_step_launches / poses, n, m, tiles)
            else:
                b = algorithmic_bytes(name, n, v, m, m_post, tiles, pixels, c, contributing)
            table[name] = {"launches_per_step": round(per_step_launches, 2), "avg_ms": round(avg, 4),
                           "ms_per_step": round(total / steps, 4),
                           "algorithmic_mb": round(b / 1e6, 2) if b else None,
                           "gb_s": round(b / (avg / 1000.0) / 1e9, 1) if b and avg > 0 else None}
        return table

    kernels, dominant = {}, None
    if profile_steps:
        kernels = kernel_table(all_timings, profile_steps)
        dominant = max(kernels.items(), key=lambda kv: kv[1]["ms_per_step"])[0] if kernels else None

    # The timed region brackets the dominant kernel with events on every
    # --sample-every-th step: a timed launch leaves the GPU idle for ~5 us on
    # each side of the kernel, which would otherwise be part of every step.
    every = max(1, args.sample_every)
    # the objects alive now (torch's, the inputs) leave the collector's
    # generations, so a collection inside the timed region scans only the
    # steps' own short-lived objects
    gc.collect()
    gc.freeze()
    for _ in range(args.warmup):
        step()
    ctx.reset_timings()
    ctx.set_timing(dominant is not None, only=dominant)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(args.steps):
        if dominant is not None and every > 1:
            ctx.enable_timing(k % every == 0)
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sampled = -(-args.steps // every)  # the steps whose dominant launch was timed
    timed = kernel_table(ctx.read_timings(), sampled) if dominant else {}
    ctx.set_timing(False)
    ms = (t1 - t0) * 1000.0 / args.steps
    mpix = pixels * poses / (ms / 1000.0) / 1e6

    roofline = None
    if dominant and dominant in timed:
        kd = timed[dominant]
        achieved = kd["gb_s"] or 0.0
        roofline = {"bound": "hbm", "kernel": dominant, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(dominant, w.name),
                    "avg_ms": kd["avg_ms"], "algorithmic_mb": kd["algorithmic_mb"],
                    "timed_launches": int(round(kd["launches_per_step"] * sampled)),
                    "timed_steps": f"every {every}th of the {args.steps} timed steps" if every > 1 else "all"}
        # the blend kernels are bound by VALU issue, not HBM: the dominant
        # kernel's instructions per launch (committed SQ counter summary) over
        # the issue slots of its live-measured duration
        valu = measured_valu(dominant, w.name)
        if valu and kd["avg_ms"]:
            slots = kd["avg_ms"] * 1e-3 * CLOCK_GHZ * 1e9 * SIMDS / CYCLES_PER_VALU
            roofline["valu"] = {"instructions": int(valu), "issue_frac": round(valu / slots, 3),
                                "model": f"{CYCLES_PER_VALU} cycles per wave64 instruction, {SIMDS} SIMDs, "
                                         f"{CLOCK_GHZ} GHz"}

    cpu = None
    if args.cpu_seconds > 0:
        try:
            cpu = cpu_baseline(mode, w, tr, sh, opac, v_out, gt, args.cpu_seconds)
        except Exception as e:  # the baseline is reported, never required
            cpu = {"error": str(e)}

    metric = {"fwd_bwd": METRIC_CFG1 if args.config == 1 else f"fwd+bwd rasterize ms & Mpix/s, {w.name}",
              "forward": f"forward render ms per view & Mpix/s, {w.name} ({poses} poses per step)",
              "train": f"training step ms & Mpix/s (render, L1+SSIM, backward, AdamScaled), {w.name}"}[mode]
    config = {"workload": w.name, "splats": w.n, "sh_degree": w.sh_degree, "img": [w.img_w, w.img_h],
              "focal": round(w.focal, 3), "distance": w.distance, "num_visible": v, "num_intersections": m,
              "num_intersections_post_raster": m_post, "poses": poses,
              "num_contributing": contributing,
              "sort": "two-stage: depth sort of visible splats, then stable tile-id sort of (tile, depth-rank) "
                      "pairs (equivalent to a 64-bit tile|depth key sort)",
              "parallelism": "single GPU",
              "tiles": f"16x{rasterizer.tile_height}"}
    if mode == "train":
        config["loss"] = round(float(stats["loss"].item()), 6)
    line = {
        "metric": metric,
        "value": round(mpix, 2),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64 generator, brush_amd/synthetic.py)",
        "config": config,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "event_timing": not args.no_timing,
        "input_gen_s": round(t_gen, 2),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
