"""Shared scene builders and comparison helpers for the test suite."""
from __future__ import annotations

import math

import numpy as np

from brush_amd.camera import Camera, focal_to_fov, fov_to_focal, project_uniforms
from oracle import oracle as O
from brush_amd.synthetic import CONFIGS, Workload, generate_splats, generate_v_output, splitmix64


def gsplat_case(name: str):
    """The reference's gsplat golden fixtures (brush-bench-test/src/reference.rs:80-150)."""
    import os

    from safetensors.numpy import load_file

    here = os.path.dirname(os.path.abspath(__file__))
    d = load_file(os.path.join(here, "golden", f"{name}.safetensors"))
    h, w, _ = d["out_img"].shape
    focal = fov_to_focal(math.pi * 0.5, w)
    cam = Camera((0.123, 0.456, -8.0), (0.0, 0.0, 0.0, 1.0), focal_to_fov(focal, w), focal_to_fov(focal, h))
    tr = np.concatenate([d["means"], d["quats"], d["scales"]], 1).astype(np.float32)
    return cam, (w, h), tr, d["coeffs"].astype(np.float32), d["opacities"].astype(np.float32), d["out_img"]


def raster_oracle_scene():
    """The 6-splat scene of brush-render/src/tests/raster_oracle.rs:184-259."""
    cam = Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.6, 0.6)
    means = [[0.0, 0.0, 0.0], [0.08, -0.04, 0.07], [-0.12, 0.06, 0.14], [0.16, 0.10, 0.21],
             [-0.04, -0.14, 0.28], [0.02, 0.03, 0.35]]
    log_scales = [[-0.65, -1.00, -0.85], [-0.80, -0.60, -0.95], [-0.55, -0.90, -0.70],
                  [-1.00, -0.55, -0.80], [-0.70, -0.75, -0.60], [-0.60, -0.65, -0.90]]
    rots = [[1.0, 0.0, 0.0, 0.0], [0.92, 0.12, 0.24, 0.08], [0.81, -0.16, 0.31, 0.10],
            [0.74, 0.28, -0.12, 0.20], [0.88, -0.20, 0.14, 0.09], [0.79, 0.18, 0.22, -0.11]]
    tr = np.concatenate([np.array(means), np.array(rots), np.array(log_scales)], 1).astype(np.float32)
    sh = np.array([0.8, 0.2, -0.5, 0.1, 0.9, 0.3, -0.3, 0.4, 1.0, 0.7, -0.2, 0.5, 0.2, 0.6, 0.8, 0.9, 0.3, 0.1],
                  dtype=np.float32).reshape(6, 1, 3)
    opac = np.array([3.6, 3.1, 2.8, 3.4, 3.0, 3.8], dtype=np.float32)
    return cam, tr, sh, opac, (0.13, 0.07, 0.19)


def random_scene(seed: int, n: int, sh_degree: int = 3, mean_range=1.0, log_scale=(-4.0, 0.5), opac=(0.0, 1.0)):
    """A small seeded scene drawn with the synthetic generator's distributions."""
    w = Workload("test", n, sh_degree, 64, 64, 60.0, 3.0, mean_lo=-mean_range, mean_hi=mean_range,
                 log_scale_mu=log_scale[0], log_scale_sigma=log_scale[1], opac_mu=opac[0], opac_sigma=opac[1],
                 seed=seed)
    return generate_splats(w)


def rng_scene(n, mean_range, log_scale_range, opacity_range, seed):
    """The reference's rng_scene (crates/brush-render/src/tests/mod.rs:180-236): SplitMix64 uniforms, per
    splat means, a non-normalised quaternion, log-scales, SH DC in [0, 1] and a
    raw opacity, drawn in that order."""
    k = np.arange(1, n * 14 + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + k * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = (z.astype(np.float64) / float(2**64 - 1)).astype(np.float32).reshape(n, 14)

    def span(x, lo, hi):
        return (np.float32(lo) + x * np.float32(hi - lo)).astype(np.float32)

    tr = np.empty((n, 10), np.float32)
    tr[:, 0:3] = span(u[:, 0:3], -mean_range, mean_range)
    tr[:, 3:7] = span(u[:, 3:7], -1.0, 1.0)
    tr[:, 7:10] = span(u[:, 7:10], *log_scale_range)
    sh = span(u[:, 10:13], 0.0, 1.0).reshape(n, 1, 3)
    opac = span(u[:, 13], *opacity_range)
    return tr, sh, opac


def uniforms_for(cam: Camera, w: int, h: int, n: int, deg: int) -> dict:
    return project_uniforms(cam, w, h, n, deg)


def assert_bits_equal(name, a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    assert a.shape == b.shape, f"{name}: shape {a.shape} vs {b.shape}"
    if a.dtype == np.float32:
        a = a.view(np.uint32)
        b = b.view(np.uint32)
    bad = np.nonzero(a.reshape(-1) != b.reshape(-1))[0]
    assert bad.size == 0, f"{name}: {bad.size} of {a.size} differ, first at {bad[:5]}: {a.reshape(-1)[bad[:5]]} vs {b.reshape(-1)[bad[:5]]}"


def rel_close(name, got, want, rtol=1e-3, atol_frac=1e-5):
    """|got - want| <= rtol * |want| + atol, atol = atol_frac * max|want| over
    the finite entries; a non-finite entry must match exactly (NaN where NaN,
    inf of the same sign), so a NaN on either side fails the check."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{name}: shape {got.shape} vs {want.shape}"
    gf, wf = np.isfinite(got), np.isfinite(want)
    odd = np.nonzero(((gf != wf) | (~gf & ~wf & ~((got == want) | (np.isnan(got) & np.isnan(want))))).reshape(-1))[0]
    assert odd.size == 0, (f"{name}: {odd.size}/{got.size} non-finite mismatches, first at {odd[:3]}: "
                           f"{got.reshape(-1)[odd[:3]]} vs {want.reshape(-1)[odd[:3]]}")
    got = np.where(gf, got, 0.0)
    want = np.where(wf, want, 0.0)
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    atol = atol_frac * scale + 1e-30
    err = np.abs(got - want)
    tol = rtol * np.abs(want) + atol
    bad = np.nonzero(err.reshape(-1) > tol.reshape(-1))[0]
    assert bad.size == 0, (f"{name}: {bad.size}/{got.size} outside rtol={rtol} atol={atol:.3g}; worst "
                           f"{err.reshape(-1)[bad[:3]]} at {bad[:3]} (want {want.reshape(-1)[bad[:3]]})")


# lanes of v_combined that are sums of the same per-pixel terms times
# different pixel offsets: 2D mean (0-1), conic (2-4), colour (5-7), opacity,
# refine, depth
LANE_GROUPS = ((0, 2), (2, 5), (5, 8), (8, 9), (9, 10), (10, 11))


def gradient_term_magnitudes(o, tr, sh, opac, vc, mip: bool = False, rel: float = 3e-5, draws: int = 3,
                             seed: int = 0):
    """For each dense gradient entry (transforms, SH coefficients, raw
    opacities), how far it moves when the gradient lanes v_combined move by
    the differences between two correct f32 summations of a lane in different
    orders: `rel` noise relative to the largest lane of the lane's group.  A
    lane's summation error scales with the size of its terms, and the lanes
    of a group are sums of the same per-pixel terms (v_sigma times dx dx,
    dx dy, dy dy for the conic lanes), so a lane that is a small difference of
    large terms carries the error of its group's large lanes.  Project
    backward turns conic lanes of 1e4-1e6 into scale and rotation gradients
    of order 1-100 through intermediates that cancel, so a few entries amplify
    lane differences of 1e-7 into percent-level changes (the CPU restatement
    and the GPU, whose lanes agree to 7 digits, differ there); for a
    well-conditioned entry the movement is ~rel * |entry|.

    Two parts, added: the first-order worst case over that box of lane errors
    (each lane moved by +rel * scale alone, the entries' absolute changes
    summed over the lanes: a deterministic bound for errors of either sign in
    every lane), and the largest movement under a few random perturbations of
    the same size, which also carries the entry's own float32 evaluation noise
    (for the ill-conditioned entries that noise, not the linear response,
    dominates; two correct GPU runs differ there by half of the random part
    alone)."""
    base = [x.astype(np.float64) for x in O.project_backward(o, tr, sh, opac, vc, mip)[:3]]
    box = [np.zeros(x.shape) for x in base]
    sens = [np.zeros(x.shape) for x in base]
    rng = np.random.default_rng(seed)
    vc64 = vc.astype(np.float64)
    scale = np.empty_like(vc64)
    for a, b in LANE_GROUPS:
        if a < vc64.shape[1]:
            scale[:, a:b] = np.max(np.abs(vc64[:, a:b]), axis=1, keepdims=True)
    for lane in range(vc.shape[1]):
        vp = vc64.copy()
        vp[:, lane] += rel * scale[:, lane]
        out = O.project_backward(o, tr, sh, opac, vp.astype(np.float32), mip)[:3]
        for s_, x, b in zip(box, out, base):
            s_ += np.abs(x.astype(np.float64) - b)
    for _ in range(draws):
        noise = rng.uniform(-1.0, 1.0, vc.shape)
        vp = (vc64 + rel * noise * scale).astype(np.float32)
        out = O.project_backward(o, tr, sh, opac, vp, mip)[:3]
        for s_, x, b in zip(sens, out, base):
            np.maximum(s_, np.abs(x.astype(np.float64) - b), out=s_)
    return [s_ + b_ for s_, b_ in zip(sens, box)]


def grad_close(name, got, want, magnitude, rtol=1e-3, atol_frac=1e-4, cond=1.0):
    """rel_close with the float error of cancellation allowed for: |got - want|
    <= rtol |want| + atol_frac max|want| + cond * magnitude, with `magnitude`
    the entry's sensitivity to f32 summation differences in its lanes
    (gradient_term_magnitudes).  For a well-conditioned entry that is ~3e-5
    |want| and the bound stays rtol relative; it widens only where the entry
    is a small difference of large intermediates."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{name}: shape {got.shape} vs {want.shape}"
    assert np.array_equal(np.isfinite(got), np.isfinite(want)), f"{name}: non-finite entries differ"
    gf = np.isfinite(got)
    got, want, magnitude = got[gf], want[gf], np.asarray(magnitude, np.float64)[gf]
    scale = float(np.max(np.abs(want))) if want.size else 0.0
    tol = rtol * np.abs(want) + atol_frac * scale + cond * magnitude + 1e-30
    err = np.abs(got - want)
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, (f"{name}: {bad.size}/{got.size} outside; worst {err[bad[:3]]} at {bad[:3]} "
                           f"(want {want[bad[:3]]}, term magnitude {magnitude[bad[:3]]})")


def gpu_forward(uniforms: dict, tr, sh, opac, flags: int, background=(0.0, 0.0, 0.0), device="cuda:0"):
    """Runs bh_render_forward on the GPU and returns every output as numpy."""
    import torch

    from brush_amd import render as R

    t = torch.from_numpy(np.ascontiguousarray(tr)).to(device)
    s = torch.from_numpy(np.ascontiguousarray(sh)).to(device)
    o = torch.from_numpy(np.ascontiguousarray(opac)).to(device)
    raster_pass = R.RasterPass.Forward
    if flags & 1:
        raster_pass = R.RasterPass.BackwardSmoothCutoff if flags & 2 else R.RasterPass.Backward
    mode = R.SplatRenderMode.Mip if flags & 8 else R.SplatRenderMode.Default
    rmode = R.RasterizationMode.RgbaAndDepth if flags & 4 else R.RasterizationMode.Rgba
    rasterizer = R.Rasterizer.Candidate if flags & 32 else R.Rasterizer.Legacy
    out = R.render(None, (uniforms["img_w"], uniforms["img_h"]), t, s, o, mode, rmode, background, raster_pass,
                   uniforms=uniforms, rasterizer=rasterizer)
    u32 = lambda x: x.cpu().numpy().view(np.uint32)
    res = dict(
        out=out,
        num_visible=out.aux.num_visible,
        num_intersections=out.aux.num_intersections,
        intersect_counts=u32(out.intersect_counts),
        max_radius=out.aux.max_radius.cpu().numpy(),
        global_from_compact_gid=u32(out.global_from_compact_gid)[: out.aux.num_visible],
        depths=out.depths.cpu().numpy(),
        cum_tiles_hit=u32(out.cum_tiles_hit),
        projected=out.projected_splats.cpu().numpy(),
        tile_id_from_isect=u32(out.tile_id_from_isect)[: out.aux.num_intersections],
        compact_gid_from_isect=u32(out.compact_gid_from_isect)[: out.aux.num_intersections],
        tile_offsets_pre=u32(out.tile_offsets_pre),
        tile_offsets=u32(out.aux.tile_offsets),
        visible=out.aux.visible.cpu().numpy(),
    )
    img = out.out_img.cpu().numpy()
    res["out_img"] = img if img.dtype == np.float32 else img.view(np.uint32)
    return res


def compare_forward(g: dict, o, exact_image=True, check_visible=True):
    """Bit-exact comparison of every integer output and of the projected rows;
    the image is compared bit for bit when ``exact_image`` else to 1e-4."""
    assert g["num_visible"] == o.num_visible, f"num_visible {g['num_visible']} vs {o.num_visible}"
    assert g["num_intersections"] == o.num_intersections, \
        f"num_intersections {g['num_intersections']} vs {o.num_intersections}"
    assert_bits_equal("intersect_counts", g["intersect_counts"], o.intersect_counts)
    assert_bits_equal("max_radius", g["max_radius"], o.max_radius)
    v, m = o.num_visible, o.num_intersections
    assert_bits_equal("global_from_compact_gid", g["global_from_compact_gid"], o.global_from_compact_gid)
    assert_bits_equal("depths", g["depths"], o.depths_sorted)
    assert_bits_equal("cum_tiles_hit", g["cum_tiles_hit"], o.cum_tiles_hit)
    if v:
        assert_bits_equal("projected", g["projected"][:v], o.projected[:v])
    assert_bits_equal("tile_id_from_isect", g["tile_id_from_isect"], o.tile_id_from_isect[:m])
    assert_bits_equal("compact_gid_from_isect", g["compact_gid_from_isect"], o.compact_gid_from_isect[:m])
    assert_bits_equal("tile_offsets_pre", g["tile_offsets_pre"], o.tile_offsets_pre)
    assert_bits_equal("tile_offsets_post", g["tile_offsets"], o.tile_offsets)
    if exact_image:
        assert_bits_equal("out_img", g["out_img"], o.out_img)
    else:
        err = np.max(np.abs(g["out_img"] - o.out_img)) if g["out_img"].size else 0.0
        assert err <= 1e-4, f"out_img max error {err}"
    if check_visible and o.visible.size == g["visible"].size:
        assert_bits_equal("visible", g["visible"], o.visible)
