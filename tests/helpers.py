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


# ---- gradient comparison -------------------------------------------------------------------------
#
# Gradients are sums of per-pixel terms formed in f32, and every parallel
# evaluation (the restatement's per-tile order, the GPU's per-block sums and
# float atomics) rounds differently.  A lane that is a small difference of
# large terms carries an error of many times its own size even in a correct
# evaluation: at config 0 the restatement itself sits a median 7e-5 and a
# 90th percentile 1.2e-3 (relative) away from a float64 evaluation of the
# same gradient (oracle rasterize_backward_f64) in the lanes driven by
# v_alpha.  So an entry's tolerance is rtol |want| plus that entry's own
# rounding noise, from the restatement's per-lane magnitudes
# (rasterize_backward_check):
#   noise = u (SUM_ORDER_ULPS * sum |terms| + TERM_NOISE_SIGMAS * sqrt(sum m^2))
# with u = 2^-24, the first part bounding a change of summation order, the
# second the terms' own rounding (m: each term's rounding scale).  No
# tolerance is scaled by an array's largest entry.  Dense gradients are held
# to rtol |want| plus the lanes' own tolerance (rtol |lane| + noise) carried
# through project backward: project backward is deterministic and the GPU's
# dense gradients equal, bit for bit, the restatement's project backward of
# the GPU's lanes, so a dense entry may differ by what the lanes' bound
# implies where project backward cancels.

UNIT_ROUNDOFF = 2.0 ** -24
SUM_ORDER_ULPS = 16.0
TERM_NOISE_SIGMAS = 8.0
GRAD_RTOL = 1e-3


def lane_noise(v_abs, v_rss):
    """Per-entry rounding noise of v_combined lanes (see above)."""
    return UNIT_ROUNDOFF * (SUM_ORDER_ULPS * np.asarray(v_abs, np.float64) +
                            TERM_NOISE_SIGMAS * np.asarray(v_rss, np.float64))


def outside(got, want, noise, rtol=GRAD_RTOL):
    """Boolean mask of the entries with |got - want| > rtol |want| + noise
    (non-finite entries must match exactly), and err / tol per entry."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    noise = np.broadcast_to(np.asarray(noise, dtype=np.float64), want.shape)
    assert got.shape == want.shape, f"shape {got.shape} vs {want.shape}"
    gf, wf = np.isfinite(got), np.isfinite(want)
    same_nonfinite = (~gf & ~wf) & ((got == want) | (np.isnan(got) & np.isnan(want)))
    tol = rtol * np.abs(np.where(wf, want, 0.0)) + noise
    err = np.abs(np.where(gf & wf, got - want, 0.0))
    ratio = np.where(tol > 0, err / np.where(tol > 0, tol, 1.0), np.where(err > 0, np.inf, 0.0))
    bad = ((gf != wf) | (~gf & ~wf & ~same_nonfinite)) | (err > tol)
    return bad, np.where(gf != wf, np.inf, ratio)


def check_close(name, got, want, noise, rtol=GRAD_RTOL) -> float:
    """Asserts |got - want| <= rtol |want| + noise entry by entry and prints
    the worst err / tol and the median tolerance relative to |want|; returns
    the worst err / tol."""
    bad, ratio = outside(got, want, noise, rtol)
    want64 = np.asarray(want, np.float64)
    nz = (want64 != 0) & np.isfinite(want64)
    rel_tol = (rtol * np.abs(want64[nz]) + np.broadcast_to(np.asarray(noise, np.float64), want64.shape)[nz]) / \
        np.abs(want64[nz])
    worst = float(ratio.max()) if ratio.size else 0.0
    med = float(np.median(rel_tol)) if rel_tol.size else 0.0
    print(f"[tol] {name}: worst err/tol {worst:.3g} over {ratio.size} entries; median tolerance {med:.3g} of |want|",
          flush=True)
    idx = np.nonzero(bad.reshape(-1))[0]
    assert idx.size == 0, (f"{name}: {idx.size}/{bad.size} outside rtol {rtol} + noise; first at {idx[:3]}: got "
                           f"{np.asarray(got).reshape(-1)[idx[:3]]} want {want64.reshape(-1)[idx[:3]]} noise "
                           f"{np.broadcast_to(np.asarray(noise, np.float64), want64.shape).reshape(-1)[idx[:3]]}")
    return worst


def propagate_noise(o, tr, sh, opac, vc, noise, mip: bool = False, draws: int = 10, seed: int = 0,
                    draw_factor: float = 3.0, rtol: float = 0.0):
    """How far the dense gradients (transforms, SH coefficients, raw
    opacities) move when the lanes move within their tolerance: the sum over
    lanes of the change from moving that lane alone by rtol |lane| plus its
    noise (a first order bound for lane errors of any sign within the lanes'
    own tolerance), plus ``draw_factor`` times the largest change under a
    few random moves by the noise alone.  The first part is what the lanes'
    bound implies for an entry where project backward cancels (a dense entry
    that is a small difference of large lane contributions moves by far more
    than rtol of itself when its lanes move by rtol of theirs).  The random
    part carries project backward's own f32 evaluation where an entry is a
    small difference of large intermediates: there a second set of lanes
    moves the entry by rounding, not linearly, and each draw is one sample
    of that rounding.  At config 2 such an entry moved by 4e-6 at most over
    three draws and by 1.8e-5 over twelve (and a correct GPU run differed
    from the restatement by 2e-5 there), so the largest of ten draws is
    taken."""
    base = [x.astype(np.float64) for x in O.project_backward(o, tr, sh, opac, vc, mip)[:3]]
    box = [np.zeros(x.shape) for x in base]
    rnd = [np.zeros(x.shape) for x in base]
    vc64 = vc.astype(np.float64)
    noise = np.asarray(noise, np.float64)
    move = noise + rtol * np.abs(vc64[: noise.shape[0]])
    for lane in range(vc.shape[1]):
        if not move[:, lane].any():
            continue
        vp = vc64.copy()
        vp[: move.shape[0], lane] += move[:, lane]
        out = O.project_backward(o, tr, sh, opac, vp.astype(np.float32), mip)[:3]
        for b, x, b0 in zip(box, out, base):
            b += np.abs(x.astype(np.float64) - b0)
    rng = np.random.default_rng(seed)
    for _ in range(draws):
        vp = (vc64 + noise * rng.uniform(-1.0, 1.0, vc.shape)).astype(np.float32)
        out = O.project_backward(o, tr, sh, opac, vp, mip)[:3]
        for r, x, b0 in zip(rnd, out, base):
            np.maximum(r, np.abs(x.astype(np.float64) - b0), out=r)
    return [b + draw_factor * r for b, r in zip(box, rnd)]


class OracleGrads:
    """The restatement's backward of one forward with the per-entry noise of
    every gradient: lanes ``v_combined`` [V, 11] (compact order) with
    ``lane_noise``; dense ``v_transforms``, ``v_coeffs``, ``v_raw_opac``,
    ``v_refine`` with ``noise_*`` (refine: its lane's noise by global id)."""

    def __init__(self, o, tr, sh, opac, v_out, flags, background=(0.0, 0.0, 0.0), mip: bool = False,
                 check: int = 0, dense: bool = True):
        v = max(o.num_visible, 1)
        vc, v_abs, v_rss = O.rasterize_backward_check(o, v_out, flags, background, check)
        self.o, self.mip = o, mip
        self.v_combined = vc
        self.lane_noise = lane_noise(v_abs, v_rss)[:v]
        if dense:
            self.v_transforms, self.v_coeffs, self.v_raw_opac, self.v_refine = \
                O.project_backward(o, tr, sh, opac, vc, mip)
            self.noise_transforms, self.noise_coeffs, self.noise_raw_opac = \
                propagate_noise(o, tr, sh, opac, vc, self.lane_noise, mip, rtol=GRAD_RTOL)
            self.noise_refine = np.zeros(tr.shape[0])
            if o.num_visible:
                self.noise_refine[o.global_from_compact_gid.astype(np.int64)] = \
                    self.lane_noise[: o.num_visible, 9]


def compare_lanes(name, lanes_compact, want: OracleGrads, rtol=GRAD_RTOL) -> float:
    """v_combined lanes [V, 11] in compact order against the restatement's,
    per entry.  Lanes 9 and 10 are compared only where the restatement wrote
    them (refine weight, depth)."""
    v = want.o.num_visible
    return check_close(name, np.asarray(lanes_compact)[:v], want.v_combined[:v], want.lane_noise[:v], rtol)


def compare_dense(prefix, got: dict, want: OracleGrads, rtol=GRAD_RTOL) -> dict:
    """Dense gradients ({"v_transforms": .., "v_coeffs": .., "v_raw_opac": ..,
    "v_refine": ..}, any subset) against the restatement's, per entry."""
    out = {}
    for key, w, n in (("v_transforms", want.v_transforms, want.noise_transforms),
                      ("v_coeffs", want.v_coeffs, want.noise_coeffs),
                      ("v_raw_opac", want.v_raw_opac, want.noise_raw_opac),
                      ("v_refine", want.v_refine, want.noise_refine)):
        if key in got:
            out[key] = check_close(f"{prefix}{key}", got[key], w, n, rtol)
    return out


def check_fused_backward(name, state, tr, sh, opac, grads: dict, want: OracleGrads):
    """The fused backward of one forward (run with the context's keep_lanes
    debug mode) against the restatement: its per-splat lanes read back by
    global id and permuted to compact order, entry by entry; its dense
    gradients bit for bit against the restatement's project backward of
    those same lanes (project backward is deterministic per splat); and the
    dense gradients against the restatement's own, entry by entry."""
    o = want.o
    lanes = state.backward_lanes()
    assert lanes is not None, "the fused backward kept no lanes (keep_lanes debug mode off?)"
    lanes = lanes.cpu().numpy()
    gfc = o.global_from_compact_gid.astype(np.int64)
    g = np.zeros_like(want.v_combined)
    g[: o.num_visible] = lanes[gfc]
    # rows of splats that were not visible stay zero
    rest = np.ones(lanes.shape[0], bool)
    rest[gfc] = False
    assert not lanes[rest].any(), f"{name}: gradient lanes written for culled splats"
    compare_lanes(f"{name} lanes", g, want)
    vt, vcoef, vo, vr = O.project_backward(o, tr, sh, opac, g, want.mip)
    for key, ref in (("v_transforms", vt), ("v_coeffs", vcoef), ("v_raw_opac", vo), ("v_refine", vr)):
        if key in grads:
            assert_bits_equal(f"{name} {key} (restatement project backward of the GPU lanes)", grads[key], ref)
    return compare_dense(f"{name} ", grads, want)


class keep_lanes:
    """Context manager: the library context keeps the fused backward's lanes."""

    def __enter__(self):
        from brush_amd import _lib

        _lib.context(0).set_debug(keep_lanes=True)
        return self

    def __exit__(self, *exc):
        from brush_amd import _lib

        _lib.context(0).set_debug()
        return False


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
