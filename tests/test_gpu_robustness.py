"""GPU robustness: the reference's stress, invariance and validation tests
(crates/brush-render/src/tests/mod.rs), the debug modes of the C ABI, and
frames with more than 16384 tiles.

* determinism: the same scene renders bit for bit the same, also with every
  workspace block poisoned (0xFF bytes) before use (mod.rs:310-332;
  brush-cube/src/host.rs:52-65 noises uninitialised test tensors);
* invariance: appending culled splats, or prepending a culled prefix that
  shifts every global id, leaves the render bit for bit the same
  (mod.rs:334-410), and the culled splats get exactly zero gradients;
* a 90 % culled scene sorts only its visible splats and renders bit for bit
  as the restatement, with counts read back first and from a plan;
* stress: 120k fullscreen splats render deterministically with no dropped
  tile, 200k large splats leave no tile empty, 30M splats render
  (mod.rs:96-142, 412-605);
* validation: BH_DEBUG_VALIDATE turns a NaN or Inf parameter into
  BH_ERR_NOT_FINITE naming the tensor, where the reference panics
  (mod.rs:607-641; gaussian_splats.rs:322-415), and likewise non-finite
  gradients;
* the fused backward takes the cutoff and depth flags from its forward and
  rejects a caller that passes others, before launching anything;
* more than 16384 tiles (the tile-order kernel keeps the first 16384 tiles'
  buckets in registers and loops over the rest): 3840x2160 with 16x16 tiles
  and 2048x1080 with 16x8 tiles, forward bit for bit and gradients against
  the CPU restatement.
"""
import ctypes

import numpy as np
import pytest

from brush_amd.camera import Camera
from oracle import oracle as O
from tests.helpers import (OracleGrads, check_close, check_fused_backward, compare_forward, gpu_forward, keep_lanes,
                           random_scene, rng_scene, uniforms_for)

pytestmark = pytest.mark.gpu

STATUS_NOT_FINITE = 6
STATUS_INVALID_ARG = 1


def _cam():
    return Camera((0.0, 0.0, -5.0), (0.0, 0.0, 0.0, 1.0), 0.5, 0.5)


def _diff_render(gpu, tr, sh, opac, cam, size, v_out):
    """render_splats_diff forward + fused backward; returns (image, grads)."""
    import torch
    from brush_amd import render as R

    t = torch.from_numpy(np.ascontiguousarray(tr)).to(gpu).requires_grad_(True)
    s = torch.from_numpy(np.ascontiguousarray(sh)).to(gpu).requires_grad_(True)
    o = torch.from_numpy(np.ascontiguousarray(opac)).to(gpu).requires_grad_(True)
    res = R.render_splats_diff(R.Splats(t, s, o), cam, size)
    res.img.backward(torch.from_numpy(v_out).to(gpu))
    torch.cuda.synchronize()
    return (res.img.detach().cpu().numpy(),
            (t.grad.cpu().numpy(), s.grad.cpu().numpy(), o.grad.cpu().numpy()))


def _magnitudes(tr, sh, opac, cam, size, v_out):
    """Per-entry rounding noise of the dense gradients of the scene, from the
    CPU restatement (tests/helpers.py OracleGrads): two GPU runs differ only
    in the order of their float atomics, well within it."""
    u = uniforms_for(cam, size[0], size[1], tr.shape[0], 0)
    o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    want = OracleGrads(o, tr, sh, opac, v_out, O.FLAG_REFINE_WEIGHT)
    return want.noise_transforms, want.noise_coeffs, want.noise_raw_opac


def _forward_arrays(u, tr, sh, opac):
    g = gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    g.pop("out")
    return g


def _assert_same(a: dict, b: dict):
    for k, v in a.items():
        if isinstance(v, np.ndarray):
            assert np.array_equal(v.view(np.uint8), b[k].view(np.uint8)), k
        else:
            assert v == b[k], k


@pytest.fixture
def debug_ctx(gpu):
    from brush_amd import _lib

    ctx = _lib.context()
    yield ctx
    ctx.set_debug()


def test_render_is_deterministic_with_poisoned_workspace(gpu, debug_ctx):
    """mod.rs:310-332 (20k large splats at 256x256, rendered twice) with every
    workspace block of the second and third render poisoned: every forward
    output bit for bit the same, gradients the same up to the order of float
    atomics (and finite), the allocation-free sort unchanged."""
    import torch
    from brush_amd import _lib

    print("[case] determinism with poisoned workspace", flush=True)
    tr, sh, opac = rng_scene(20_000, 2.0, (0.5, 3.0), (-1.0, 2.0), 0xA11CE)
    cam = _cam()
    u = uniforms_for(cam, 256, 256, tr.shape[0], 0)
    v_out = np.random.default_rng(5).standard_normal((256, 256, 4)).astype(np.float32)
    debug_ctx.set_debug()
    f0 = _forward_arrays(u, tr, sh, opac)
    img0, g0 = _diff_render(gpu, tr, sh, opac, cam, (256, 256), v_out)
    mags = _magnitudes(tr, sh, opac, cam, (256, 256), v_out)
    debug_ctx.set_debug(poison=True)
    for rep in range(2):
        f1 = _forward_arrays(u, tr, sh, opac)
        _assert_same(f0, f1)
        img1, g1 = _diff_render(gpu, tr, sh, opac, cam, (256, 256), v_out)
        assert np.array_equal(img0.view(np.uint32), img1.view(np.uint32))
        for name, a, b, m in zip(("v_transforms", "v_coeffs", "v_raw_opac"), g0, g1, mags):
            assert np.all(np.isfinite(b)), name
            check_close(f"{name} (poisoned rep {rep})", b, a, m, rtol=1e-4)
    # the allocation-free sort's fixed scratch is poisoned too
    n = 300_001
    keys = np.random.default_rng(9).integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    tk = torch.from_numpy(keys.view(np.int32)).to(gpu)
    tv = torch.arange(n, dtype=torch.int32, device=gpu)
    outs = []
    for fn in ("bh_radix_argsort", "bh_radix_argsort_noalloc"):
        ok, ov = torch.empty_like(tk), torch.empty_like(tv)
        debug_ctx.check(getattr(_lib.lib(), fn)(debug_ctx.handle, _lib.ptr(tk), _lib.ptr(tv), n, 32, _lib.ptr(ok),
                                                _lib.ptr(ov)), fn)
        outs.append((ok.cpu().numpy(), ov.cpu().numpy()))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("where", ["appended", "prefix"])
def test_culled_splats_do_not_perturb_render(gpu, where):
    """mod.rs:334-410: culled splats (opacity far below 1/255, behind the
    camera, far off screen) appended after, or prepended before (shifting
    every global id) the visible scene leave the image bit for bit the same;
    the visible splats' gradients are unchanged and the culled splats' are
    exactly zero."""
    print(f"[case] culled splats {where}", flush=True)
    cam = _cam()
    if where == "appended":
        vis = rng_scene(5_000, 1.5, (0.0, 2.5), (0.0, 3.0), 0xBEEF)
        hid = rng_scene(20_000, 1.0, (-1.0, 1.0), (-20.0, -20.0), 0xDEAD)
        hid[0][1::3, 0:3] = [0.0, 0.0, 1000.0]   # behind the camera after the view transform
        hid[0][2::3, 0:3] = [1e6, 1e6, 10.0]     # far off screen
        parts = (vis, hid)
    else:
        vis = rng_scene(4_000, 1.5, (0.0, 2.5), (0.0, 3.0), 0xC0FFEE)
        hid = rng_scene(50_000, 1.0, (-1.0, 1.0), (-20.0, -20.0), 0xF00D)
        parts = (hid, vis)
    tr, sh, op = (np.concatenate([p[i] for p in parts]) for i in range(3))
    v_out = np.random.default_rng(11).standard_normal((256, 256, 4)).astype(np.float32)
    img_v, g_v = _diff_render(gpu, *vis, cam, (256, 256), v_out)
    img_c, g_c = _diff_render(gpu, tr, sh, op, cam, (256, 256), v_out)
    assert np.array_equal(img_v.view(np.uint32), img_c.view(np.uint32)), "culled splats changed the render"
    mags = _magnitudes(*vis, cam, (256, 256), v_out)
    nv = vis[0].shape[0]
    sl = slice(0, nv) if where == "appended" else slice(tr.shape[0] - nv, tr.shape[0])
    hs = slice(nv, tr.shape[0]) if where == "appended" else slice(0, tr.shape[0] - nv)
    for name, a, b, m in zip(("v_transforms", "v_coeffs", "v_raw_opac"), g_v, g_c, mags):
        check_close(f"{name} (with culled splats)", b[sl], a, m, rtol=1e-4)
        assert np.all(b[hs] == 0.0), f"{name}: culled splats got gradients"


def test_mostly_culled_scene_sorts_only_visible(gpu):
    """The depth sort covers only the visible splats (render.rs:339-346): its
    first pass drops the culled ones.  A scene whose splats are 90 % culled
    (behind the camera, far off screen, transparent), interleaved with the
    visible ones so that culled global ids fall in every sort partition,
    renders bit for bit as the CPU restatement, on a fresh context (counts
    read back first) and again on the same context (launches queued from the
    previous forward's plan, the visible count read on the device)."""
    print("[case] 90 % culled scene", flush=True)
    cam = _cam()
    vis = rng_scene(12_000, 1.5, (0.0, 2.5), (0.0, 3.0), 0xA11CE)
    hid = rng_scene(108_000, 1.0, (-1.0, 1.0), (-1.0, 3.0), 0xB0B)
    hid[0][0::3, 0:3] = [0.0, 0.0, -1000.0]  # behind the camera
    hid[0][1::3, 0:3] = [1e6, 1e6, 10.0]     # far off screen
    hid[2][2::3] = -20.0                     # opacity far below 1/255
    order = np.random.default_rng(5).permutation(120_000)
    tr, sh, op = (np.concatenate([vis[i], hid[i]])[order] for i in range(3))
    u = uniforms_for(cam, 256, 256, tr.shape[0], 0)
    o = O.render_forward(u, tr, sh, op, O.FLAG_BWD_INFO)
    assert 10_000 <= o.num_visible <= 13_000, o.num_visible
    for run in range(2):
        g = gpu_forward(u, tr, sh, op, O.FLAG_BWD_INFO)
        compare_forward(g, o)


@pytest.mark.parametrize("case", ["crowded_bucket", "one_depth", "chunked_bucket", "wide_range", "counted_sizes"])
def test_depth_sort_bucket_extremes(gpu, case):
    """The depth sort's bucket path (one pass by the top 8 bits of the key
    range, then each bucket sorted by one workgroup) at its extremes, and the
    switch to the LSD passes, bit for bit against the restatement's stable
    sort, from a fresh context (counts read first) and from a plan:
    * crowded_bucket: 150k of 200k splats share one depth, so one bucket holds
      them all (above the 16384 pairs sorted in LDS) among spread buckets;
    * one_depth: every splat at one depth (a one-key range: the top-digit
      pass alone sorts, no bits below it);
    * chunked_bucket: 40k splats within 1e-3 of one depth among 20k spread
      over [4, 6], so one or two buckets of ~40k pairs are sorted in chunks
      by the key bits below the top digit;
    * wide_range: depths from ~0.3 to ~50 (a key range above 24 bits), which
      takes the LSD passes; the second run queues them from the plan;
    * counted_sizes: depths in [4, 6] (15 key bits below the top digit, so a
      bucket is 1/64 of depth wide and is counted), with buckets of ~3k, ~7k
      and ~11k pairs (4, 8 and 12 items a lane), one of ~14k (more than 12 a
      lane: the LSD passes), runs of 2 to 20 equal depths (put back in input
      order), and a small bucket with 40 equal depths (longer than a counted
      run may be: that bucket takes the LSD passes)."""
    print(f"[case] depth sort buckets: {case}", flush=True)
    cam = _cam()
    if case == "crowded_bucket":
        tr, sh, op = rng_scene(200_000, 1.0, (-5.0, -4.0), (0.0, 3.0), 0xD5)
        tr[:150_000, 2] = 0.25
    elif case == "one_depth":
        tr, sh, op = rng_scene(60_000, 1.0, (-5.0, -4.0), (0.0, 3.0), 0xD6)
        tr[:, 2] = -0.5
    elif case == "chunked_bucket":
        tr, sh, op = rng_scene(60_000, 1.0, (-5.0, -4.0), (0.0, 3.0), 0xD7)
        tr[:40_000, 2] = np.linspace(0.0, 1e-3, 40_000, dtype=np.float32)[np.random.default_rng(3).permutation(40_000)]
    elif case == "counted_sizes":
        rng = np.random.default_rng(5)
        # the key range from 4 to 6 exactly: 2^22 keys, 15 bits below the top digit
        parts = [np.array([4.0, 6.0]), rng.uniform(4.0, 5.999, 20_000)]
        for b, cnt in ((10, 3_000), (30, 7_000), (50, 11_000), (70, 14_000)):
            parts.append(4.0 + (b + rng.uniform(0.02, 0.98, cnt)) / 64.0)
        # runs of equal depths inside the 7k bucket, and 40 equal ones in a small bucket
        for r in range(2, 21):
            parts.append(np.full(r, 4.0 + (30 + 0.01 * r + 0.05) / 64.0))
        parts.append(np.full(40, 4.0 + (90 + 0.5) / 64.0))
        depth = np.concatenate(parts).astype(np.float32)
        depth = depth[rng.permutation(depth.shape[0])]
        tr, sh, op = rng_scene(depth.shape[0], 1.0, (-5.0, -4.0), (0.0, 3.0), 0xD9)
        z = depth - 5.0
        tr[:, 0:2] *= ((z + 5.0) / 5.0)[:, None]
        tr[:, 2] = z
    else:
        tr, sh, op = rng_scene(60_000, 1.0, (-5.0, -4.0), (0.0, 3.0), 0xD8)
        # depth z + 5 from ~0.3 to ~50, the x, y spread with it so they stay on screen
        z = np.exp(np.random.default_rng(4).uniform(np.log(0.3), np.log(50.0), 60_000)).astype(np.float32) - 5.0
        tr[:, 0:2] *= ((z + 5.0) / 5.0)[:, None]
        tr[:, 2] = z
    u = uniforms_for(cam, 256, 256, tr.shape[0], 0)
    o = O.render_forward(u, tr, sh, op, O.FLAG_BWD_INFO)
    assert o.num_visible > 0.9 * tr.shape[0], o.num_visible
    for run in range(2):
        g = gpu_forward(u, tr, sh, op, O.FLAG_BWD_INFO)
        compare_forward(g, o)


def _tiles_alpha_sums(img, tile=16):
    h, w = img.shape[:2]
    a = img[: h // tile * tile, : w // tile * tile, 3]
    return a.reshape(h // tile, tile, w // tile, tile).sum(axis=(1, 3))


def test_mega_stress_fullscreen_splats(gpu):
    """mod.rs:412-475: 120k fullscreen-sized splats at 512x512 (~120M tile
    intersections) render bit for bit the same before and after an unrelated
    render, and no tile is dropped."""
    print("[case] mega stress", flush=True)
    cam = _cam()
    tr, sh, opac = rng_scene(120_000, 0.1, (3.5, 4.0), (-3.0, -1.5), 0x5EED)
    u = uniforms_for(cam, 512, 512, tr.shape[0], 0)
    a = gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    print(f"[case] mega stress: intersections={a['num_intersections']}", flush=True)
    assert a["num_intersections"] > 50_000_000
    filler = rng_scene(100, 0.5, (-1.0, 0.5), (0.0, 1.0), 0xFACE)
    gpu_forward(uniforms_for(cam, 512, 512, 100, 0), *filler, O.FLAG_BWD_INFO)
    b = gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    assert np.array_equal(a["out_img"].view(np.uint32), b["out_img"].view(np.uint32))
    assert np.array_equal(a["tile_offsets"], b["tile_offsets"])
    assert np.all(_tiles_alpha_sums(a["out_img"]) > 1e-3), "dropped tile"


def test_many_large_splats_leave_no_tile_empty(gpu):
    """mod.rs:531-605: 200k large splats at 128x128: a finite image with
    alpha in every tile."""
    print("[case] 200k large splats", flush=True)
    rng = np.random.default_rng(0x200)
    n = 200_000
    tr = np.empty((n, 10), np.float32)
    tr[:, 0:3] = rng.uniform(-0.5, 0.5, (n, 3))
    tr[:, 3:7] = rng.uniform(-1.0, 1.0, (n, 4))
    tr[:, 7:10] = rng.uniform(-1.0, 2.5, (n, 3))
    sh = rng.uniform(0.0, 1.0, (n, 1, 3)).astype(np.float32)
    opac = rng.uniform(-2.0, 2.0, n).astype(np.float32)
    g = gpu_forward(uniforms_for(_cam(), 128, 128, n, 0), tr, sh, opac, O.FLAG_BWD_INFO)
    assert np.all(np.isfinite(g["out_img"]))
    assert int(np.sum(_tiles_alpha_sums(g["out_img"]) < 1e-4)) == 0, "dropped tiles"


def test_renders_30m_splats(gpu):
    """mod.rs:96-142: 30M splats in front of the camera at 64x64 (past any 1D
    launch limit): some survive projection, the image is finite and not empty,
    and the tile-count total equals the intersection count."""
    import torch
    from brush_amd import render as R

    print("[case] 30M splats", flush=True)
    n = 30_000_000
    g = torch.Generator(device=gpu).manual_seed(30)

    def uni(shape, lo, hi):
        return torch.rand(shape, generator=g, device=gpu, dtype=torch.float32) * (hi - lo) + lo

    tr = torch.cat([uni((n, 3), -2.0, 2.0), uni((n, 4), -1.0, 1.0), uni((n, 3), -4.0, -2.0)], 1).contiguous()
    sh = uni((n, 1, 3), 0.0, 1.0).contiguous()
    op = uni((n,), -2.0, 2.0).contiguous()
    cam = _cam()
    out = R.render(cam, (64, 64), tr, sh, op, raster_pass=R.RasterPass.Backward)
    try:
        assert out.aux.num_visible > 0, "30M splats in front of the camera, none survived projection"
        img = out.out_img.cpu().numpy()
        assert np.all(np.isfinite(img))
        assert np.any(img[..., 3] > 1e-3), "30M splats rendered to an empty image"
        total = int(out.intersect_counts.to(torch.int64).sum().item())
        assert total == out.aux.num_intersections
    finally:
        out.state.release()


_POISONS = [
    ("means", lambda t, s, o: t.__setitem__((3, 1), np.nan)),
    ("rotations", lambda t, s, o: t.__setitem__((5, 4), np.inf)),
    ("log_scales", lambda t, s, o: t.__setitem__((7, 9), np.nan)),
    ("sh_coeffs", lambda t, s, o: s.__setitem__((2, 0, 1), -np.inf)),
    ("raw_opacity", lambda t, s, o: o.__setitem__(9, np.nan)),
]


@pytest.mark.parametrize("name,poison", _POISONS, ids=[p[0] for p in _POISONS])
def test_validation_rejects_non_finite_parameters(gpu, debug_ctx, name, poison):
    """mod.rs:607-641: with BH_DEBUG_VALIDATE a NaN / Inf parameter fails the
    render with BH_ERR_NOT_FINITE naming the tensor (the reference panics);
    without it the splat is culled and the render goes on."""
    from brush_amd._lib import BrushHipError

    print(f"[case] validation {name}", flush=True)
    n = 16
    tr = np.zeros((n, 10), np.float32)
    tr[:, 0] = np.linspace(-0.5, 0.5, n)
    tr[:, 3] = 1.0
    sh = np.ones((n, 1, 3), np.float32)
    opac = np.zeros(n, np.float32)
    poison(tr, sh, opac)
    u = uniforms_for(Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.5, 0.5), 32, 32, n, 0)
    debug_ctx.set_debug()
    gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    debug_ctx.set_debug(validate=True)
    with pytest.raises(BrushHipError) as e:
        gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    assert e.value.status == STATUS_NOT_FINITE
    assert f"'{name}'" in str(e.value)


def test_validation_rejects_non_finite_gradients(gpu, debug_ctx):
    """Splats::bwd_validate (gaussian_splats.rs:384-415): a NaN upstream
    gradient on a covered pixel gives NaN parameter gradients, which the fused
    backward reports as BH_ERR_NOT_FINITE under BH_DEBUG_VALIDATE."""
    from brush_amd._lib import BrushHipError

    print("[case] validation of gradients", flush=True)
    tr, sh, opac = random_scene(41, 500, 1, log_scale=(-2.5, 0.5))
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 40.0, 48, 40)
    v_out = np.zeros((40, 48, 4), np.float32)
    v_out[20, 24, 0] = np.nan
    debug_ctx.set_debug(validate=True)
    _diff_render(gpu, tr, sh, opac, cam, (48, 40), np.zeros_like(v_out))
    with pytest.raises(BrushHipError) as e:
        _diff_render(gpu, tr, sh, opac, cam, (48, 40), v_out)
    assert e.value.status == STATUS_NOT_FINITE and "'gradient_" in str(e.value)


@pytest.mark.parametrize("fwd_flags,bwd_flags", [(1, 2), (1, 4), (3, 0), (5, 0), (1, 6)])
def test_render_backward_rejects_flags_of_another_forward(gpu, fwd_flags, bwd_flags):
    """The cutoff and the image layout belong to the forward (burn_glue.rs:
    326-328): bh_render_backward with a SMOOTH_CUTOFF or RENDER_DEPTH flag the
    forward did not have (or without one it had) returns BH_ERR_INVALID_ARG,
    and the gradient buffers are left untouched (nothing was launched)."""
    import torch
    from brush_amd import _lib
    from brush_amd import render as R

    print(f"[case] backward flags {bwd_flags} after forward flags {fwd_flags}", flush=True)
    tr, sh, opac = random_scene(43, 300, 0, log_scale=(-2.5, 0.5))
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 40.0, 32, 32)
    t = torch.from_numpy(tr).to(gpu)
    s = torch.from_numpy(sh).to(gpu)
    o = torch.from_numpy(opac).to(gpu)
    rp = R.RasterPass.BackwardSmoothCutoff if fwd_flags & 2 else R.RasterPass.Backward
    rm = R.RasterizationMode.RgbaAndDepth if fwd_flags & 4 else R.RasterizationMode.Rgba
    out = R.render(cam, (32, 32), t, s, o, R.SplatRenderMode.Default, rm, (0.0, 0.0, 0.0), rp)
    n = tr.shape[0]
    grads = [torch.full(shape, 7.0, device=gpu) for shape in ((n, 10), (n, 1, 3), (n,), (n,))]
    v_out = torch.ones_like(out.out_img)
    ctx = _lib.context()
    bg = (ctypes.c_float * 3)(0.0, 0.0, 0.0)
    st = _lib.lib().bh_render_backward(ctx.handle, out.state.handle, _lib.ptr(out.out_img),
                                       _lib.ptr(out.aux.tile_offsets), bg, _lib.ptr(t), _lib.ptr(s), _lib.ptr(o),
                                       _lib.ptr(v_out), bwd_flags, *[_lib.ptr(x) for x in grads])
    torch.cuda.synchronize()
    assert st == STATUS_INVALID_ARG
    assert "differ from the forward" in _lib.lib().bh_last_error(ctx.handle).decode()
    for x in grads:
        assert bool((x == 7.0).all())
    out.state.release()


@pytest.mark.parametrize("n", [300_000, 600_000])
def test_render_backward_writes_every_output_entry(gpu, n):
    """The fused backward writes every entry of its four output arrays: fill
    workgroups of the rasterize backward zero them and project backward
    writes the rows of splats with a gradient.  Outputs poisoned with NaN before the call
    come back finite, zero in exactly the rows that are zero when the outputs
    start at zero, and equal to those elsewhere up to the float atomics'
    order (two backwards of one forward)."""
    import torch
    from brush_amd import _lib
    from brush_amd import render as R

    print(f"[case] backward over poisoned outputs, {n} splats", flush=True)
    tr, sh, opac = random_scene(47, n, 1, log_scale=(-4.5, 0.5))
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 200.0, 256, 192)
    t = torch.from_numpy(tr).to(gpu)
    s = torch.from_numpy(sh).to(gpu)
    o = torch.from_numpy(opac).to(gpu)
    out = R.render(cam, (256, 192), t, s, o, R.SplatRenderMode.Default, R.RasterizationMode.Rgba, (0.0, 0.0, 0.0),
                   R.RasterPass.Backward)
    g = torch.Generator(device=gpu).manual_seed(5)
    v_out = torch.randn(out.out_img.shape, generator=g, device=gpu)
    ctx = _lib.context()
    bg = (ctypes.c_float * 3)(0.0, 0.0, 0.0)

    def backward(fill):
        grads = [torch.full(shape, fill, device=gpu) for shape in ((n, 10), (n, 4, 3), (n,), (n,))]
        st = _lib.lib().bh_render_backward(ctx.handle, out.state.handle, _lib.ptr(out.out_img),
                                           _lib.ptr(out.aux.tile_offsets), bg, _lib.ptr(t), _lib.ptr(s),
                                           _lib.ptr(o), _lib.ptr(v_out), 0, *[_lib.ptr(x) for x in grads])
        torch.cuda.synchronize()
        assert st == 0, _lib.lib().bh_last_error(ctx.handle).decode()
        return [x.reshape(n, -1).cpu().numpy() for x in grads]

    poisoned = backward(float("nan"))
    clean = backward(0.0)
    out.state.release()
    with_gradient = np.zeros(n, bool)
    for a, b in zip(poisoned, clean):
        assert np.isfinite(a).all()
        zero_a, zero_b = ~np.any(a != 0.0, axis=1), ~np.any(b != 0.0, axis=1)
        assert (zero_a == zero_b).all()
        with_gradient |= ~zero_b
        np.testing.assert_allclose(a, b, rtol=1e-3, atol=1e-6 * float(np.abs(b).max()))
    print(f"[tol] {with_gradient.sum()} of {n} splats with a gradient", flush=True)
    assert 0 < with_gradient.sum() < n


def test_render_backward_without_intersections_zeroes_outputs(gpu):
    """With every splat behind the camera there is no rasterize backward to
    zero the outputs: project backward writes zeros into every row of outputs
    poisoned with NaN."""
    import torch
    from brush_amd import _lib
    from brush_amd import render as R

    print("[case] backward over poisoned outputs, no splat in view", flush=True)
    n = 5000
    tr, sh, opac = random_scene(48, n, 1)
    cam = Camera.from_focal((0.0, 0.0, 3.0), (0.0, 0.0, 0.0, 1.0), 200.0, 256, 192)
    t = torch.from_numpy(tr).to(gpu)
    s = torch.from_numpy(sh).to(gpu)
    o = torch.from_numpy(opac).to(gpu)
    out = R.render(cam, (256, 192), t, s, o, R.SplatRenderMode.Default, R.RasterizationMode.Rgba, (0.0, 0.0, 0.0),
                   R.RasterPass.Backward)
    assert int(out.aux.num_visible) == 0
    v_out = torch.ones_like(out.out_img)
    ctx = _lib.context()
    bg = (ctypes.c_float * 3)(0.0, 0.0, 0.0)
    grads = [torch.full(shape, float("nan"), device=gpu) for shape in ((n, 10), (n, 4, 3), (n,), (n,))]
    st = _lib.lib().bh_render_backward(ctx.handle, out.state.handle, _lib.ptr(out.out_img),
                                       _lib.ptr(out.aux.tile_offsets), bg, _lib.ptr(t), _lib.ptr(s), _lib.ptr(o),
                                       _lib.ptr(v_out), 0, *[_lib.ptr(x) for x in grads])
    torch.cuda.synchronize()
    assert st == 0, _lib.lib().bh_last_error(ctx.handle).decode()
    out.state.release()
    for x in grads:
        assert bool((x == 0.0).all())


@pytest.mark.parametrize("w,h,tile16x8", [(3840, 2160, False), (2048, 1080, True), (4096, 2160, True)])
def test_more_than_16384_tiles(gpu, w, h, tile16x8):
    """Frames with more tiles than the tile-order kernel keeps in registers
    (16 x 1024): 3840x2160 with 16x16 tiles (32400 tiles), 2048x1080 with
    16x8 tiles (17280 tiles), and 4096x2160 with 16x8 tiles (69120 tiles:
    from 2^16 tiles the tile sort's keys are 32-bit throughout).  Forward bit
    for bit, every tile's offsets before and after the blend, and the fused
    backward entry by entry to rtol 1e-3 plus the entry's rounding noise,
    against the CPU restatement."""
    print(f"[case] {w}x{h} tiles 16x{8 if tile16x8 else 16}", flush=True)
    tr, sh, opac = random_scene(57, 20_000, 1, mean_range=1.2, log_scale=(-3.5, 0.6))
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.45 * w, w, h)
    u = uniforms_for(cam, w, h, tr.shape[0], 1)
    flags = O.FLAG_BWD_INFO | (O.FLAG_TILE_16X8 if tile16x8 else 0)
    o = O.render_forward(u, tr, sh, opac, flags)
    g = gpu_forward(u, tr, sh, opac, flags)
    assert o.uniforms["tile_bw"] * o.uniforms["tile_bh"] > 16384
    compare_forward(g, o)
    import torch
    from brush_amd import render as R

    rasterizer = R.Rasterizer.Candidate if tile16x8 else R.Rasterizer.Legacy
    t = torch.from_numpy(tr).to(gpu).requires_grad_(True)
    s = torch.from_numpy(sh).to(gpu).requires_grad_(True)
    op = torch.from_numpy(opac).to(gpu).requires_grad_(True)
    v_out = np.random.default_rng(3).standard_normal((h, w, 4)).astype(np.float32)
    with keep_lanes():
        res = R.render_splats_diff(R.Splats(t, s, op), cam, (w, h), rasterizer=rasterizer)
        res.img.backward(torch.from_numpy(v_out).to(gpu))
    want = OracleGrads(o, tr, sh, opac, v_out, O.FLAG_REFINE_WEIGHT)
    grads = {"v_transforms": t.grad.cpu().numpy(), "v_coeffs": s.grad.cpu().numpy(),
             "v_raw_opac": op.grad.cpu().numpy(), "v_refine": res._cfg.refine_weight.cpu().numpy()}
    check_fused_backward(f"{w}x{h}", res._cfg.state, tr, sh, opac, grads, want)


def test_second_backward_of_one_forward(gpu):
    """The forward zeroes the gradient rows its first backward uses; a second
    backward of the same forward (retain_graph) zeroes its own and matches the
    first entry by entry (float atomics: to rtol 1e-5 plus the entry's
    rounding noise), and both match the CPU restatement."""
    import torch
    from brush_amd import render as R

    w, h = 320, 240
    print(f"[case] two backwards of one forward, {w}x{h}", flush=True)
    tr, sh, opac = random_scene(61, 3000, 1, mean_range=1.0, log_scale=(-3.0, 0.5))
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.8 * w, w, h)
    t = torch.from_numpy(tr).to(gpu).requires_grad_(True)
    s = torch.from_numpy(sh).to(gpu).requires_grad_(True)
    op = torch.from_numpy(opac).to(gpu).requires_grad_(True)
    res = R.render_splats_diff(R.Splats(t, s, op), cam, (w, h))
    v_out = torch.from_numpy(np.random.default_rng(5).standard_normal((h, w, 4)).astype(np.float32)).to(gpu)
    res.img.backward(v_out, retain_graph=True)
    first = [x.grad.clone() for x in (t, s, op)]
    for x in (t, s, op):
        x.grad = None
    res.img.backward(v_out)
    u = uniforms_for(cam, w, h, tr.shape[0], 1)
    o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    want = OracleGrads(o, tr, sh, opac, v_out.cpu().numpy(), O.FLAG_REFINE_WEIGHT)
    noise = (want.noise_transforms, want.noise_coeffs, want.noise_raw_opac)
    refs = (want.v_transforms, want.v_coeffs, want.v_raw_opac)
    for name, a, b, n, ref in zip(("v_transforms", "v_coeffs", "v_raw_opac"), first, (t.grad, s.grad, op.grad),
                                  noise, refs):
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert np.all(np.isfinite(b)), name
        assert np.abs(a).max() > 0.0, name
        check_close(f"{name} (second backward vs first)", b, a, n, rtol=1e-5)
        check_close(f"{name} (second backward)", b, ref, n)


def _validated_diff(gpu, tr, sh, opac, cam, size, mip=False):
    """render_splats_diff + backward of mean(image) on a context in
    BH_DEBUG_VALIDATE mode: a non-finite parameter or gradient raises."""
    import torch
    from brush_amd import render as R

    t = torch.from_numpy(np.ascontiguousarray(tr)).to(gpu).requires_grad_(True)
    s = torch.from_numpy(np.ascontiguousarray(sh)).to(gpu).requires_grad_(True)
    o = torch.from_numpy(np.ascontiguousarray(opac)).to(gpu).requires_grad_(True)
    res = R.render_splats_diff(R.Splats(t, s, o, render_mip=mip), cam, size)
    res.img.mean().backward()
    torch.cuda.synchronize()
    grads = (t.grad.cpu().numpy(), s.grad.cpu().numpy(), o.grad.cpu().numpy(), res._cfg.refine_weight.cpu().numpy())
    for g in grads:
        assert np.all(np.isfinite(g))
    return res, grads


@pytest.mark.parametrize("ls", [-20.0, -5.0, 0.0, 5.0, 15.0, 30.0, 40.0])
def test_bwd_extreme_inputs_stay_finite(gpu, debug_ctx, ls):
    """fuzz.rs:519-551 on the fused backward, under BH_DEBUG_VALIDATE: eight
    splats at the origin with log-scales up to 40 and SH DC magnitudes up to
    f32::MAX / 2 render with every splat visible and every gradient finite;
    the forward is bit for bit the restatement's."""
    from tests.test_oracle import STD_CAM

    print(f"[case] extreme inputs log_scale={ls}", flush=True)
    n = 8
    tr = np.tile(np.array([0, 0, 3, 1, 0, 0, 0, ls, ls, ls], np.float32), (n, 1))
    debug_ctx.set_debug(validate=True)
    for mag in (0.1, 10.0, 1e6, 3.4028235e38 / 2):
        sh = np.tile(np.array([mag, -mag, mag], np.float32), (n, 1)).reshape(n, 1, 3)
        opac = np.full(n, 2.0, np.float32)
        res, _ = _validated_diff(gpu, tr, sh, opac, STD_CAM, (64, 64))
        assert res.num_visible == n, (ls, mag)
        u = uniforms_for(STD_CAM, 64, 64, n, 0)
        o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
        assert np.array_equal(res.img.detach().cpu().numpy().view(np.uint32), o.out_img.view(np.uint32)), (ls, mag)


def test_bwd_random_scenes_gradients_are_finite(gpu, debug_ctx):
    """fuzz.rs:492-517 on the fused backward, under BH_DEBUG_VALIDATE: 100
    random scenes (4-255 splats) seen from cameras anywhere, image sides
    16-127, Mip mode 30 % of the time; every gradient finite and equal to
    the restatement's to rtol 1e-3 plus its rounding noise."""
    from brush_amd.camera import project_uniforms
    from tests.helpers import OracleGrads, compare_dense
    from tests.test_oracle import _fuzz_finite_scene, _fuzz_rand_cam
    from tests.test_oracle_fuzz import MASK64, Sm64

    debug_ctx.set_debug(validate=True)
    live = 0
    for seed in range(100):
        rng = Sm64(0xBDBDBDBD ^ ((seed * 0xA5A5CAFE) & MASK64))
        n = rng.usize_in(4, 256)
        w, h = rng.usize_in(16, 128), rng.usize_in(16, 128)
        cam = _fuzz_rand_cam(rng)
        mip = bool(rng.f01() < 0.3)
        tr, sh, opac = _fuzz_finite_scene(seed, n)
        res, g = _validated_diff(gpu, tr, sh, opac, cam, (w, h), mip)
        u = project_uniforms(cam, w, h, n, 0)
        flags = O.FLAG_BWD_INFO | (O.FLAG_MIP if mip else 0)
        o = O.render_forward(u, tr, sh, opac, flags)
        assert res.num_visible == o.num_visible, seed
        want = OracleGrads(o, tr, sh, opac, np.full((h, w, 4), 1.0 / (h * w * 4), np.float32),
                           O.FLAG_REFINE_WEIGHT, mip=mip)
        compare_dense(f"seed {seed} ", {"v_transforms": g[0], "v_coeffs": g[1], "v_raw_opac": g[2]}, want)
        live += bool(np.any(g[0] != 0))
    assert live > 10
