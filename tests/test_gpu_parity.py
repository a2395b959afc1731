"""GPU parity: every HIP kernel against the CPU restatement on identical inputs.

Integer outputs (visibility, tile counts, sorted tile ids and compact ids,
tile offsets before and after the blend) and the projected rows are compared
bit for bit; so is the image, because the blend uses the same reproducible
exp() as the checker.  Gradients are compared entry by entry to rtol 1e-3
plus the entry's own f32 rounding noise (tests/helpers.py: rasterize
backward sums per-block partials with float atomics, whose order varies);
project backward fed the same v_combined is compared bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import (OracleGrads, assert_bits_equal, check_fused_backward, compare_forward, compare_lanes,
                           gpu_forward, gsplat_case, keep_lanes, random_scene, raster_oracle_scene, uniforms_for)
from brush_amd.synthetic import CONFIGS, generate_splats, generate_v_output

pytestmark = pytest.mark.gpu


def _dev(gpu):
    return gpu


# ---- primitives ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,bits", [(1, 32), (255, 8), (4096, 13), (4097, 32), (65537, 4), (100000, 0),
                                    (300001, 17), (1 << 20, 32), (3_000_017, 24), (5_000_001, 13)])
def test_radix_argsort_matches_stable_sort(gpu, n, bits):
    import torch
    from brush_amd import _lib

    print(f"[case] radix_argsort n={n} bits={bits}", flush=True)
    rng = np.random.default_rng(n * 7 + bits)
    keys = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    if bits and bits < 32:
        keys[: n // 2] &= np.uint32((1 << bits) - 1)  # many keys inside the width, some with high bits
    vals = np.arange(n, dtype=np.uint32)
    ctx = _lib.context()
    tk = torch.from_numpy(keys.view(np.int32)).to(gpu)
    tv = torch.from_numpy(vals.view(np.int32)).to(gpu)
    ok = torch.empty_like(tk)
    ov = torch.empty_like(tv)
    ctx.check(_lib.lib().bh_radix_argsort(ctx.handle, _lib.ptr(tk), _lib.ptr(tv), n, bits, _lib.ptr(ok),
                                          _lib.ptr(ov)))
    # brush-sort orders by the low 4*ceil(bits/4) bits
    width = 4 * ((bits + 3) // 4)
    ek, ev = O.stable_sort(keys, vals, width)
    assert_bits_equal("keys", ok.cpu().numpy().view(np.uint32), ek)
    assert_bits_equal("vals", ov.cpu().numpy().view(np.uint32), ev)


@pytest.mark.parametrize("n", [4, 255, 256, 257, 1024, 4095, 4096, 4097, 41000, 1 << 20, 3_000_001, 9_000_001])
def test_prefix_sum_closed_form(gpu, n):
    import torch
    from brush_amd import _lib

    print(f"[case] prefix_sum n={n}", flush=True)
    rng = np.random.default_rng(n)
    x = rng.integers(0, 64, size=n).astype(np.uint32)
    ctx = _lib.context()
    tx = torch.from_numpy(x.view(np.int32)).to(gpu)
    out = torch.empty_like(tx)
    ctx.check(_lib.lib().bh_prefix_sum(ctx.handle, _lib.ptr(tx), _lib.ptr(out), n))
    assert_bits_equal("scan", out.cpu().numpy().view(np.uint32), np.cumsum(x, dtype=np.uint64).astype(np.uint32))


def test_tile_offsets_run_length_fixture(gpu):
    """get_tile_offset.rs:88-129: runs [31,1,223,1,1791,1,17,0] + 13 sentinel rows."""
    import torch
    from brush_amd import _lib

    runs = [31, 1, 223, 1, 1791, 1, 17, 0]
    ids, expected = [], np.zeros(16, np.uint32)
    for t, r in enumerate(runs):
        if r == 0:
            continue
        expected[2 * t] = len(ids)
        ids += [t] * r
        expected[2 * t + 1] = len(ids)
    ids += [8] * 13
    ids = np.array(ids, np.uint32)
    ctx = _lib.context()
    ti = torch.from_numpy(ids.view(np.int32)).to(gpu)
    off = torch.full((16,), -1, dtype=torch.int32, device=gpu)
    ctx.check(_lib.lib().bh_get_tile_offsets(ctx.handle, _lib.ptr(ti), ids.size, 8, _lib.ptr(off)))
    assert_bits_equal("offsets", off.cpu().numpy().view(np.uint32), expected)


# ---- forward ----------------------------------------------------------------------------------

def test_gsplat_goldens_forward(gpu):
    for name in ["tiny_case", "basic_case"]:
        print(f"[case] gsplat {name}", flush=True)
        cam, (w, h), tr, sh, opac, ref = gsplat_case(name)
        u = uniforms_for(cam, w, h, tr.shape[0], 3)
        g = gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
        o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
        compare_forward(g, o)
        err = np.abs(g["out_img"] - ref)
        assert np.all(err < 1e-5 + 1e-2 * np.abs(ref)), f"{name} vs gsplat: max err {err.max()}"


@pytest.mark.parametrize("size", [(23, 19), (15, 7), (16, 8), (17, 9), (9, 17)])
@pytest.mark.parametrize("flags", [1, 3])
def test_raster_oracle_scene(gpu, size, flags):
    """raster_oracle.rs:271-397 scenes and sizes, hard and smooth cutoff."""
    print(f"[case] raster_oracle size={size} flags={flags}", flush=True)
    cam, tr, sh, opac, bg = raster_oracle_scene()
    w, h = size
    u = uniforms_for(cam, w, h, 6, 0)
    g = gpu_forward(u, tr, sh, opac, flags, bg)
    o = O.render_forward(u, tr, sh, opac, flags, bg)
    compare_forward(g, o)
    ref = O.rasterize_reference(o.projected[: o.num_visible], w, h, bg, bool(flags & 2))
    assert np.max(np.abs(g["out_img"] - ref)) <= 2e-5


@pytest.mark.parametrize("seed,n,deg,flags", [(1, 1000, 0, 1), (2, 5000, 3, 1), (3, 3000, 1, 9), (4, 2000, 2, 5),
                                              (5, 4000, 4, 1), (6, 2500, 3, 0), (7, 20000, 3, 3)])
def test_random_scene_forward(gpu, seed, n, deg, flags):
    print(f"[case] random forward seed={seed} n={n} deg={deg} flags={flags}", flush=True)
    tr, sh, opac = random_scene(1000 + seed, n, deg, log_scale=(-3.0, 0.6))
    from brush_amd.camera import Camera

    cam = Camera.from_focal((0.1, -0.2, -3.0), (0.0, 0.0, 0.0, 1.0), 70.0, 97, 75)
    u = uniforms_for(cam, 97, 75, n, deg)
    g = gpu_forward(u, tr, sh, opac, flags, (0.1, 0.2, 0.3))
    o = O.render_forward(u, tr, sh, opac, flags, (0.1, 0.2, 0.3))
    compare_forward(g, o)


def test_config0_forward_full_size(gpu):
    """BASELINE config 0 (100k splats, SH0, 256x256) bit for bit."""
    w = CONFIGS[0]
    print(f"[case] config0 forward {w.name}", flush=True)
    tr, sh, opac = generate_splats(w)
    u = uniforms_for(w.camera(), w.img_w, w.img_h, w.n, w.sh_degree)
    g = gpu_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    compare_forward(g, o)


def test_empty_and_culled_scenes(gpu):
    """render.rs:145-253 empty contract; fuzz.rs:330-448 all-bad geometry."""
    from brush_amd.camera import Camera

    cam = Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.5, 0.5)
    u = uniforms_for(cam, 64, 64, 0, 0)
    for flags in (0, 1):
        g = gpu_forward(u, np.zeros((0, 10), np.float32), np.zeros((0, 1, 3), np.float32),
                        np.zeros((0,), np.float32), flags, (0.25, 0.5, 0.75))
        assert g["num_visible"] == 0 and g["num_intersections"] == 0
        if flags:
            assert np.all(g["out_img"][..., :3] == np.array([0.25, 0.5, 0.75], np.float32))
            assert np.all(g["out_img"][..., 3] == 0)
        else:
            expect = (63) | (127 << 8) | (191 << 16)
            assert np.all(g["out_img"] == expect)
        assert np.all(g["tile_offsets"] == 0)
    n = 16
    base_tr = np.tile(np.array([0, 0, 3, 1, 0, 0, 0, 0, 0, 0], np.float32), (n, 1))
    cases = {
        "nan_positions": lambda t: t.__setitem__((slice(None), slice(0, 3)), np.nan),
        "inf_positions": lambda t: t.__setitem__((slice(None), 0), np.inf),
        "zero_quats": lambda t: t.__setitem__((slice(None), slice(3, 7)), 0.0),
        "nan_quats": lambda t: t.__setitem__((slice(None), 4), np.nan),
        "nan_scales": lambda t: t.__setitem__((slice(None), 8), np.nan),
        "inf_scales": lambda t: t.__setitem__((slice(None), slice(7, 10)), 120.0),
        "behind_camera": lambda t: t.__setitem__((slice(None), 2), -3.5),
    }
    for name, poison in cases.items():
        tr = base_tr.copy()
        poison(tr)
        sh = np.full((n, 1, 3), 0.5, np.float32)
        opac = np.zeros(n, np.float32)
        g = gpu_forward(u, tr, sh, opac, 1)
        assert g["num_visible"] == 0 and g["num_intersections"] == 0, name
    g = gpu_forward(u, base_tr, np.full((n, 1, 3), 0.5, np.float32), np.full(n, np.nan, np.float32), 1)
    assert g["num_visible"] == 0


def test_extreme_but_valid_stays_visible(gpu):
    """fuzz.rs:450-490."""
    from brush_amd.camera import Camera

    cam = Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.5, 0.5)
    n = 4
    u = uniforms_for(cam, 64, 64, n, 0)
    for ls in [-30.0, -10.0, 0.0, 10.0, 20.0, 30.0, 40.0]:
        tr = np.tile(np.array([0, 0, 3, 1, 0, 0, 0, ls, ls, ls], np.float32), (n, 1))
        g = gpu_forward(u, tr, np.full((n, 1, 3), 0.5, np.float32), np.full(n, 2.0, np.float32), 0)
        o = O.render_forward(u, tr, np.full((n, 1, 3), 0.5, np.float32), np.full(n, 2.0, np.float32), 0)
        assert g["num_visible"] == n, f"log_scale={ls} over-culled"
        compare_forward(g, o)


def test_poison_fuzz_single_slot(gpu):
    """fuzz.rs:267-302: every (slot, poison) combination, counts match the checker."""
    from brush_amd.camera import Camera

    poisons = [np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 1.1754944e-38, 5.877472e-39, 1e-40, 1.1920929e-07,
               1e38, -1e38, 3.4028235e38, -3.4028235e38, 1e20, -1e20, 1.0, -1.0, 0.01, 1e10, 1.0 / 255.0, 16.0]
    cam = Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.5, 0.5)
    n = 120
    u = uniforms_for(cam, 48, 48, n, 0)
    for slot in range(14):
        for p in poisons:
            tr = np.tile(np.array([0, 0, 3, 1, 0, 0, 0, -1, -1, -1], np.float32), (n, 1))
            sh = np.full((n, 1, 3), 0.5, np.float32)
            opac = np.full(n, 2.0, np.float32)
            if slot < 10:
                tr[0, slot] = p
            elif slot < 13:
                sh[0, 0, slot - 10] = p
            else:
                opac[0] = p
            g = gpu_forward(u, tr, sh, opac, 0)
            o = O.render_forward(u, tr, sh, opac, 0)
            assert g["num_visible"] == o.num_visible, (slot, p)
            assert g["num_intersections"] == o.num_intersections, (slot, p)
            assert_bits_equal(f"img slot={slot} p={p}", g["out_img"], o.out_img)


# ---- backward -----------------------------------------------------------------------------------

def _gpu_backward(g, v_output, flags_bwd, bg, tr, sh, opac, mode_mip=False):
    import torch
    from brush_amd import render as R

    out = g["out"]
    dev = out.out_img.device
    vo = torch.from_numpy(np.ascontiguousarray(v_output)).to(dev)
    v_comb = R.rasterize_bwd(out.out_img, out.projected_splats, out.compact_gid_from_isect, out.aux.tile_offsets,
                             bg, out.aux.img_size, vo, bool(flags_bwd & 2), bool(flags_bwd & 4),
                             bool(flags_bwd & 16))
    return v_comb


@pytest.mark.parametrize("seed,n,deg,flags", [(11, 800, 3, 1), (12, 3000, 0, 1), (13, 2000, 3, 3),
                                              (14, 1500, 2, 5), (15, 1200, 1, 9)])
def test_backward_matches_checker(gpu, seed, n, deg, flags):
    import torch
    from brush_amd import render as R
    from brush_amd.camera import Camera

    print(f"[case] backward seed={seed} n={n} deg={deg} flags={flags}", flush=True)
    tr, sh, opac = random_scene(2000 + seed, n, deg, log_scale=(-3.0, 0.6))
    cam = Camera.from_focal((0.1, -0.2, -3.0), (0.0, 0.0, 0.0, 1.0), 70.0, 61, 53)
    u = uniforms_for(cam, 61, 53, n, deg)
    bg = (0.1, 0.2, 0.3)
    g = gpu_forward(u, tr, sh, opac, flags, bg)
    o = O.render_forward(u, tr, sh, opac, flags, bg)
    compare_forward(g, o)
    chans = 5 if flags & 4 else 4
    rng = np.random.default_rng(seed)
    v_out = rng.standard_normal((53, 61, chans)).astype(np.float32)
    bflags = (flags & 6) | 16
    vc_gpu = _gpu_backward(g, v_out, bflags, bg, tr, sh, opac).cpu().numpy()
    want = OracleGrads(o, tr, sh, opac, v_out, bflags, bg, mip=bool(flags & 8), dense=False)
    compare_lanes("v_combined", vc_gpu, want)
    vc_ref = want.v_combined
    # project backward fed the checker's v_combined: deterministic per splat, bit for bit
    dev = gpu
    mode = R.SplatRenderMode.Mip if flags & 8 else R.SplatRenderMode.Default
    grads = R.project_bwd(torch.from_numpy(tr).to(dev), torch.from_numpy(sh).to(dev), torch.from_numpy(opac).to(dev),
                          g["out"].global_from_compact_gid, g["out"].project_uniforms, mode,
                          torch.from_numpy(vc_ref).to(dev))
    vt, vcoef, vo, vr = O.project_backward(o, tr, sh, opac, vc_ref, mip=bool(flags & 8))
    assert_bits_equal("v_transforms", grads.v_transforms.cpu().numpy(), vt)
    assert_bits_equal("v_coeffs", grads.v_coeffs.cpu().numpy(), vcoef)
    assert_bits_equal("v_raw_opac", grads.v_raw_opac.cpu().numpy(), vo)
    assert_bits_equal("v_refine", grads.v_refine_weight.cpu().numpy(), vr)


@pytest.mark.parametrize("smooth,depth,mip,refine", [(False, False, False, True), (True, False, False, True),
                                                      (False, True, False, False), (True, True, True, True),
                                                      (False, False, True, False)])
def test_autograd_end_to_end(gpu, smooth, depth, mip, refine):
    """render_splats_diff + loss.backward() (the fused bh_render_backward, which
    accumulates the gradient lanes per global id) vs the checker's rasterize
    backward followed by project backward, for every backward flag."""
    import torch
    from brush_amd import render as R
    from brush_amd.camera import Camera

    print(f"[case] autograd smooth={smooth} depth={depth} mip={mip} refine={refine}", flush=True)
    n, deg = 2000, 3
    tr, sh, opac = random_scene(3001, n, deg, log_scale=(-3.0, 0.6))
    cam = Camera.from_focal((0.0, 0.1, -3.0), (0.0, 0.0, 0.0, 1.0), 80.0, 64, 48)
    t = torch.from_numpy(tr).to(gpu).requires_grad_(True)
    s = torch.from_numpy(sh).to(gpu).requires_grad_(True)
    op = torch.from_numpy(opac).to(gpu).requires_grad_(True)
    splats = R.Splats(t, s, op, render_mip=mip)
    rpass = R.RasterPass.BackwardSmoothCutoff if smooth else R.RasterPass.Backward
    rmode = R.RasterizationMode.RgbaAndDepth if depth else R.RasterizationMode.Rgba
    chans = 5 if depth else 4
    rng = np.random.default_rng(5)
    w = torch.from_numpy(rng.standard_normal((48, 64, chans)).astype(np.float32)).to(gpu)
    with keep_lanes():
        res = R.render_splats_diff(splats, cam, (64, 48), (0.1, 0.0, 0.2), compute_refine_weight=refine,
                                   raster_pass=rpass, raster_mode=rmode)
        loss = (res.img * w).sum()
        loss.backward()
    u = uniforms_for(cam, 64, 48, n, deg)
    fflags = O.FLAG_BWD_INFO | (O.FLAG_SMOOTH_CUTOFF if smooth else 0) | (O.FLAG_RENDER_DEPTH if depth else 0) | \
        (O.FLAG_MIP if mip else 0)
    o = O.render_forward(u, tr, sh, opac, fflags, (0.1, 0.0, 0.2))
    compare_forward(gpu_forward(u, tr, sh, opac, fflags, (0.1, 0.0, 0.2)), o)
    bflags = (fflags & 6) | (O.FLAG_REFINE_WEIGHT if refine else 0)
    want = OracleGrads(o, tr, sh, opac, w.cpu().numpy(), bflags, (0.1, 0.0, 0.2), mip=mip)
    grads = {"v_transforms": t.grad.cpu().numpy(), "v_coeffs": s.grad.cpu().numpy(),
             "v_raw_opac": op.grad.cpu().numpy(), "v_refine": res._cfg.refine_weight.cpu().numpy()}
    check_fused_backward("autograd", res._cfg.state, tr, sh, opac, grads, want)
    if not refine:
        assert not res._cfg.refine_weight.any().item()


def test_autograd_fully_culled_scene(gpu):
    """A scene whose splats are all behind the camera: the fused backward
    writes exactly-zero dense gradients (render.rs:145-253 empty contract)."""
    import torch
    from brush_amd import render as R
    from brush_amd.camera import Camera

    tr, sh, opac = random_scene(3002, 500, 1)
    tr[:, 2] = -10.0  # z of every mean behind a camera at z = -3 looking down +z
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 50.0, 40, 30)
    t = torch.from_numpy(tr).to(gpu).requires_grad_(True)
    s = torch.from_numpy(sh).to(gpu).requires_grad_(True)
    op = torch.from_numpy(opac).to(gpu).requires_grad_(True)
    res = R.render_splats_diff(R.Splats(t, s, op), cam, (40, 30))
    assert res.num_visible == 0
    res.img.sum().backward()
    for g in (t.grad, s.grad, op.grad, res._cfg.refine_weight):
        assert g is not None and not g.any().item()


@pytest.mark.parametrize("flags", [1, 3])
def test_alpha_cutoff_boundary_scene(gpu, flags):
    """Low opacities put many (splat, pixel) pairs right at alpha = 1/255 (and
    inside the smooth band): the blend's early reject must not change any
    decision, so image and post-blend tile ends stay bit-exact."""
    from brush_amd.camera import Camera

    print(f"[case] cutoff boundary flags={flags}", flush=True)
    tr, sh, opac = random_scene(4242 + flags, 6000, 1, log_scale=(-2.5, 0.5), opac=(-4.8, 0.6))
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 60.0, 80, 64)
    u = uniforms_for(cam, 80, 64, tr.shape[0], 1)
    g = gpu_forward(u, tr, sh, opac, flags, (0.2, 0.1, 0.0))
    o = O.render_forward(u, tr, sh, opac, flags, (0.2, 0.1, 0.0))
    compare_forward(g, o)
    v_out = np.random.default_rng(flags).standard_normal((64, 80, 4)).astype(np.float32)
    vc_gpu = _gpu_backward(g, v_out, (flags & 2) | 16, (0.2, 0.1, 0.0), tr, sh, opac).cpu().numpy()
    compare_lanes("v_combined", vc_gpu, OracleGrads(o, tr, sh, opac, v_out, (flags & 2) | 16, (0.2, 0.1, 0.0),
                                                    dense=False))


@pytest.mark.parametrize("flags", [1, 3])
def test_needle_splats_strip_culling(gpu, flags):
    """Very anisotropic, rotated splats (the worst case for cancellation in the
    power) through the per-strip culling of both blend kernels: image, tile
    ends and gradients still match the checker, which culls nothing."""
    from brush_amd.camera import Camera

    print(f"[case] needle splats flags={flags}", flush=True)
    rng = np.random.default_rng(99 + flags)
    n = 3000
    tr = np.zeros((n, 10), np.float32)
    tr[:, 0:3] = rng.uniform(-0.9, 0.9, (n, 3))
    q = rng.standard_normal((n, 4))
    tr[:, 3:7] = q / np.linalg.norm(q, axis=1, keepdims=True)
    tr[:, 7] = rng.uniform(-1.5, -0.5, n)
    tr[:, 8:10] = rng.uniform(-7.0, -5.0, (n, 2))
    sh = rng.uniform(0.0, 0.8, (n, 1, 3)).astype(np.float32)
    opac = rng.uniform(-2.0, 3.0, n).astype(np.float32)
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 90.0, 96, 80)
    u = uniforms_for(cam, 96, 80, n, 0)
    g = gpu_forward(u, tr, sh, opac, flags)
    o = O.render_forward(u, tr, sh, opac, flags)
    compare_forward(g, o)
    v_out = rng.standard_normal((80, 96, 4)).astype(np.float32)
    vc_gpu = _gpu_backward(g, v_out, (flags & 2) | 16, (0.0, 0.0, 0.0), tr, sh, opac).cpu().numpy()
    compare_lanes("v_combined", vc_gpu, OracleGrads(o, tr, sh, opac, v_out, (flags & 2) | 16, dense=False))


def test_workspace_stops_growing_when_sizes_creep(gpu):
    """A scene that grows a little from call to call (as a trained scene's
    intersection count does) reuses the library's cached workspace: after
    the first calls, the pool holds no more memory than it did."""
    import torch
    from brush_amd import _lib
    from brush_amd import render as R
    from brush_amd.camera import Camera

    tr, sh, op = random_scene(9090, 60000, 1, log_scale=(-3.0, 0.5))
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 300.0, 256, 256)
    # start from an empty pool: what earlier tests cached would serve some sizes
    _lib.context(0).release_workspace()
    sizes = []
    for k in range(12):
        n = 50000 + 500 * k  # more splats, more intersections, every call
        t = torch.from_numpy(tr[:n].copy()).to(gpu)
        s = torch.from_numpy(sh[:n].copy()).to(gpu)
        o = torch.from_numpy(op[:n].copy()).to(gpu)
        out = R.render(cam, (256, 256), t, s, o, raster_pass=R.RasterPass.Backward)
        out.state.release()
        torch.cuda.synchronize()
        sizes.append(_lib.context(0).workspace_bytes())
    print(f"[case] workspace bytes per call {sizes}", flush=True)
    assert sizes[-1] <= sizes[4], sizes
