"""The forward's planned launches against its exact ones.

bh_render_forward queues the launches that depend on its counts (visible
splats, intersections, depth-key range) in one of two ways: sized from the
counts read back first, the reference's order (render.rs:309-329), selected
here with BH_DEBUG_EXACT_SIZES; or, by default after the first forward on a
context, sized from the previous forward's plan with the kernels reading the
counts from device memory, the host checking them only after queueing and
queueing the exact launches again when they do not fit.  Every output must be
bit for bit the same either way:

* along a sequence of scenes whose counts outgrow the plan in each way it can
  (four times the intersections, a wider depth-key range, no visible splat)
  and fit it (the same scene again, a smaller scene), with the rasterize
  launches counted to show which renders were re-queued;
* at the north-star size (config 1, 1M splats at 1080p), where the timed loop
  of the benchmark runs the planned launches;
* for the fused backward of a planned forward (the record of contributing
  pairs sized for the plan), and of a planned forward that outgrew its plan
  and was queued again (its gradient rows allocated and zeroed anew), to the
  order of float atomics.
"""
import numpy as np
import pytest

from brush_amd.camera import Camera
from brush_amd.synthetic import CONFIGS, generate_splats
from oracle import oracle as O
from tests.helpers import OracleGrads, check_close, check_fused_backward, gpu_forward, keep_lanes, rng_scene, uniforms_for

pytestmark = pytest.mark.gpu

SIZE = (192, 160)


def _cam():
    return Camera((0.0, 0.0, -5.0), (0.0, 0.0, 0.0, 1.0), 0.5, 0.5)


@pytest.fixture
def ctx(gpu):
    from brush_amd import _lib

    c = _lib.context()
    yield c
    c.set_timing(False)
    c.set_debug()


def _forward(ctx, u, scene, exact):
    """Every forward output (numpy) and how many rasterize launches it made."""
    import torch

    ctx.set_debug(exact_sizes=exact)
    ctx.reset_timings()
    ctx.set_timing(True, only="rasterize")
    g = gpu_forward(u, *scene, O.FLAG_BWD_INFO)
    torch.cuda.synchronize()
    launches = ctx.read_timings().get("rasterize", (0, 0.0))[0]
    ctx.set_timing(False)
    ctx.set_debug()
    g.pop("out")
    return g, launches


def _assert_same(tag, a, b):
    for k, v in a.items():
        if isinstance(v, np.ndarray):
            x, y = v, b[k]
            assert x.shape == y.shape, f"{tag}: {k} shape {x.shape} vs {y.shape}"
            if x.dtype == np.float32:
                x, y = x.view(np.uint32), y.view(np.uint32)
            bad = np.nonzero(x.reshape(-1) != y.reshape(-1))[0]
            assert bad.size == 0, f"{tag}: {k} differs at {bad.size} of {x.size}, first {bad[:4]}"
        else:
            assert v == b[k], f"{tag}: {k} {v} vs {b[k]}"


def _key_width(g):
    """Bits of the depth-key range of the visible splats (their f32 depths)."""
    if g["num_visible"] == 0:
        return 0
    bits = g["depths"].view(np.uint32).astype(np.int64)
    return int(bits.max() - bits.min() + 1).bit_length()


def test_plan_outgrown_and_fitting_renders_match_exact(ctx):
    scenes = {
        "small": rng_scene(2_000, 1.5, (-3.0, -1.5), (-1.0, 2.0), 0x51),
        "large": rng_scene(20_000, 1.5, (-2.5, -0.5), (-1.0, 2.0), 0x52),
        "narrow_depth": rng_scene(30_000, 0.03, (-3.0, -1.0), (-1.0, 2.0), 0x53),
        "culled": rng_scene(3_000, 1.5, (-3.0, -1.5), (-20.0, -20.0), 0x54),
    }
    cam = _cam()
    u = {k: uniforms_for(cam, SIZE[0], SIZE[1], v[0].shape[0], 0) for k, v in scenes.items()}
    exact = {}
    for k, sc in scenes.items():
        print(f"[case] exact forward {k}", flush=True)
        exact[k], launches = _forward(ctx, u[k], sc, exact=True)
        assert launches == 1
    e = exact
    # the sequence's premises
    # more than any plan made for "small" (its count plus 1/8 plus 4096, in 4096 steps) holds
    assert e["large"]["num_intersections"] > 4 * e["small"]["num_intersections"] + 8192
    assert e["small"]["num_intersections"] > 0
    assert _key_width(e["narrow_depth"]) < _key_width(e["small"])
    assert e["small"]["num_intersections"] < e["narrow_depth"]["num_intersections"]
    assert e["culled"]["num_visible"] == 0
    # (scene, whether it must be queued again: None when the plan could go either way)
    seq = [("small", None), ("small", False), ("large", True), ("large", False), ("small", False),
           ("narrow_depth", None), ("small", True), ("culled", True), ("small", None), ("large", None),
           ("large", False)]
    requeued = 0
    for i, (k, must) in enumerate(seq):
        print(f"[case] planned forward {i}: {k}", flush=True)
        g, launches = _forward(ctx, u[k], scenes[k], exact=False)
        _assert_same(f"{k} (step {i})", e[k], g)
        assert launches in (1, 2)
        if must is not None:
            assert launches == (2 if must else 1), f"step {i} ({k}): {launches} rasterize launches"
        requeued += launches == 2
    assert requeued >= 3


def test_north_star_planned_forward_matches_exact(ctx):
    w = CONFIGS[1]
    print(f"[case] {w.name} exact vs planned forward", flush=True)
    scene = generate_splats(w)
    u = uniforms_for(w.camera(), w.img_w, w.img_h, w.n, w.sh_degree)
    ref, _ = _forward(ctx, u, scene, exact=True)
    for rep in range(2):
        g, launches = _forward(ctx, u, scene, exact=False)
        assert launches == 1, "the second render of a scene fits its plan"
        _assert_same(f"config 1 planned #{rep}", ref, g)


def _diff(ctx, gpu, scene, cam, v_out, exact, lanes=False):
    """render_splats_diff + backward, exact or planned; returns the image,
    the dense gradients and the result (its forward state)."""
    import torch
    from brush_amd import render as R

    tr, sh, opac = scene
    ctx.set_debug(exact_sizes=exact, keep_lanes=lanes)
    t = torch.from_numpy(tr).to(gpu).requires_grad_(True)
    s = torch.from_numpy(sh).to(gpu).requires_grad_(True)
    o = torch.from_numpy(opac).to(gpu).requires_grad_(True)
    res = R.render_splats_diff(R.Splats(t, s, o), cam, SIZE)
    res.img.backward(torch.from_numpy(v_out).to(gpu))
    torch.cuda.synchronize()
    ctx.set_debug()
    grads = {"v_transforms": t.grad.cpu().numpy(), "v_coeffs": s.grad.cpu().numpy(),
             "v_raw_opac": o.grad.cpu().numpy(), "v_refine": res._cfg.refine_weight.cpu().numpy()}
    return res.img.detach().cpu().numpy(), grads, res


def _oracle(scene, cam, v_out):
    tr, sh, opac = scene
    uo = uniforms_for(cam, SIZE[0], SIZE[1], tr.shape[0], 0)
    o = O.render_forward(uo, tr, sh, opac, O.FLAG_BWD_INFO)
    return OracleGrads(o, tr, sh, opac, v_out, O.FLAG_REFINE_WEIGHT)


def test_backward_of_a_planned_forward(ctx, gpu):
    print("[case] backward after planned forward", flush=True)
    scene = rng_scene(20_000, 1.5, (-2.5, -0.5), (-1.0, 2.0), 0x55)
    cam = _cam()
    v_out = np.random.default_rng(3).standard_normal((SIZE[1], SIZE[0], 4)).astype(np.float32)
    img0, g0, _ = _diff(ctx, gpu, scene, cam, v_out, True)
    _diff(ctx, gpu, scene, cam, v_out, False)  # plans this scene
    img1, g1, res = _diff(ctx, gpu, scene, cam, v_out, False, lanes=True)
    assert np.array_equal(img0.view(np.uint32), img1.view(np.uint32))
    want = _oracle(scene, cam, v_out)
    noise = {"v_transforms": want.noise_transforms, "v_coeffs": want.noise_coeffs,
             "v_raw_opac": want.noise_raw_opac, "v_refine": want.noise_refine}
    for name in ("v_transforms", "v_coeffs", "v_raw_opac"):
        assert np.all(np.isfinite(g1[name])), name
        check_close(f"{name} planned vs exact", g1[name], g0[name], noise[name], rtol=1e-4)
    check_fused_backward("planned", res._cfg.state, *scene, g1, want)


def test_backward_of_a_forward_that_outgrew_its_plan(ctx, gpu):
    """A planned forward whose scene has four times the intersections its plan
    was made for is queued again with exact sizes (its state's buffers,
    gradient rows included, released and allocated anew); its backward
    matches the backward of an exact-size forward and the restatement."""
    print("[case] backward after a forward that outgrew its plan", flush=True)
    small = rng_scene(2_000, 1.5, (-3.0, -1.5), (-1.0, 2.0), 0x51)
    large = rng_scene(20_000, 1.5, (-2.5, -0.5), (-1.0, 2.0), 0x52)
    cam = _cam()
    v_out = np.random.default_rng(4).standard_normal((SIZE[1], SIZE[0], 4)).astype(np.float32)
    img0, g0, _ = _diff(ctx, gpu, large, cam, v_out, True)
    _diff(ctx, gpu, small, cam, v_out, False)  # the plan: the small scene
    ctx.reset_timings()
    ctx.set_timing(True, only="rasterize")
    img1, g1, res = _diff(ctx, gpu, large, cam, v_out, False, lanes=True)
    launches = ctx.read_timings().get("rasterize", (0, 0.0))[0]
    ctx.set_timing(False)
    assert launches == 2, "the large scene must outgrow the small scene's plan"
    assert np.array_equal(img0.view(np.uint32), img1.view(np.uint32))
    want = _oracle(large, cam, v_out)
    noise = {"v_transforms": want.noise_transforms, "v_coeffs": want.noise_coeffs,
             "v_raw_opac": want.noise_raw_opac}
    for name in ("v_transforms", "v_coeffs", "v_raw_opac"):
        check_close(f"{name} re-queued vs exact", g1[name], g0[name], noise[name], rtol=1e-4)
    check_fused_backward("re-queued", res._cfg.state, *large, g1, want)
