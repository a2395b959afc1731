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
  pairs sized for the plan), to the order of float atomics.
"""
import numpy as np
import pytest

from brush_amd.camera import Camera
from brush_amd.synthetic import CONFIGS, generate_splats
from oracle import oracle as O
from tests.helpers import gpu_forward, grad_close, gradient_term_magnitudes, rng_scene, uniforms_for

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


def test_backward_of_a_planned_forward(ctx, gpu):
    import torch
    from brush_amd import render as R

    print("[case] backward after planned forward", flush=True)
    tr, sh, opac = rng_scene(20_000, 1.5, (-2.5, -0.5), (-1.0, 2.0), 0x55)
    cam = _cam()
    v_out = np.random.default_rng(3).standard_normal((SIZE[1], SIZE[0], 4)).astype(np.float32)

    def run(exact):
        ctx.set_debug(exact_sizes=exact)
        t = torch.from_numpy(tr).to(gpu).requires_grad_(True)
        s = torch.from_numpy(sh).to(gpu).requires_grad_(True)
        o = torch.from_numpy(opac).to(gpu).requires_grad_(True)
        res = R.render_splats_diff(R.Splats(t, s, o), cam, SIZE)
        res.img.backward(torch.from_numpy(v_out).to(gpu))
        torch.cuda.synchronize()
        ctx.set_debug()
        return res.img.detach().cpu().numpy(), (t.grad.cpu().numpy(), s.grad.cpu().numpy(), o.grad.cpu().numpy())

    img0, g0 = run(True)
    run(False)  # plans this scene
    img1, g1 = run(False)
    assert np.array_equal(img0.view(np.uint32), img1.view(np.uint32))
    uo = uniforms_for(cam, SIZE[0], SIZE[1], tr.shape[0], 0)
    o = O.render_forward(uo, tr, sh, opac, O.FLAG_BWD_INFO)
    vc = O.rasterize_backward(o, v_out, O.FLAG_REFINE_WEIGHT)
    mags = gradient_term_magnitudes(o, tr, sh, opac, vc)
    for name, a, b, m in zip(("v_transforms", "v_coeffs", "v_raw_opac"), g0, g1, mags):
        assert np.all(np.isfinite(b)), name
        grad_close(name, b, a, m, rtol=1e-4, atol_frac=1e-6)
