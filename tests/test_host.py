"""Host-side pieces: camera conversions and uniforms (camera.rs), the seeded
workload generator, and the render API's argument checks."""
import math

import numpy as np
import pytest

from brush_amd.camera import (Camera, affine_inverse, focal_to_fov, fov_to_focal, jacobian_clamp_limits,
                              look_at_rotation, project_uniforms, quat_to_mat3, tile_bounds)
from brush_amd.synthetic import CONFIGS, Workload, generate_splats, generate_v_output, splitmix64


def test_fov_focal_round_trip():
    """tests/mod.rs:795-874 (pinhole)."""
    for pixels in (1, 17, 256, 1080, 1920, 4000):
        for fov in (0.1, 0.5, 1.0, 1.5, 2.5):
            f = fov_to_focal(fov, pixels)
            assert abs(focal_to_fov(f, pixels) - fov) < 1e-12
    assert abs(fov_to_focal(math.pi / 2, 123) - 61.5) < 1e-12


def test_uniforms_identity_camera():
    cam = Camera.from_focal((0.0, 0.0, -4.0), (0.0, 0.0, 0.0, 1.0), 1100.0, 1920, 1080)
    u = project_uniforms(cam, 1920, 1080, 10, 3)
    np.testing.assert_array_equal(u["viewmat"], np.array([1, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 4], np.float32))
    assert abs(float(u["fx"]) - 1100.0) < 1e-3 and abs(float(u["fy"]) - 1100.0) < 1e-3
    assert float(u["cx"]) == 960.0 and float(u["cy"]) == 540.0
    assert (u["tile_bw"], u["tile_bh"]) == (120, 68)
    lims = jacobian_clamp_limits(1920, 1080, u["fx"], u["fy"], u["cx"], u["cy"])
    assert np.float32(lims[0]) == (np.float32(1.15) * np.float32(1920) - u["cx"]) / u["fx"]
    with pytest.raises(ValueError):
        project_uniforms(cam, 0, 10, 1, 0)


def test_world_to_local_inverts_pose():
    rng = np.random.default_rng(0)
    for _ in range(20):
        eye = rng.uniform(-5, 5, 3)
        q = look_at_rotation(eye)
        cam = Camera(tuple(eye), q, 0.7, 0.6)
        rot, t = cam.world_to_local()
        r = quat_to_mat3(q)
        # the world origin lands on the camera's +z axis at distance |eye|
        assert np.allclose(rot @ np.zeros(3) + t, [0, 0, np.linalg.norm(eye)], atol=1e-4)
        assert np.allclose(rot @ r, np.eye(3), atol=1e-5)
        assert np.allclose(rot @ eye.astype(np.float32) + t, 0, atol=1e-4)


def test_tile_bounds():
    assert tile_bounds(1920, 1080) == (120, 68)
    assert tile_bounds(1, 1) == (1, 1)
    assert tile_bounds(16, 17) == (1, 2)


def test_splitmix64_matches_scalar_definition():
    """The reference tests' SplitMix64 (tests/mod.rs:197-207), computed
    draw-by-draw in pure Python."""
    seed = 0xB5C00001
    state = seed
    expect = []
    for _ in range(8):
        state = (state + 0x9E3779B97F4A7C15) & (2**64 - 1)
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        expect.append(z ^ (z >> 31))
    got = splitmix64(seed, np.arange(8, dtype=np.uint64))
    assert [int(x) for x in got] == expect


def test_generator_is_deterministic_and_matches_distributions():
    w = Workload("t", 20_000, 3, 64, 64, 60.0, 3.0, seed=123)
    a = generate_splats(w)
    b = generate_splats(w, chunk=777)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)
    tr, sh, opac = a
    assert tr.shape == (20_000, 10) and sh.shape == (20_000, 16, 3) and opac.shape == (20_000,)
    assert np.all((tr[:, 0:3] >= -1) & (tr[:, 0:3] < 1))
    assert abs(tr[:, 7:10].mean() + 4.0) < 0.02 and abs(tr[:, 7:10].std() - 0.5) < 0.02
    np.testing.assert_allclose(np.linalg.norm(tr[:, 3:7], axis=1), 1.0, atol=1e-6)
    assert abs(opac.mean()) < 0.03 and abs(opac.std() - 1.0) < 0.03
    assert abs(sh[:, 0].std() - 0.5) < 0.02 and abs(sh[:, 1:].std() - 0.05) < 0.002
    v = generate_v_output(Workload("t", 1, 0, 64, 48, 60.0, 3.0, seed=5))
    assert v.shape == (48, 64, 4) and abs(v.std() - 1.0) < 0.05


def test_config_table_matches_baseline():
    c1 = CONFIGS[1]
    assert (c1.n, c1.sh_degree, c1.img_w, c1.img_h, c1.focal, c1.distance) == (1_000_000, 3, 1920, 1080, 1100.0, 4.0)
    c0 = CONFIGS[0]
    assert (c0.n, c0.sh_degree, c0.img_w, c0.img_h, c0.focal, c0.distance) == (100_000, 0, 256, 256, 300.0, 3.0)


def test_render_rejects_bad_arguments_without_gpu():
    import torch

    from brush_amd import render as R

    t = torch.zeros((4, 10))
    with pytest.raises((ValueError, TypeError)):
        R.render(Camera(), (0, 16), t, torch.zeros((4, 1, 3)), torch.zeros(4))
    with pytest.raises((ValueError, TypeError)):
        R.render(Camera(), (16, 16), t, torch.zeros((4, 1, 3)), torch.zeros(4))  # CPU tensors
    with pytest.raises(ValueError):
        R.sh_degree_from_coeffs(5)


def test_diff_render_frees_its_state_without_the_cycle_collector(monkeypatch):
    """The differentiable render's autograd node must not close a reference
    cycle through its own output image: a step's forward state (and the
    image) are released when the caller drops the result, not when Python's
    cyclic garbage collector happens to run.  Otherwise every step of a
    training or benchmark loop keeps its count-sized buffers until a
    collection, and the library and torch allocate afresh each step.  The
    render is stubbed with CPU tensors (only the host-side object graph is
    under test)."""
    import gc
    import weakref

    import torch

    from brush_amd import render as R

    class FakeState:
        handle = None

        def release(self):
            pass

    states = []

    def fake_render(camera, img_size, transforms, sh, opac, mode, rmode, bg, rpass, rasterizer=None, **kw):
        st = FakeState()
        states.append(weakref.ref(st))
        w, h = img_size
        aux = R.RenderAux(1, 1, torch.zeros(transforms.shape[0]), torch.zeros(transforms.shape[0]),
                          torch.zeros((1, 1, 2), dtype=torch.int32), (w, h))
        return R.RenderOutput(torch.zeros((h, w, 4)), aux, {}, st)

    monkeypatch.setattr(R, "render", fake_render)
    t = torch.zeros((3, 10), requires_grad=True)
    s = torch.zeros((3, 1, 3), requires_grad=True)
    o = torch.zeros((3,), requires_grad=True)
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        res = R.render_splats_diff(R.Splats(t, s, o), None, (4, 2))
        img_ref = weakref.ref(res.img)
        assert states[0]() is not None
        del res
        assert states[0]() is None, "the forward state outlived its result (reference cycle)"
        assert img_ref() is None, "the rendered image outlived its result (reference cycle)"
    finally:
        if was_enabled:
            gc.enable()


def test_bench_splits_a_kernel_trace_into_kernel_and_idle_time(tmp_path):
    """bench.py --split-trace on a hand-made csv trace: two steps that start at
    project_forward, with a 5 us gap before the second kernel of each step and
    overlapping dispatches counted once."""
    import bench

    rows = [  # (start ns, end ns, name)
        (0, 10_000, "void bh::project_forward_kernel<false, 0, 16, 3>(float const*)"),
        (15_000, 20_000, "bh::tile_order_kernel(unsigned int const*)"),
        (18_000, 30_000, "void bh::rasterize_kernel<true>(float)"),
        (30_000, 40_000, "void bh::project_forward_kernel<false, 0, 16, 3>(float const*)"),
        (45_000, 50_000, "bh::tile_order_kernel(unsigned int const*)"),
        (50_000, 60_000, "void bh::rasterize_kernel<true>(float)"),
    ]
    p = tmp_path / "run_kernel_trace.csv"
    p.write_text("Kernel_Name,Start_Timestamp,End_Timestamp\n"
                 + "".join(f'"{n}",{a},{b}\n' for a, b, n in rows))
    out = bench.split_trace(str(p), 2)
    # step 1 spans 0..30 us with 25 us of kernels, step 2 spans 30..60 us with 25 us
    assert "| step (first dispatch to the next step's first dispatch) | 30.0 |" in out
    assert "| kernels running | 25.0 |" in out
    assert "| GPU idle | 5.0 (16.7 %) |" in out
    assert "| `bh::project_forward_kernel` -> `bh::tile_order_kernel` | 10.0 | 2 | 5.00 |" in out
    assert "| `bh::rasterize_kernel<true>` | 1 | 11.00 | 11.00 |" in out
    with pytest.raises(SystemExit):
        bench.split_trace(str(p), 3)
