"""GPU parity of the camera models (KB4, RT8, thin-prism fisheye) against the
CPU restatement, whose models are pinned by tests/test_oracle_camera.py.

The forward (visibility, tile counts, intersections, sorted ids, offsets,
projected rows, image) is compared bit for bit: both sides evaluate the same
f32 operations, including the reproducible atan2.  The rasterize backward is
compared entry by entry to rtol 1e-3 plus the entry's own rounding noise
(float atomics; tests/helpers.py); project backward fed the checker's
v_combined is compared bit for bit.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import (OracleGrads, assert_bits_equal, compare_forward, compare_lanes, gpu_forward, random_scene,
                           uniforms_for)
from brush_amd import camera as C
from brush_amd.camera import Camera

pytestmark = pytest.mark.gpu

MODELS = {
    "kb4": C.KannalaBrandt4(k1=-0.05, k2=0.01, k3=-0.001, k4=5e-5),
    "kb4_heavy": C.KannalaBrandt4(k1=0.25, k2=-0.12, k3=0.04, k4=-0.015),
    "rt8": C.RadialTangential8(k1=-0.2, k2=0.05, k3=-0.001, k4=0.01, k5=-0.002, p1=1e-3, p2=-1e-3),
    "rt8_heavy": C.RadialTangential8(k1=-0.35, k2=0.15, k3=-0.04, k4=0.008, k5=-0.004, p1=0.04, p2=-0.03),
    "tpf": C.ThinPrismFisheye(kb4=C.KannalaBrandt4(k1=-0.05, k2=0.01, k3=-0.001, k4=5e-5), p1=1e-3, p2=-1e-3,
                              sx1=5e-4, sy1=-5e-4),
    "tpf_heavy": C.ThinPrismFisheye(kb4=C.KannalaBrandt4(k1=-0.18, k2=0.08, k3=-0.015, k4=0.004), p1=0.025,
                                    p2=-0.02, sx1=0.015, sy1=-0.018),
}


@pytest.mark.parametrize("name,flags,deg", [("kb4", 1, 3), ("kb4_heavy", 3, 1), ("rt8", 1, 3), ("rt8_heavy", 9, 2),
                                            ("tpf", 5, 3), ("tpf_heavy", 1, 0)])
def test_camera_model_forward_and_backward(gpu, name, flags, deg):
    import torch
    from brush_amd import render as R

    print(f"[case] camera model {name} flags={flags} deg={deg}", flush=True)
    n, w, h = 4000, 83, 61
    tr, sh, opac = random_scene(5000 + deg + flags, n, deg, log_scale=(-3.0, 0.6))
    cam = Camera.from_focal((0.1, -0.2, -3.0), (0.0, 0.0, 0.0, 1.0), 60.0, w, h, camera_model=MODELS[name])
    u = uniforms_for(cam, w, h, n, deg)
    bg = (0.1, 0.2, 0.3)
    g = gpu_forward(u, tr, sh, opac, flags, bg)
    o = O.render_forward(u, tr, sh, opac, flags, bg)
    assert o.num_visible > n // 4 and o.num_intersections > 0
    compare_forward(g, o)
    chans = 5 if flags & 4 else 4
    v_out = np.random.default_rng(flags).standard_normal((h, w, chans)).astype(np.float32)
    bflags = (flags & 6) | 16
    out = g["out"]
    vc_gpu = R.rasterize_bwd(out.out_img, out.projected_splats, out.compact_gid_from_isect, out.aux.tile_offsets, bg,
                             out.aux.img_size, torch.from_numpy(v_out).to(gpu), bool(bflags & 2), bool(bflags & 4),
                             True).cpu().numpy()
    want = OracleGrads(o, tr, sh, opac, v_out, bflags, bg, mip=bool(flags & 8), dense=False)
    compare_lanes("v_combined", vc_gpu, want)
    vc_ref = want.v_combined
    mode = R.SplatRenderMode.Mip if flags & 8 else R.SplatRenderMode.Default
    grads = R.project_bwd(torch.from_numpy(tr).to(gpu), torch.from_numpy(sh).to(gpu), torch.from_numpy(opac).to(gpu),
                          out.global_from_compact_gid, out.project_uniforms, mode, torch.from_numpy(vc_ref).to(gpu))
    vt, vcoef, vo, vr = O.project_backward(o, tr, sh, opac, vc_ref, mip=bool(flags & 8))
    assert_bits_equal("v_transforms", grads.v_transforms.cpu().numpy(), vt)
    assert_bits_equal("v_coeffs", grads.v_coeffs.cpu().numpy(), vcoef)
    assert_bits_equal("v_raw_opac", grads.v_raw_opac.cpu().numpy(), vo)
    assert_bits_equal("v_refine", grads.v_refine_weight.cpu().numpy(), vr)


def test_wide_fisheye_renders_behind_the_image_plane(gpu):
    """A 200-degree KB4 lens sees splats with z < 0 (project_forward.rs:49-62);
    the forward matches the checker bit for bit and some visible splat lies
    behind the camera plane."""
    n, w, h = 3000, 64, 64
    rng = np.random.default_rng(77)
    tr, sh, opac = random_scene(7001, n, 1, log_scale=(-2.5, 0.4))
    # a shell of splats around the camera at the origin
    d = rng.standard_normal((n, 3))
    tr[:, 0:3] = (d / np.linalg.norm(d, axis=1, keepdims=True) * rng.uniform(2.0, 3.0, (n, 1))).astype(np.float32)
    fov = math.radians(200.0)
    cam = Camera((0.0, 0.0, 0.0), (0.0, 0.0, 0.0, 1.0), fov, fov, (0.5, 0.5), MODELS["kb4"])
    u = uniforms_for(cam, w, h, n, 1)
    g = gpu_forward(u, tr, sh, opac, 1, (0.0, 0.0, 0.0))
    o = O.render_forward(u, tr, sh, opac, 1, (0.0, 0.0, 0.0))
    compare_forward(g, o)
    behind = tr[o.global_from_compact_gid[: o.num_visible], 2] < 0.0
    assert behind.any()
