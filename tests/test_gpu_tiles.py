"""GPU parity of the 16x8 candidate rasterizer (Rasterizer::Candidate,
gaussian_splats.rs:68-101) against the CPU restatement: every forward output
bit for bit, rasterize backward entry by entry to rtol 1e-3 plus the entry's
own rounding noise (tests/helpers.py), project backward bit for bit;
the same image as the 16x16 rasterizer; the differentiable path end to end.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import (OracleGrads, assert_bits_equal, check_fused_backward, compare_forward, compare_lanes,
                           gpu_forward, keep_lanes, random_scene, uniforms_for)
from brush_amd.camera import Camera

pytestmark = pytest.mark.gpu

TILE = O.FLAG_TILE_16X8


@pytest.mark.parametrize("seed,n,deg,flags,size", [(1, 3000, 3, 1, (97, 75)), (2, 5000, 0, 3, (64, 64)),
                                                   (3, 2000, 2, 5, (41, 23)), (4, 4000, 1, 9, (130, 17)),
                                                   (5, 2500, 3, 0, (97, 75))])
def test_candidate_tiles_match_checker(gpu, seed, n, deg, flags, size):
    import torch
    from brush_amd import render as R

    w, h = size
    print(f"[case] 16x8 seed={seed} n={n} deg={deg} flags={flags} size={size}", flush=True)
    tr, sh, opac = random_scene(800 + seed, n, deg, log_scale=(-3.0, 0.6))
    cam = Camera.from_focal((0.1, -0.2, -3.0), (0.0, 0.0, 0.0, 1.0), 70.0, w, h)
    u = uniforms_for(cam, w, h, n, deg)
    bg = (0.1, 0.2, 0.3)
    g = gpu_forward(u, tr, sh, opac, flags | TILE, bg)
    o = O.render_forward(u, tr, sh, opac, flags | TILE, bg)
    assert tuple(g["tile_offsets"].shape) == (-(-h // 8), -(-w // 16), 2)
    compare_forward(g, o)
    legacy = gpu_forward(u, tr, sh, opac, flags, bg)
    assert_bits_equal("16x8 vs 16x16 image", g["out_img"], legacy["out_img"])
    if not flags & 1:
        return
    chans = 5 if flags & 4 else 4
    v_out = np.random.default_rng(seed).standard_normal((h, w, chans)).astype(np.float32)
    bflags = (flags & 6) | 16
    out = g["out"]
    vc_gpu = R.rasterize_bwd(out.out_img, out.projected_splats, out.compact_gid_from_isect, out.aux.tile_offsets, bg,
                             out.aux.img_size, torch.from_numpy(v_out).to(gpu), bool(bflags & 2), bool(bflags & 4),
                             True, R.Rasterizer.Candidate).cpu().numpy()
    compare_lanes("v_combined", vc_gpu, OracleGrads(o, tr, sh, opac, v_out, bflags, bg, dense=False))


def test_candidate_tiles_autograd(gpu):
    """render_splats_diff with 16x8 tiles: gradients through bh_render_backward
    against the checker's chain."""
    import torch
    from brush_amd import render as R

    n, deg, w, h = 2000, 3, 70, 52
    tr, sh, opac = random_scene(901, n, deg, log_scale=(-3.0, 0.6))
    cam = Camera.from_focal((0.0, 0.1, -3.0), (0.0, 0.0, 0.0, 1.0), 65.0, w, h)
    splats = R.Splats(torch.from_numpy(tr).to(gpu).requires_grad_(True), torch.from_numpy(sh).to(gpu).requires_grad_(True),
                      torch.from_numpy(opac).to(gpu).requires_grad_(True))
    weights = np.random.default_rng(3).standard_normal((h, w, 4)).astype(np.float32)
    with keep_lanes():
        res = R.render_splats_diff(splats, cam, (w, h), (0.1, 0.2, 0.3), compute_refine_weight=True,
                                   rasterizer=R.Rasterizer.Candidate)
        (res.img * torch.from_numpy(weights).to(gpu)).sum().backward()
    u = uniforms_for(cam, w, h, n, deg)
    o = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO | TILE, (0.1, 0.2, 0.3))
    want = OracleGrads(o, tr, sh, opac, weights, O.FLAG_REFINE_WEIGHT, (0.1, 0.2, 0.3))
    grads = {"v_transforms": splats.transforms.grad.cpu().numpy(), "v_coeffs": splats.sh_coeffs.grad.cpu().numpy(),
             "v_raw_opac": splats.raw_opacities.grad.cpu().numpy(), "v_refine": res.refine_weight_fn().cpu().numpy()}
    check_fused_backward("16x8 autograd", res._cfg.state, tr, sh, opac, grads, want)
