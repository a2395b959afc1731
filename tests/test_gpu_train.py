"""GPU parity of the training-step pieces downstream of the rasterizer.

* image loss forward map and VJP (bh_image_loss_forward / _backward) against
  the CPU restatement, bit for bit: both evaluate the same f32 operations in
  the same order (blur sums d = 1..5 then the centre, no contraction);
* AdamScaled (bh_adam_scaled_step) against the restatement, bit for bit, over
  several steps, with and without a per-column scale and a per-row second
  moment;
* the differentiable image_loss through torch autograd;
* SplatTrainer.step: its gradients against the restatement's chain (render,
  loss map, loss VJP, rasterize and project backward) entry by entry to rtol
  1e-3 plus the entry's own rounding noise (tests/helpers.py), and its
  parameter update against the restatement's Adam applied to the same
  gradients, bit for bit; at config 4's full size one step against the
  restatement the same way, and a loss that falls over a few steps.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import OracleGrads, assert_bits_equal, check_close, compare_dense, random_scene, uniforms_for
from brush_amd.synthetic import CONFIGS, generate_splats, generate_target

pytestmark = pytest.mark.gpu


def _pack(b):
    b = b.astype(np.uint32)
    return (b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)).astype(np.uint32)


def _i32(gt_u32):
    import torch

    return torch.from_numpy(gt_u32.view(np.int32))


@pytest.mark.parametrize("h,w,stride,ch,cfg", [
    (1, 1, 3, 3, (0.8, -0.2, None, False)),
    (17, 19, 4, 3, (0.8, -0.2, None, False)),
    (33, 35, 4, 4, (0.8, -0.2, (0.05, 0.1, 0.15), True)),
    (40, 56, 3, 3, (0.0, 1.0, None, False)),
    (70, 100, 4, 3, (0.73, 0.0, (0.07, 0.11, 0.19), True)),
    (1064, 1600, 4, 3, (0.8, -0.2, None, False)),
])
def test_image_loss_matches_checker(gpu, h, w, stride, ch, cfg):
    import torch
    from brush_amd import loss as L

    print(f"[case] image loss {h}x{w} stride={stride} ch={ch} cfg={cfg}", flush=True)
    rng = np.random.default_rng(h * 1000 + w)
    pred = rng.random((h, w, stride), dtype=np.float32)
    gt = _pack(rng.integers(0, 256, (h, w, 4), dtype=np.uint8))
    chain = rng.standard_normal((h, w, ch)).astype(np.float32)
    c = L.ImageLossConfig(*cfg)
    tp = torch.from_numpy(pred).to(gpu)
    view = tp[..., :ch]
    tg = _i32(gt).to(gpu)
    m = L.image_loss_forward_raw(view, tg, c).cpu().numpy()
    g = L.image_loss_backward_raw(view, tg, c, torch.from_numpy(chain).to(gpu)).cpu().numpy()
    oc = O.loss_config(*cfg)
    assert_bits_equal("loss map", m, O.image_loss_forward(pred, ch, gt, oc))
    assert_bits_equal("loss vjp", g, O.image_loss_backward(pred, ch, gt, oc, chain))


def test_image_loss_autograd(gpu):
    """image_loss on an RGB slice of an RGBA tensor, through torch autograd."""
    import torch
    from brush_amd import loss as L

    h, w = 45, 61
    rng = np.random.default_rng(7)
    pred = rng.random((h, w, 4), dtype=np.float32)
    gt = _pack(rng.integers(0, 256, (h, w, 4), dtype=np.uint8))
    chain = rng.standard_normal((h, w, 3)).astype(np.float32)
    tp = torch.from_numpy(pred).to(gpu).requires_grad_(True)
    c = L.ImageLossConfig(0.8, -0.2)
    m = L.image_loss(tp[..., :3], _i32(gt).to(gpu), c)
    (m * torch.from_numpy(chain).to(gpu)).sum().backward()
    want = O.image_loss_backward(pred[..., :3].copy(), 3, gt, O.loss_config(0.8, -0.2), chain)
    got = tp.grad.cpu().numpy()
    assert_bits_equal("autograd rgb", got[..., :3], want)
    assert np.all(got[..., 3] == 0.0)
    ev = L.image_loss_eval(tp[..., :3], _i32(gt).to(gpu), c).cpu().numpy()
    assert_bits_equal("eval", ev, O.image_loss_forward(pred, 3, gt, O.loss_config(0.8, -0.2)))


@pytest.mark.parametrize("shape,reduce,scaled", [((5000, 10), False, True), ((3000, 16, 3), True, True),
                                                  ((100000,), False, False), ((777, 9, 3), True, False),
                                                  ((1, 1), False, False), ((1001, 7), False, True),
                                                  ((40, 700), True, True), ((3, 5), True, False)])
def test_adam_matches_checker(gpu, shape, reduce, scaled):
    import torch
    from brush_amd.train import AdamScaled, AdamState

    print(f"[case] adam shape={shape} reduce={reduce} scaled={scaled}", flush=True)
    rng = np.random.default_rng(sum(shape))
    p = rng.standard_normal(shape).astype(np.float32)
    rows = shape[0]
    row_len = int(np.prod(shape[1:])) if len(shape) > 1 else 1
    scale = (rng.random(row_len).astype(np.float32) + 0.5) if scaled else None
    opt = AdamScaled(epsilon=1e-15)
    st = AdamState(reduce_moment_2=reduce, scaling=torch.from_numpy(scale).to(gpu) if scaled else None)
    tp = torch.from_numpy(p.copy()).to(gpu)
    m1 = np.zeros_like(p)
    m2 = np.zeros((rows,) if reduce else shape, np.float32)
    for t in range(1, 5):
        g = rng.standard_normal(shape).astype(np.float32)
        opt.step(2.5e-3, tp, torch.from_numpy(g).to(gpu), st)
        O.adam_scaled_step(p, g, m1, m2, scale, reduce, 2.5e-3, t)
        assert_bits_equal(f"param t={t}", tp.cpu().numpy(), p)
        assert_bits_equal(f"moment_1 t={t}", st.moment_1.cpu().numpy(), m1)
        assert_bits_equal(f"moment_2 t={t}", st.moment_2.cpu().numpy().reshape(-1), m2.reshape(-1))


def _oracle_step_grads(u, tr, sh, op, gt, ssim_weight) -> tuple:
    """The restatement's training-step chain: (OracleGrads of the render for
    the loss VJP, loss map)."""
    fwd = O.render_forward(u, tr, sh, op, O.FLAG_BWD_INFO)
    img = fwd.out_img
    cfg = O.loss_config(1.0 - ssim_weight, -ssim_weight)
    h, w = gt.shape
    chain = np.full((h, w, 3), np.float32(1.0 / (3 * h * w)), np.float32)
    v_img = O.image_loss_backward(img, 3, gt, cfg, chain)
    return OracleGrads(fwd, tr, sh, op, v_img, O.FLAG_REFINE_WEIGHT), O.image_loss_forward(img, 3, gt, cfg)


def _fold_noise(tr, op, f, n_t, n_o):
    """Carries per-entry noise of the gradients with respect to the folded
    parameters (fold_min_scale's outputs) back to its inputs through the
    absolute Jacobian of the fold, which acts on each splat alone (one
    forward-mode product per input column, in float64)."""
    import torch
    from brush_amd import render as R

    t = torch.from_numpy(tr).double()
    o = torch.from_numpy(op).double()
    ff = torch.from_numpy(f).double()
    n = tr.shape[0]
    out_t, out_o = np.zeros((n, 10)), np.zeros(n)
    for c in range(11):
        dt, do = torch.zeros_like(t), torch.zeros_like(o)
        if c < 10:
            dt[:, c] = 1.0
        else:
            do[:] = 1.0
        _, (jt, jo) = torch.func.jvp(lambda a, b: R.fold_min_scale(a, b, ff), (t, o), (dt, do))
        contrib = (np.abs(jt.numpy()) * n_t).sum(1) + np.abs(jo.numpy()) * n_o
        if c < 10:
            out_t[:, c] = contrib
        else:
            out_o = contrib
    return out_t, out_o


def test_training_step_matches_checker(gpu):
    import torch
    from brush_amd import render as R
    from brush_amd.camera import Camera
    from brush_amd.train import SplatTrainer

    n, deg, W, H = 3000, 3, 80, 64
    tr, sh, op = random_scene(4101, n, deg, log_scale=(-3.0, 0.6))
    cam = Camera.from_focal((0.0, 0.1, -3.0), (0.0, 0.0, 0.0, 1.0), 90.0, W, H)
    rng = np.random.default_rng(11)
    gt = _pack(np.concatenate([rng.integers(0, 256, (H, W, 3), dtype=np.uint8),
                               np.full((H, W, 1), 255, np.uint8)], -1))
    splats = R.Splats(torch.from_numpy(tr.copy()).to(gpu), torch.from_numpy(sh.copy()).to(gpu),
                      torch.from_numpy(op.copy()).to(gpu))
    trainer = SplatTrainer()
    u = uniforms_for(cam, W, H, n, deg)
    p = [tr.copy(), sh.copy(), op.copy()]
    m1 = [np.zeros_like(x) for x in p]
    m2 = [np.zeros_like(p[0]), np.zeros((n,), np.float32), np.zeros_like(p[2])]
    c = trainer.config
    scales = [np.array([c.lr_mean] * 3 + [c.lr_rotation] * 4 + [c.lr_scale] * 3, np.float32),
              np.repeat(np.array([1.0] + [1.0 / c.lr_coeffs_sh_scale] * (sh.shape[1] - 1), np.float32), 3), None]
    lrs = [1.0, c.lr_coeffs_dc, c.lr_opac]
    for step in range(1, 3):
        print(f"[case] training step {step}", flush=True)
        res = trainer.step(splats, cam, _i32(gt).to(gpu), record_grads=True)
        want, lmap = _oracle_step_grads(u, p[0], p[1], p[2], gt, c.ssim_weight)
        assert abs(float(res["loss"].item()) - float(lmap.astype(np.float64).mean())) < 1e-5
        grads = [res["v_transforms"].cpu().numpy(), res["v_coeffs"].cpu().numpy(), res["v_raw_opac"].cpu().numpy()]
        compare_dense(f"train step {step} ", dict(zip(("v_transforms", "v_coeffs", "v_raw_opac"), grads)), want)
        # the optimizer fed the GPU's gradients: bit for bit
        for k in range(3):
            O.adam_scaled_step(p[k], grads[k], m1[k], m2[k], scales[k], k == 1, lrs[k], step)
        assert_bits_equal("transforms", splats.transforms.cpu().numpy(), p[0])
        assert_bits_equal("sh_coeffs", splats.sh_coeffs.cpu().numpy(), p[1])
        assert_bits_equal("raw_opacities", splats.raw_opacities.cpu().numpy(), p[2])


def test_config4_full_size_step_matches_checker(gpu):
    """BASELINE config 4 at full size (1M SH3 splats, 1600x1064, the 8x8-block
    target), one SplatTrainer step against the restatement's chain: the loss
    to 1e-5, the gradients entry by entry to rtol 1e-3 plus their rounding
    noise, and the parameter update bit for bit from the GPU's gradients."""
    import os

    import torch
    from brush_amd import render as R
    from brush_amd.train import SplatTrainer

    O.set_threads(max(1, min(16, os.cpu_count() or 1)))
    try:
        w = CONFIGS[4]
        print(f"[case] {w.name} one step against the restatement", flush=True)
        tr, sh, op = generate_splats(w)
        gt = generate_target(w)
        splats = R.Splats(torch.from_numpy(tr.copy()).to(gpu), torch.from_numpy(sh.copy()).to(gpu),
                          torch.from_numpy(op.copy()).to(gpu))
        trainer = SplatTrainer()
        cam = w.camera()
        res = trainer.step(splats, cam, _i32(gt).to(gpu), record_grads=True)
        u = uniforms_for(cam, w.img_w, w.img_h, w.n, w.sh_degree)
        want, lmap = _oracle_step_grads(u, tr, sh, op, gt, trainer.config.ssim_weight)
        assert abs(float(res["loss"].item()) - float(lmap.astype(np.float64).mean())) < 1e-5
        grads = [res["v_transforms"].cpu().numpy(), res["v_coeffs"].cpu().numpy(), res["v_raw_opac"].cpu().numpy()]
        compare_dense(f"{w.name} ", dict(zip(("v_transforms", "v_coeffs", "v_raw_opac"), grads)), want)
        c = trainer.config
        scales = [np.array([c.lr_mean] * 3 + [c.lr_rotation] * 4 + [c.lr_scale] * 3, np.float32),
                  np.repeat(np.array([1.0] + [1.0 / c.lr_coeffs_sh_scale] * (sh.shape[1] - 1), np.float32), 3),
                  None]
        lrs = [1.0, c.lr_coeffs_dc, c.lr_opac]
        p = [tr.copy(), sh.copy(), op.copy()]
        for k in range(3):
            m1 = np.zeros_like(p[k])
            m2 = np.zeros((p[k].shape[0],), np.float32) if k == 1 else np.zeros_like(p[k])
            O.adam_scaled_step(p[k], grads[k], m1, m2, scales[k], k == 1, lrs[k], 1)
        assert_bits_equal("transforms", splats.transforms.cpu().numpy(), p[0])
        assert_bits_equal("sh_coeffs", splats.sh_coeffs.cpu().numpy(), p[1])
        assert_bits_equal("raw_opacities", splats.raw_opacities.cpu().numpy(), p[2])
    finally:
        O.set_threads(1)


def test_config4_training_steps_reduce_the_loss(gpu):
    """BASELINE config 4 at full size: 1M SH3 splats, 1600x1064, the 8x8-block target."""
    import torch
    from brush_amd import render as R
    from brush_amd.train import SplatTrainer

    w = CONFIGS[4]
    print(f"[case] {w.name}", flush=True)
    tr, sh, op = generate_splats(w)
    gt = generate_target(w)
    splats = R.Splats(torch.from_numpy(tr).to(gpu), torch.from_numpy(sh).to(gpu), torch.from_numpy(op).to(gpu))
    trainer = SplatTrainer()
    cam = w.camera()
    tg = _i32(gt).to(gpu)
    losses = []
    for _ in range(5):
        res = trainer.step(splats, cam, tg, record_grads=True)
        losses.append(float(res["loss"].item()))
        for k in ("v_transforms", "v_coeffs", "v_raw_opac"):
            assert bool(torch.isfinite(res[k]).all()), k
    print(f"[case] {w.name} losses {losses}", flush=True)
    assert losses[-1] < losses[0]
    for t in (splats.transforms, splats.sh_coeffs, splats.raw_opacities):
        assert bool(torch.isfinite(t).all())


def test_min_scale_floor_in_render_and_training(gpu):
    """Splats.min_scale (gaussian_splats.rs:139-164): both render paths render
    the folded splat, and the trainer's gradients are the restatement's chain
    at the folded parameters pulled back through the fold (rtol 1e-3)."""
    import torch
    from brush_amd import render as R
    from brush_amd.camera import Camera
    from brush_amd.train import SplatTrainer

    n, deg, W, H = 2000, 1, 72, 56
    tr, sh, op = random_scene(4202, n, deg, log_scale=(-4.0, -1.0))
    cam = Camera.from_focal((0.0, 0.1, -3.0), (0.0, 0.0, 0.0, 1.0), 90.0, W, H)
    f = np.random.default_rng(5).uniform(0.002, 0.03, n).astype(np.float32)
    t_d, s_d, o_d, f_d = (torch.from_numpy(a.copy()).to(gpu) for a in (tr, sh, op, f))
    floored = R.Splats(t_d.clone(), s_d.clone(), o_d.clone(), min_scale=f_d)
    ft, fo = R.fold_min_scale(t_d, o_d, f_d)
    plain = R.Splats(ft.contiguous(), s_d.clone(), fo.contiguous())
    img_a, _ = R.render_splats(floored, cam, (W, H))
    img_b, _ = R.render_splats(plain, cam, (W, H))
    assert torch.equal(img_a, img_b)
    # differentiable path: gradients reach the unfolded leaves through the fold
    leaves = [t_d.clone().requires_grad_(), s_d.clone().requires_grad_(), o_d.clone().requires_grad_()]
    out = R.render_splats_diff(R.Splats(*leaves, min_scale=f_d), cam, (W, H))
    v_img = torch.randn(out.img.shape, device=gpu, generator=torch.Generator(device=gpu).manual_seed(3))
    out.img.backward(v_img)
    ref = [t_d.clone().requires_grad_(), o_d.clone().requires_grad_()]
    rt, ro = R.fold_min_scale(ref[0], ref[1], f_d)
    out2 = R.render_splats_diff(R.Splats(rt, s_d.clone().requires_grad_(), ro), cam, (W, H))
    out2.img.backward(v_img)
    # the two renders differ only in the order of their float atomics: the
    # restatement's noise of the folded splats' gradients, carried through
    # the fold
    uf = uniforms_for(cam, W, H, n, deg)
    ftn, fon = ft.cpu().numpy(), fo.cpu().numpy()
    fwd_f = O.render_forward(uf, ftn, sh, fon, O.FLAG_BWD_INFO)
    diff_want = OracleGrads(fwd_f, ftn, sh, fon, v_img.cpu().numpy(), O.FLAG_REFINE_WEIGHT)
    nt, no = _fold_noise(tr, op, f, diff_want.noise_transforms, diff_want.noise_raw_opac)
    check_close("v_transforms (diff)", leaves[0].grad.cpu().numpy(), ref[0].grad.cpu().numpy(), nt)
    check_close("v_raw_opac (diff)", leaves[2].grad.cpu().numpy(), ref[1].grad.cpu().numpy(), no)
    # the training step
    rng = np.random.default_rng(13)
    gt = _pack(np.concatenate([rng.integers(0, 256, (H, W, 3), dtype=np.uint8),
                               np.full((H, W, 1), 255, np.uint8)], -1))
    trainer = SplatTrainer()
    res = trainer.step(R.Splats(t_d.clone(), s_d.clone(), o_d.clone(), min_scale=f_d), cam, _i32(gt).to(gpu),
                       record_grads=True)
    u = uniforms_for(cam, W, H, n, deg)
    want, _ = _oracle_step_grads(u, ftn, sh, fon, gt, trainer.config.ssim_weight)
    pt, po = t_d.clone().requires_grad_(), o_d.clone().requires_grad_()
    qt, qo = R.fold_min_scale(pt, po, f_d)
    want_t, want_o = torch.autograd.grad([qt, qo], [pt, po], [torch.from_numpy(want.v_transforms).to(gpu),
                                                               torch.from_numpy(want.v_raw_opac).to(gpu)])
    nt, no = _fold_noise(tr, op, f, want.noise_transforms, want.noise_raw_opac)
    check_close("v_transforms (train)", res["v_transforms"].cpu().numpy(), want_t.cpu().numpy(), nt)
    check_close("v_raw_opac (train)", res["v_raw_opac"].cpu().numpy(), want_o.cpu().numpy(), no)
    check_close("v_coeffs (train)", res["v_coeffs"].cpu().numpy(), want.v_coeffs, want.noise_coeffs)
