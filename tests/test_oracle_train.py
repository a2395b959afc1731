"""Pins the CPU restatement of the image loss and of AdamScaled.

* image loss: the reference's own tests (crates/brush-loss/tests/reference.rs):
  SSIM(x, x) = 1 (:219-240), SSIM within [-1, 1] (:242-264), the L1-only map
  against its closed form on the reference's fixed bytes (:140-173, :371-416),
  and the VJP against central finite differences on the reference's inputs,
  probes and tolerance (:60-97, :175-206, :300-369); plus an independent
  float64 SSIM built from scipy's separable correlation.
* AdamScaled: a float64 restatement of adam_scaled.rs:216-383 written from the
  update equations, over several steps, with and without a per-column scale
  and a reduced second moment; and the first-step identity
  param_1 = param_0 - lr * scale * g / (|g| + eps') that the bias correction
  fixes.
"""
import numpy as np
import pytest
from scipy import ndimage

from oracle import oracle as O


def pack_rgba(b: np.ndarray) -> np.ndarray:
    b = b.astype(np.uint32).reshape(-1, 4)
    return (b[:, 0] | (b[:, 1] << 8) | (b[:, 2] << 16) | (b[:, 3] << 24)).astype(np.uint32)


def make_pattern(h, w, scale, offset):
    """reference.rs:27-31"""
    i = np.arange(h * w * 4, dtype=np.uint64)
    return ((i * scale + offset) % 251).astype(np.uint8)


def pred_from_bytes(b, h, w):
    return (b.reshape(h, w, 4)[..., :3].astype(np.float32) / np.float32(255.0)).astype(np.float32)


def test_gauss_taps_closed_form():
    t = O.gauss_taps().astype(np.float64)
    x = np.arange(-5, 6, dtype=np.float64)
    g = np.exp(-x * x / 4.5)
    g /= g.sum()
    np.testing.assert_allclose(t, g[:6], rtol=1e-6)
    assert abs(2 * t[:5].sum() + t[5] - 1.0) < 1e-6


def test_ssim_identical_inputs_is_one():
    h, w = 40, 56
    b = make_pattern(h, w, 11, 13)
    m = O.image_loss_forward(pred_from_bytes(b, h, w), 3, pack_rgba(b).reshape(h, w), O.loss_config(0.0, 1.0))
    assert abs(float(m.mean()) - 1.0) < 1e-4


def test_ssim_in_clamp_range():
    h, w = 40, 56
    a, b = make_pattern(h, w, 7, 19), make_pattern(h, w, 13, 7)
    m = O.image_loss_forward(pred_from_bytes(a, h, w), 3, pack_rgba(b).reshape(h, w), O.loss_config(0.0, 1.0))
    assert m.min() >= -1.0 and m.max() <= 1.0


def _ssim_f64(x, y):
    """SSIM map of two float64 planes, 11-tap Gaussian (sigma 1.5) with zero padding."""
    k = np.exp(-np.arange(-5, 6) ** 2 / 4.5)
    k /= k.sum()

    def blur(z):
        z = ndimage.correlate1d(z, k, axis=1, mode="constant", cval=0.0)
        return ndimage.correlate1d(z, k, axis=0, mode="constant", cval=0.0)

    mu1, mu2 = blur(x), blur(y)
    s1 = np.maximum(0.0, blur(x * x) - mu1 ** 2)
    s2 = np.maximum(0.0, blur(y * y) - mu2 ** 2)
    s12 = blur(x * y) - mu1 * mu2
    c1, c2 = 0.01 ** 2, 0.03 ** 2
    return np.clip((2 * mu1 * mu2 + c1) * (2 * s12 + c2) / ((mu1 ** 2 + mu2 ** 2 + c1) * (s1 + s2 + c2)), -1, 1)


@pytest.mark.parametrize("shape", [(5, 7), (23, 41), (64, 48)])
def test_ssim_against_float64_scipy(shape):
    h, w = shape
    rng = np.random.default_rng(h * w)
    pred = rng.random((h, w, 4), dtype=np.float32)
    gt_bytes = rng.integers(0, 256, (h, w, 4), dtype=np.uint8)
    m = O.image_loss_forward(pred, 3, pack_rgba(gt_bytes).reshape(h, w), O.loss_config(0.0, 1.0))
    for c in range(3):
        ref = _ssim_f64(pred[..., c].astype(np.float64), gt_bytes[..., c].astype(np.float64) / 255.0)
        np.testing.assert_allclose(m[..., c], ref, atol=2e-5)


def test_l1_forward_known_answers():
    """reference.rs:371-416 with the closed form of reference.rs:140-173."""
    gt_b = np.array([10, 100, 200, 0, 250, 50, 25, 64, 30, 90, 150, 192, 240, 180, 60, 255], np.uint8)
    rgb = np.array([0.9, 0.1, 0.4, 0.2, 0.8, 0.5, 0.7, 0.3, 0.05, 0.4, 0.6, 0.95], np.float32)
    rgba = np.array([0.9, 0.1, 0.4, 0.8, 0.2, 0.8, 0.5, 0.1, 0.7, 0.3, 0.05, 0.9, 0.4, 0.6, 0.95, 0.2], np.float32)
    gt = pack_rgba(gt_b).reshape(2, 2)
    cases = [(rgb, 3, 0.73, None, False), (rgb, 3, 0.41, (0.1, 0.25, 0.8), True), (rgba, 4, 0.19, None, False)]
    for data, ch, l1w, bg, mask in cases:
        pred = data.reshape(2, 2, ch)
        m = O.image_loss_forward(pred, ch, gt, O.loss_config(l1w, 0.0, bg, mask))
        for pix in range(4):
            a = gt_b[pix * 4 + 3] / 255.0
            for c in range(ch):
                if c == 3:
                    g = a
                else:
                    g = gt_b[pix * 4 + c] / 255.0
                    if bg is not None:
                        g = g + (1.0 - a) * bg[c]
                wgt = 1.0 if c == 3 else l1w
                expect = wgt * abs(data[pix * ch + c] - g) * (a if mask else 1.0)
                assert abs(m.reshape(-1)[pix * ch + c] - expect) < 2e-6, (pix, c)


def _vjp_inputs(h, w, ch):
    """reference.rs:60-97"""
    pred, gt, chain = [], [], []
    for p in range(h * w):
        off = (p % 17) * 0.002
        pred += [0.75 + off, 0.65 + off, 0.10 + off] + ([0.05 + off] if ch == 4 else [])
        gt += [30 + (p * 7) % 31, 80 + (p * 11) % 31, 130 + (p * 13) % 31, 100 + (p * 17) % 131]
    for i in range(h * w * ch):
        mag = 0.25 + ((i * 19 + 7) % 31) / 31.0
        chain.append(mag if i % 2 == 0 else -mag)
    return (np.array(pred, np.float32).reshape(h, w, ch), pack_rgba(np.array(gt, np.uint8)).reshape(h, w),
            np.array(chain, np.float32).reshape(h, w, ch))


def _loss_f64(pred, ch, gt, cfg):
    """The loss map in float64 from its definition (lib.rs:228-555), SSIM via scipy."""
    l1w, ssimw, bg, mask = cfg
    gb = np.stack([(gt >> (8 * k)) & 255 for k in range(4)], -1).astype(np.float64) / 255.0
    a = gb[..., 3]
    out = np.zeros(pred.shape[:2] + (ch,))
    for k in range(ch):
        p = pred[..., k].astype(np.float64)
        if k == 3:
            v = np.abs(p - a)
        else:
            g = gb[..., k] + ((1.0 - a) * bg[k] if bg is not None else 0.0)
            v = l1w * np.abs(p - g) + (ssimw * _ssim_f64(p, g) if ssimw != 0.0 else 0.0)
        out[..., k] = v * a if mask else v
    return out


@pytest.mark.parametrize("shape,cfg,probes", [
    ((1, 1, 3), (0.8, -0.2, None, False), [(0, 0, 0), (0, 0, 2)]),
    ((3, 7, 4), (0.8, -0.2, (0.05, 0.10, 0.15), True), [(0, 0, 0), (1, 3, 3), (2, 6, 2)]),
    ((17, 19, 3), (0.0, 1.0, (0.05, 0.10, 0.15), False), [(0, 0, 0), (15, 16, 1), (16, 18, 2), (8, 8, 1)]),
    ((33, 35, 3), (0.8, -0.2, None, True), [(16, 16, 0), (32, 34, 2)]),
    ((7, 9, 4), (0.73, 0.0, (0.07, 0.11, 0.19), True), [(0, 0, 0), (3, 4, 1), (6, 8, 2), (2, 5, 3)]),
])
def test_loss_vjp_matches_finite_differences(shape, cfg, probes):
    """The cases, probes and tolerance (1e-3 + 1 %) of reference.rs:175-206 and
    :300-369.  The central differences are taken on the float64 loss (epsilon
    1e-3): the f32 map of these near-constant images carries ~5e-5 of rounding
    (E[x^2] - mu^2 cancels), too much for a difference quotient."""
    h, w, ch = shape
    c = O.loss_config(*cfg)
    base, gt, chain = _vjp_inputs(h, w, ch)
    grad = O.image_loss_backward(base, ch, gt, c, chain)
    assert np.all(np.isfinite(grad))

    def dot(p):
        return float((_loss_f64(p, ch, gt, cfg) * chain).sum())

    eps = 1e-3
    for y, x, k in probes:
        plus, minus = base.astype(np.float64), base.astype(np.float64)
        plus[y, x, k] += eps
        minus[y, x, k] -= eps
        num = (dot(plus) - dot(minus)) / (2.0 * eps)
        ana = float(grad[y, x, k])
        scale = max(abs(num), abs(ana), 1e-6)
        assert abs(num - ana) <= 1e-3 + 0.01 * scale, (y, x, k, num, ana)


def test_loss_forward_matches_float64():
    """The f32 map against the float64 definition on the VJP inputs, every config."""
    for (h, w, ch), cfg in [((17, 19, 3), (0.8, -0.2, (0.05, 0.1, 0.15), False)), ((9, 13, 4), (0.8, -0.2, None, True)),
                            ((7, 9, 4), (0.73, 0.0, (0.07, 0.11, 0.19), True))]:
        base, gt, _ = _vjp_inputs(h, w, ch)
        m = O.image_loss_forward(base, ch, gt, O.loss_config(*cfg))
        np.testing.assert_allclose(m, _loss_f64(base, ch, gt, cfg), atol=1e-4)


def test_loss_backward_writes_zero_past_channels():
    h, w = 9, 11
    rng = np.random.default_rng(3)
    pred = rng.random((h, w, 4), dtype=np.float32)
    gt = pack_rgba(rng.integers(0, 256, (h, w, 4), dtype=np.uint8)).reshape(h, w)
    g = O.image_loss_backward(pred, 3, gt, O.loss_config(0.8, -0.2), np.ones((h, w, 3), np.float32))
    assert np.all(g[..., 3] == 0.0) and np.any(g[..., :3] != 0.0)


def _adam_f64(p, g, m1, m2, scale, reduce, lr, t, b1=0.9, b2=0.999, eps=1e-15):
    # the reference's constants are f32: beta, 1 - beta and the bias
    # corrections are formed in f32 (adam_scaled.rs:57-69, 330-383)
    b1, b2 = float(np.float32(b1)), float(np.float32(b2))
    f1, f2 = float(np.float32(1.0) - np.float32(b1)), float(np.float32(1.0) - np.float32(b2))
    bc1 = float(np.float32(1.0) - np.float32(b1) ** np.float32(t))
    bc2 = float(np.float32(1.0) - np.float32(b2) ** np.float32(t))
    g = g.astype(np.float64)
    g2 = (g * g).reshape(g.shape[0], -1).mean(1).reshape((-1,) + (1,) * (g.ndim - 1)) if reduce else g * g
    if t == 1:
        m1 = f1 * g
        m2 = f2 * g2
    else:
        m1 = b1 * m1 + f1 * g
        m2 = b2 * m2 + f2 * g2
    step = (m1 / bc1) / (np.sqrt(m2 / bc2) + eps)
    sc = lr if scale is None else (scale.astype(np.float32) * np.float32(lr)).astype(np.float64).reshape(p.shape[1:])
    return p - step * sc, m1, m2


@pytest.mark.parametrize("shape,reduce,scaled", [((50, 10), False, True), ((40, 16, 3), True, True),
                                                  ((64,), False, False), ((30, 4, 3), True, False)])
def test_adam_matches_float64_update(shape, reduce, scaled):
    rng = np.random.default_rng(sum(shape))
    p = rng.standard_normal(shape).astype(np.float32)
    rows = shape[0]
    row_len = int(np.prod(shape[1:])) if len(shape) > 1 else 1
    scale = (rng.random(row_len).astype(np.float32) + 0.5) if scaled else None
    m1 = np.zeros_like(p)
    m2 = np.zeros((rows,) if reduce else shape, np.float32)
    m1_64, m2_64 = None, None
    lr = 2.5e-3
    for t in range(1, 5):
        g = rng.standard_normal(shape).astype(np.float32)
        before = p.copy()
        O.adam_scaled_step(p, g, m1, m2, scale, reduce, lr, t)
        p64, m1_64, m2_64 = _adam_f64(before.astype(np.float64), g, m1_64, m2_64, scale, reduce, lr, t)
        # each step's decrement from the same f32 parameter; slack of one
        # parameter ulp for the f32 store, and 1e-6 of each moment's scale for
        # moment sums that nearly cancel
        delta, delta64 = before.astype(np.float64) - p, before.astype(np.float64) - p64
        np.testing.assert_allclose(delta, delta64, rtol=1e-4, atol=1.2e-7 * np.abs(before).max())
        np.testing.assert_allclose(m1, m1_64, rtol=1e-5, atol=1e-6 * np.abs(m1_64).max())
        np.testing.assert_allclose(m2.reshape(-1), np.asarray(m2_64).reshape(-1), rtol=1e-5,
                                   atol=1e-6 * np.abs(m2_64).max())


def test_adam_first_step_is_sign_step():
    """With t = 1 the bias-corrected moments are g and g^2, so the step is lr * scale * g / |g|."""
    rng = np.random.default_rng(9)
    p = rng.standard_normal((100, 10)).astype(np.float32)
    g = rng.standard_normal((100, 10)).astype(np.float32)
    scale = np.linspace(0.5, 2.0, 10).astype(np.float32)
    p0 = p.copy()
    O.adam_scaled_step(p, g, np.zeros_like(p), np.zeros_like(p), scale, False, 1e-3, 1)
    np.testing.assert_allclose(p0.astype(np.float64) - p, 1e-3 * scale[None, :] * np.sign(g), rtol=1e-4,
                               atol=1.2e-7 * np.abs(p0).max())
