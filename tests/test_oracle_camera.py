"""Pins the CPU restatement's camera models (KB4, RT8, thin-prism fisheye)
before the GPU is checked against it.

Each check is independent of the restatement's own formulas: float64 libm for
atan2, the reference's fov/focal round trips (brush-render/src/tests/mod.rs:
795-874), float64 closed forms of each projection written from the model
definitions, float64 finite differences for the Jacobians and the projection
VJPs, identities between models, and finite differences of the whole render.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import uniforms_for
from brush_amd import camera as C
from brush_amd.camera import Camera

KB4 = C.KannalaBrandt4(k1=-0.05, k2=0.01, k3=-0.001, k4=5e-5)
RT8 = C.RadialTangential8(k1=-0.2, k2=0.05, k3=-0.001, k4=0.01, k5=-0.002, k6=0.0, p1=1e-3, p2=-1e-3)
TPF = C.ThinPrismFisheye(kb4=KB4, p1=1e-3, p2=-1e-3, sx1=5e-4, sy1=-5e-4)
HEAVY = {
    "kb4": C.KannalaBrandt4(k1=0.25, k2=-0.12, k3=0.04, k4=-0.015),
    "rt8": C.RadialTangential8(k1=-0.35, k2=0.15, k3=-0.04, k4=0.008, k5=-0.004, p1=0.04, p2=-0.03),
    "tpf": C.ThinPrismFisheye(kb4=C.KannalaBrandt4(k1=-0.18, k2=0.08, k3=-0.015, k4=0.004), p1=0.025,
                              p2=-0.02, sx1=0.015, sy1=-0.018),
}
MODELS = {"kb4": KB4, "rt8": RT8, "tpf": TPF}


def _ulp_err(got, ref):
    ref_f = ref.astype(np.float32)
    ulp = np.maximum(np.spacing(np.abs(ref_f)).astype(np.float64), 1.401298464324817e-45)
    return np.abs(got.astype(np.float64) - ref) / ulp


# ---- atan2 -------------------------------------------------------------------------------------

def test_atan2f_within_2ulp_of_libm():
    rng = np.random.default_rng(5)
    n = 400_000
    mags = np.exp(rng.uniform(-20, 20, (2, n)))
    signs = rng.choice([-1.0, 1.0], (2, n))
    y = (mags[0] * signs[0]).astype(np.float32)
    x = (mags[1] * signs[1]).astype(np.float32)
    # ratios near the reduction breakpoints and near 1
    t = rng.uniform(0.25, 0.29, 50_000).astype(np.float32)
    y = np.concatenate([y, t, np.ones(50_000, np.float32), rng.uniform(-1, 1, 50_000).astype(np.float32)])
    x = np.concatenate([x, np.ones(50_000, np.float32), t, rng.uniform(-1, 1, 50_000).astype(np.float32)])
    got = O.atan2f(y, x)
    ref = np.arctan2(y.astype(np.float64), x.astype(np.float64))
    err = _ulp_err(got, ref)
    assert err.max() <= 2.0, f"max {err.max()} ulp at y={y[err.argmax()]}, x={x[err.argmax()]}"


def test_atan2f_special_cases():
    inf, nan = np.float32(np.inf), np.float32(np.nan)
    cases = [(0.0, 1.0), (-0.0, 1.0), (0.0, -1.0), (-0.0, -1.0), (0.0, 0.0), (0.0, -0.0), (-0.0, -0.0),
             (1.0, 0.0), (-1.0, 0.0), (inf, 1.0), (-inf, 1.0), (1.0, inf), (1.0, -inf), (-1.0, -inf),
             (inf, inf), (inf, -inf), (-inf, -inf), (1e-45, 1.0), (1.0, 1e-45), (3e38, 1e-38)]
    y = np.array([c[0] for c in cases], np.float32)
    x = np.array([c[1] for c in cases], np.float32)
    got = O.atan2f(y, x)
    want = np.arctan2(y.astype(np.float64), x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(np.signbit(got), np.signbit(want))
    assert np.all(_ulp_err(got, np.arctan2(y.astype(np.float64), x.astype(np.float64))) <= 2.0)
    assert np.isnan(O.atan2f(np.array([nan, 1.0], np.float32), np.array([1.0, nan], np.float32))).all()


# ---- fov <-> focal (brush-render/src/tests/mod.rs:795-874) ---------------------------------------

def test_pinhole_focal_to_fov_and_back():
    fov = C.focal_to_fov(800.0, 1920, C.PINHOLE)
    assert abs(C.fov_to_focal(fov, 1920, C.PINHOLE) - 800.0) < 1e-9


def test_kb4_focal_to_fov_no_distortion_is_pixels_over_focal():
    m = C.KannalaBrandt4()
    fov = C.focal_to_fov(300.0, 1024, m)
    assert abs(fov - 1024 / 300.0) < 1e-9
    assert abs(C.fov_to_focal(fov, 1024, m) - 300.0) < 1e-9


@pytest.mark.parametrize("model,f,px", [
    (C.KannalaBrandt4(k1=-0.01, k2=0.003, k3=-0.0005, k4=0.00002), 280.0, 1024),
    (C.RadialTangential8(k1=-0.2, k2=0.05, k3=-0.001), 900.0, 1920),
    (C.ThinPrismFisheye(kb4=C.KannalaBrandt4(k1=-0.01, k2=0.003, k3=-0.0005, k4=0.00002), p1=1e-3, p2=-2e-3,
                        sx1=5e-4, sy1=-5e-4), 280.0, 1024),
])
def test_distorted_focal_to_fov_and_back(model, f, px):
    assert abs(C.fov_to_focal(C.focal_to_fov(f, px, model), px, model) - f) < 1e-6


# ---- float64 closed forms of each model -----------------------------------------------------------

def _coeffs(model):
    return [float(np.float32(v)) for v in model.params()]


def _project64(name, model, fx, fy, cx, cy, p):
    """Screen position of camera-space points p [n, 3] from the model's definition."""
    x, y, z = p[:, 0], p[:, 1], p[:, 2]
    k = _coeffs(model)
    if name == "rt8":
        xn, yn = x / z, y / z
        r2 = xn * xn + yn * yn
        rad = (1 + k[0] * r2 + k[1] * r2 ** 2 + k[2] * r2 ** 3) / (1 + k[3] * r2 + k[4] * r2 ** 2 + k[5] * r2 ** 3)
        xd = xn * rad + 2 * k[6] * xn * yn + k[7] * (r2 + 2 * xn * xn)
        yd = yn * rad + 2 * k[7] * xn * yn + k[6] * (r2 + 2 * yn * yn)
        return np.stack([fx * xd + cx, fy * yd + cy], 1)
    r = np.hypot(x, y)
    th = np.arctan2(r, z)
    d = th * (1 + k[0] * th ** 2 + k[1] * th ** 4 + k[2] * th ** 6 + k[3] * th ** 8)
    u = fx * d * x / r + cx
    v = fy * d * y / r + cy
    if name == "tpf":
        p1, p2, sx1, sy1 = k[4:8]
        un, vn = x / z, y / z
        rn2 = un * un + vn * vn
        u = u + fx * (2 * p1 * un * vn + p2 * (rn2 + 2 * un * un) + sx1 * rn2)
        v = v + fy * (2 * p2 * un * vn + p1 * (rn2 + 2 * vn * vn) + sy1 * rn2)
    return np.stack([u, v], 1)


def _uniforms(model, w=64, h=48, f=60.0):
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), f, w, h, camera_model=model)
    return uniforms_for(cam, w, h, 1, 0)


def _points(rng, n, u, fov_frac=0.9):
    """Camera-space points in front of the camera within the unclamped region."""
    z = rng.uniform(1.0, 6.0, n)
    lim_x = min(abs(float(u["lim_pos_x"])), abs(float(u["lim_neg_x"]))) or 0.6
    lim_y = min(abs(float(u["lim_pos_y"])), abs(float(u["lim_neg_y"]))) or 0.6
    x = rng.uniform(-1, 1, n) * lim_x * fov_frac * z
    y = rng.uniform(-1, 1, n) * lim_y * fov_frac * z
    return np.stack([x, y, z], 1).astype(np.float32)


@pytest.mark.parametrize("name", ["kb4", "rt8", "tpf"])
@pytest.mark.parametrize("heavy", [False, True])
def test_projection_matches_float64_closed_form(name, heavy):
    model = HEAVY[name] if heavy else MODELS[name]
    u = _uniforms(model)
    pts = _points(np.random.default_rng(3), 4000, u)
    got, _ = O.camera_project(u, pts)
    want = _project64(name, model, float(u["fx"]), float(u["fy"]), float(u["cx"]), float(u["cy"]),
                      pts.astype(np.float64))
    scale = float(u["fx"]) * (1.0 + np.abs((want[:, :1] - float(u["cx"])) / float(u["fx"])))
    assert np.max(np.abs(got - want) / scale) < 2e-6


def test_kb4_without_distortion_is_equidistant_and_near_axis_is_pinhole():
    u = _uniforms(C.KannalaBrandt4())
    rng = np.random.default_rng(4)
    pts = _points(rng, 2000, u)
    got, _ = O.camera_project(u, pts)
    p = pts.astype(np.float64)
    r = np.hypot(p[:, 0], p[:, 1])
    th = np.arctan2(r, p[:, 2])
    want = np.stack([float(u["fx"]) * th * p[:, 0] / r + float(u["cx"]),
                     float(u["fy"]) * th * p[:, 1] / r + float(u["cy"])], 1)
    assert np.max(np.abs(got - want)) < 2e-4
    near = np.array([[1e-8, -2e-8, 2.0], [0.0, 0.0, 1.5]], np.float32)
    got, _ = O.camera_project(u, near)
    pin = near[:, :2] / near[:, 2:] * np.array([u["fx"], u["fy"]], np.float32) + np.array([u["cx"], u["cy"]],
                                                                                         np.float32)
    assert np.allclose(got, pin, rtol=1e-6, atol=1e-5)


def test_thin_prism_without_prism_terms_equals_kb4_bit_for_bit():
    u_kb = _uniforms(KB4)
    u_tp = _uniforms(C.ThinPrismFisheye(kb4=KB4))
    rng = np.random.default_rng(6)
    pts = _points(rng, 1000, u_kb)
    assert np.array_equal(O.camera_project(u_kb, pts)[0].view(np.uint32), O.camera_project(u_tp, pts)[0].view(np.uint32))
    assert np.array_equal(O.camera_jacobian(u_kb, pts), O.camera_jacobian(u_tp, pts))
    cov, vc, vm = _vjp_inputs(rng, len(pts))
    assert np.array_equal(O.camera_vjp(u_kb, pts, cov, vc, vm), O.camera_vjp(u_tp, pts, cov, vc, vm))


def test_fisheye_cull_uses_view_angle_not_depth():
    """project_forward.rs:49-62: fisheye models keep points behind the image
    plane within half_max_render_fov and drop those beyond it."""
    cam = Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 3.4, 3.4, (0.5, 0.5), KB4)
    u = uniforms_for(cam, 64, 48, 1, 0)
    half = float(u["half_max_render_fov"])
    assert half > math.pi / 2
    ang_in, ang_out = 0.5 * (math.pi / 2 + half), min(half + 0.05, math.pi)
    pts = np.array([[math.sin(ang_in), 0.0, math.cos(ang_in)], [math.sin(ang_out), 0.0, math.cos(ang_out)],
                    [0.0, 0.0, 0.005]], np.float32)
    _, culled = O.camera_project(u, pts)
    assert culled.tolist() == [False, True, False]
    _, culled = O.camera_project(_uniforms(C.PINHOLE), pts)
    assert culled.tolist() == [True, True, True]


# ---- Jacobians and VJPs against float64 finite differences ---------------------------------------

def _jac64(name, model, u, p, h=1e-6):
    f = (float(u["fx"]), float(u["fy"]), float(u["cx"]), float(u["cy"]))
    cols = []
    for i in range(3):
        e = np.zeros(3)
        e[i] = h * max(1.0, float(np.abs(p).max()))
        cols.append((_project64(name, model, *f, (p + e)[None]) - _project64(name, model, *f, (p - e)[None]))[0]
                    / (2 * e[i]))
    return np.stack(cols, 1)  # [2, 3]


@pytest.mark.parametrize("name", ["kb4", "rt8", "tpf"])
@pytest.mark.parametrize("heavy", [False, True])
def test_jacobian_matches_finite_differences(name, heavy):
    model = HEAVY[name] if heavy else MODELS[name]
    u = _uniforms(model)
    pts = _points(np.random.default_rng(8), 300, u)
    got = O.camera_jacobian(u, pts)
    for i in range(len(pts)):
        want = _jac64(name, model, u, pts[i].astype(np.float64))
        scale = np.abs(want).max()
        assert np.max(np.abs(got[i] - want)) <= 1e-5 * scale, (i, got[i], want)


def _vjp_inputs(rng, n):
    a = rng.standard_normal((n, 3, 3)) * 0.05
    cov = np.einsum("nij,nkj->nik", a, a) + np.eye(3) * 1e-3
    cov6 = np.stack([cov[:, 0, 0], cov[:, 0, 1], cov[:, 0, 2], cov[:, 1, 1], cov[:, 1, 2], cov[:, 2, 2]], 1)
    return (cov6.astype(np.float32), rng.standard_normal((n, 3)).astype(np.float32),
            rng.standard_normal((n, 2)).astype(np.float32))


@pytest.mark.parametrize("name", ["kb4", "rt8", "tpf"])
@pytest.mark.parametrize("heavy", [False, True])
def test_projection_vjp_matches_finite_differences(name, heavy):
    """The VJP is the gradient of v_mean2d . pi(p) + tr(V J(p) S J(p)^T) with
    V the symmetric v_cov2d and S the camera-space covariance."""
    model = HEAVY[name] if heavy else MODELS[name]
    u = _uniforms(model)
    rng = np.random.default_rng(9)
    pts = _points(rng, 60, u)
    cov6, vc, vm = _vjp_inputs(rng, len(pts))
    got = O.camera_vjp(u, pts, cov6, vc, vm)
    f = (float(u["fx"]), float(u["fy"]), float(u["cx"]), float(u["cy"]))
    for i in range(len(pts)):
        c = cov6[i].astype(np.float64)
        S = np.array([[c[0], c[1], c[2]], [c[1], c[3], c[4]], [c[2], c[4], c[5]]])
        V = np.array([[vc[i, 0], vc[i, 1]], [vc[i, 1], vc[i, 2]]], np.float64)

        def loss(p):
            J = _jac64(name, model, u, p)
            return float(vm[i].astype(np.float64) @ _project64(name, model, *f, p[None])[0] +
                         np.trace(V @ J @ S @ J.T))

        p0 = pts[i].astype(np.float64)
        h = 1e-4 * max(1.0, float(np.abs(p0).max()))
        want = np.array([(loss(p0 + h * e) - loss(p0 - h * e)) / (2 * h) for e in np.eye(3)])
        assert np.max(np.abs(got[i] - want)) <= 2e-3 * np.abs(want).max() + 1e-6, (i, got[i], want)


# ---- the whole render through each model ----------------------------------------------------------

def _fd_scene(model):
    rng = np.random.default_rng(31)
    n = 8
    tr = np.zeros((n, 10), np.float32)
    tr[:, 0:2] = rng.uniform(-0.5, 0.5, (n, 2))
    tr[:, 2] = rng.permutation(np.linspace(-0.3, 0.3, n))
    q = rng.standard_normal((n, 4))
    tr[:, 3:7] = q / np.linalg.norm(q, axis=1, keepdims=True)
    tr[:, 7:10] = rng.uniform(-2.3, -1.6, (n, 3))
    sh = (rng.standard_normal((n, 4, 3)) * 0.3).astype(np.float32)
    sh[:, 0, :] += 0.4
    opac = rng.uniform(-1.0, 0.0, n).astype(np.float32)
    cam = Camera.from_focal((0.05, -0.03, -3.0), (0.0, 0.0, 0.0, 1.0), 45.0, 40, 32, camera_model=model)
    return tr, sh, opac, cam


@pytest.mark.parametrize("name", ["kb4", "rt8", "tpf"])
def test_render_backward_matches_finite_differences(name):
    """finite_diff.rs:1132-1180 (camera-model fuzz) on the restatement: analytic
    gradients of sum(W * image) through each camera model against central
    differences, smooth cutoff."""
    tr, sh, opac, cam = _fd_scene(HEAVY[name])
    n = tr.shape[0]
    u = uniforms_for(cam, 40, 32, n, 1)
    bg = (0.1, 0.2, 0.3)
    flags = O.FLAG_BWD_INFO | O.FLAG_SMOOTH_CUTOFF
    weights = np.random.default_rng(2).standard_normal((32, 40, 4)).astype(np.float32)
    fwd = O.render_forward(u, tr, sh, opac, flags, bg)
    assert fwd.num_visible == n
    vc = O.rasterize_backward(fwd, weights, O.FLAG_SMOOTH_CUTOFF, bg)
    vt, vcoef, vo, _ = O.project_backward(fwd, tr, sh, opac, vc)

    def loss(t):
        r = O.render_forward(u, t, sh, opac, flags, bg)
        return float(np.sum(r.out_img.astype(np.float64) * weights))

    for i in range(n):
        for k in (0, 1, 2, 7, 8, 9):
            eps = 1e-3
            plus, minus = tr.copy(), tr.copy()
            plus[i, k] += eps
            minus[i, k] -= eps
            fd = (loss(plus) - loss(minus)) / (2 * eps)
            assert abs(vt[i, k] - fd) <= 0.03 * abs(fd) + 0.03, f"{name} t[{i},{k}]: {vt[i, k]} vs {fd}"


# ---- beyond the Jacobian clamp ------------------------------------------------------------------------
#
# Splats centred beyond 1.15 W (or -0.15 W, and likewise for H) get a
# Jacobian evaluated at the clamped direction (camera.rs:200-254,
# pinhole.rs:32-56, radial_tangential_8.rs:67-130).  The pinhole VJP
# (pinhole.rs:58-123) is the exact derivative of that forward: the screen
# position uses the unclamped point, the covariance the clamped Jacobian, so
# d/dx of the Jacobian is zero and d/dz goes through the clamped x.  RT8's VJP
# (radial_tangential_8.rs:155-330) differentiates a surrogate instead: the
# projection of the clamped point c(p) = (clamp(x/z) z, clamp(y/z) z, z), and a
# covariance J(c(p)) S V S^T J(c(p))^T with S = dc/dp (constant inside a
# clamped region), so that no gradient moves a clamped splat along the
# clamped axis.  Both are checked against float64 central differences, at
# points whose normalised coordinate is 20-80 % of the limit beyond it, so no
# step crosses the kink.


def _clamp_points(rng, n, u, axes):
    """Camera-space points beyond the clamp limit on the given axes ("x", "y"
    or both), on either side, inside the limit on the others."""
    z = rng.uniform(1.0, 6.0, n)
    out = []
    for ax in ("x", "y"):
        pos, neg = float(u[f"lim_pos_{ax}"]), float(u[f"lim_neg_{ax}"])
        if ax in axes:
            side = rng.integers(0, 2, n)
            t = np.where(side == 1, pos + rng.uniform(0.2, 0.8, n) * abs(pos),
                         neg - rng.uniform(0.2, 0.8, n) * abs(neg))
        else:
            t = rng.uniform(0.1, 0.9, n) * np.where(rng.integers(0, 2, n) == 1, pos, neg)
        out.append(t * z)
    return np.stack([out[0], out[1], z], 1).astype(np.float32)


def _clampmap(u, p):
    """c(p) and S = dc/dp at p (float64)."""
    lims = {ax: (float(np.float32(u[f"lim_neg_{ax}"])), float(np.float32(u[f"lim_pos_{ax}"]))) for ax in "xy"}
    c = p.copy()
    S = np.eye(3)
    for i, ax in enumerate("xy"):
        t = p[i] / p[2]
        lo, hi = lims[ax]
        if t < lo or t > hi:
            tc = min(max(t, lo), hi)
            c[i] = tc * p[2]
            S[i, i], S[i, 2] = 0.0, tc
    return c, S


def _pinhole64(u, p):
    fx, fy, cx, cy = (float(u[k]) for k in ("fx", "fy", "cx", "cy"))
    return np.array([fx * p[0] / p[2] + cx, fy * p[1] / p[2] + cy])


def _pinhole_jac_clamped64(u, p):
    fx, fy = float(u["fx"]), float(u["fy"])
    c, _ = _clampmap(u, p)
    tx, ty = c[0] / p[2], c[1] / p[2]
    return np.array([[fx / p[2], 0.0, -fx * tx / p[2]], [0.0, fy / p[2], -fy * ty / p[2]]])


@pytest.mark.parametrize("axes", ["x", "y", "xy"])
def test_clamped_pinhole_vjp_is_the_derivative_of_the_forward(axes):
    u = _uniforms(C.PINHOLE)
    rng = np.random.default_rng(40 + len(axes))
    pts = _clamp_points(rng, 80, u, axes)
    cov6, vc, vm = _vjp_inputs(rng, len(pts))
    # the forward's Jacobian is the clamped one
    got_j = O.camera_jacobian(u, pts)
    for i in range(len(pts)):
        want_j = _pinhole_jac_clamped64(u, pts[i].astype(np.float64))
        assert np.max(np.abs(got_j[i] - want_j)) <= 1e-5 * np.abs(want_j).max(), (i, got_j[i], want_j)
    got = O.camera_vjp(u, pts, cov6, vc, vm)
    for i in range(len(pts)):
        c = cov6[i].astype(np.float64)
        S = np.array([[c[0], c[1], c[2]], [c[1], c[3], c[4]], [c[2], c[4], c[5]]])
        V = np.array([[vc[i, 0], vc[i, 1]], [vc[i, 1], vc[i, 2]]], np.float64)

        def loss(p):
            J = _pinhole_jac_clamped64(u, p)
            return float(vm[i].astype(np.float64) @ _pinhole64(u, p) + np.trace(V @ J @ S @ J.T))

        p0 = pts[i].astype(np.float64)
        h = 1e-5 * max(1.0, float(np.abs(p0).max()))
        want = np.array([(loss(p0 + h * e) - loss(p0 - h * e)) / (2 * h) for e in np.eye(3)])
        assert np.max(np.abs(got[i] - want)) <= 2e-4 * np.abs(want).max() + 1e-6, (i, got[i], want)
    # through the covariance alone a clamped axis gets exactly zero
    zero_vm = np.zeros_like(vm)
    g0 = O.camera_vjp(u, pts, cov6, vc, zero_vm)
    for i, p in enumerate(pts):
        for k, ax in enumerate("xy"):
            t = float(p[k]) / float(p[2])
            if t > float(u[f"lim_pos_{ax}"]) or t < float(u[f"lim_neg_{ax}"]):
                assert g0[i, k] == 0.0, (i, ax, g0[i])


@pytest.mark.parametrize("heavy", [False, True])
@pytest.mark.parametrize("axes", ["x", "y", "xy"])
def test_clamped_rt8_vjp_is_the_derivative_of_its_surrogate(heavy, axes):
    model = HEAVY["rt8"] if heavy else MODELS["rt8"]
    u = _uniforms(model)
    rng = np.random.default_rng(50 + len(axes) + (7 if heavy else 0))
    pts = _clamp_points(rng, 60, u, axes)
    cov6, vc, vm = _vjp_inputs(rng, len(pts))
    got = O.camera_vjp(u, pts, cov6, vc, vm)
    f = (float(u["fx"]), float(u["fy"]), float(u["cx"]), float(u["cy"]))
    for i in range(len(pts)):
        c6 = cov6[i].astype(np.float64)
        Sig = np.array([[c6[0], c6[1], c6[2]], [c6[1], c6[3], c6[4]], [c6[2], c6[4], c6[5]]])
        V = np.array([[vc[i, 0], vc[i, 1]], [vc[i, 1], vc[i, 2]]], np.float64)
        p0 = pts[i].astype(np.float64)
        _, S0 = _clampmap(u, p0)
        # the forward's Jacobian is the model's Jacobian at the clamped point
        c0, _ = _clampmap(u, p0)
        want_j = _jac64("rt8", model, u, c0)
        assert np.max(np.abs(O.camera_jacobian(u, pts[i:i + 1])[0] - want_j)) <= 1e-5 * np.abs(want_j).max()

        def loss(p):
            c, _ = _clampmap(u, p)
            J = _jac64("rt8", model, u, c)
            return float(vm[i].astype(np.float64) @ _project64("rt8", model, *f, c[None])[0] +
                         np.trace(V @ J @ S0 @ Sig @ S0.T @ J.T))

        def loss_open(p):
            # the same terms without the clamp's routing: the size of what
            # cancels when both axes are clamped (J(c(p)) S is then zero)
            J = _jac64("rt8", model, u, p)
            return float(vm[i].astype(np.float64) @ _project64("rt8", model, *f, p[None])[0] +
                         np.trace(V @ J @ Sig @ J.T))

        h = 1e-4 * max(1.0, float(np.abs(p0).max()))
        want = np.array([(loss(p0 + h * e) - loss(p0 - h * e)) / (2 * h) for e in np.eye(3)])
        terms = np.array([(loss_open(c0 + h * e) - loss_open(c0 - h * e)) / (2 * h) for e in np.eye(3)])
        tol = 2e-3 * np.abs(want).max() + 1e-5 * np.abs(terms).max() + 1e-6
        assert np.max(np.abs(got[i] - want)) <= tol, (i, got[i], want)
        # a clamped axis gets no gradient at all
        for k in range(2):
            if S0[k, k] == 0.0:
                assert got[i, k] == 0.0, (i, k, got[i])
