"""Pins the CPU restatement's backward paths that the SH-3 north-star workload
and the Mip / depth / refine variants take, independently of the kernels:

* central finite differences of the restatement's own forward, on the
  reference's scenes and with its tolerances
  (crates/brush-bench-test/tests/finite_diff.rs): the broad check (:530-595),
  tangential quaternion directions (:600-673), Mip mode (:677-792), the view
  direction of SH degree 2-4 through the means (:1659-1745) and every band of
  the SH coefficients (:1748-1831);
* closed forms for the lanes finite differences cannot reach: the refine
  weight (rasterize_backwards.rs:412-427) and its NaN / clamp cleanup
  (project_backwards.rs:194-195), and the detached depth lane
  (rasterize_backwards.rs:379-396), whose blending weights come from a
  float64 front-to-back walk written here.

The reference computes its losses in f32 on the GPU; here the f32 image of
the restatement is summed in float64, and each difference quotient divides by
the step actually taken in f32.
"""
import math

import numpy as np
import pytest

from brush_amd.camera import Camera
from oracle import oracle as O
from tests.helpers import uniforms_for

SMOOTH = O.FLAG_BWD_INFO | O.FLAG_SMOOTH_CUTOFF


def _reference_base_scene():
    """finite_diff.rs:48-77: four splats inside the image, non-axis-aligned
    (non-unit) rotations, moderate opacity."""
    means = [[0.20, -0.10, 0.00], [-0.30, 0.40, 0.20], [0.10, 0.30, -0.30], [-0.20, -0.20, 0.10]]
    rots = [[0.90, 0.10, 0.05, 0.03], [0.70, 0.20, 0.30, 0.10], [0.50, 0.40, 0.30, 0.20], [0.80, 0.10, 0.10, 0.20]]
    log_scales = [[-1.4, -1.5, -1.6], [-1.5, -1.4, -1.3], [-1.7, -1.5, -1.4], [-1.3, -1.6, -1.5]]
    sh_dc = [[0.45, 0.55, 0.50], [0.60, 0.40, 0.30], [0.35, 0.50, 0.65], [0.50, 0.45, 0.55]]
    tr = np.concatenate([np.array(means), np.array(rots), np.array(log_scales)], 1).astype(np.float32)
    sh = np.array(sh_dc, np.float32).reshape(4, 1, 3)
    opac = np.array([2.5, 2.0, 2.2, 2.4], np.float32)
    return tr, sh, opac


def _std_cam():
    """finite_diff.rs:79-88: at (0, 0, -3), identity rotation, fov 0.6 x 0.6."""
    return Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.6, 0.6)


class _Problem:
    """mean(image) of a scene (the reference's loss, finite_diff.rs:102-131)
    and its analytic gradient through the restatement's backward."""

    def __init__(self, cam, size, tr, sh, opac, flags=SMOOTH):
        self.cam, self.size, self.flags = cam, size, flags
        self.tr, self.sh, self.opac = tr, sh, opac
        w, h = size
        self.u = uniforms_for(cam, w, h, tr.shape[0], int(round(sh.shape[1] ** 0.5)) - 1)
        self.weight = np.float32(1.0 / (w * h * 4))

    def loss(self, tr, sh, opac) -> float:
        r = O.render_forward(self.u, tr, sh, opac, self.flags)
        return float(np.sum(r.out_img.astype(np.float64))) / (self.size[0] * self.size[1] * 4)

    def grads(self):
        fwd = O.render_forward(self.u, self.tr, self.sh, self.opac, self.flags)
        v_out = np.full(fwd.out_img.shape, self.weight, np.float32)
        vc = O.rasterize_backward(fwd, v_out, self.flags & O.FLAG_SMOOTH_CUTOFF)
        return fwd, O.project_backward(fwd, self.tr, self.sh, self.opac, vc, mip=bool(self.flags & O.FLAG_MIP))

    def fd(self, which: str, index, eps: float) -> float:
        """Central difference along one scalar of transforms ('t'), SH ('c') or
        opacity ('o')."""
        arrs = {"t": self.tr, "c": self.sh, "o": self.opac}
        plus, minus = arrs[which].copy(), arrs[which].copy()
        plus[index] += np.float32(eps)
        minus[index] -= np.float32(eps)
        step = float(plus[index]) - float(minus[index])
        args = {"t": lambda a: (a, self.sh, self.opac), "c": lambda a: (self.tr, a, self.opac),
                "o": lambda a: (self.tr, self.sh, a)}[which]
        return (self.loss(*args(plus)) - self.loss(*args(minus))) / step

    def fd_dir(self, index_row: int, cols, direction, eps: float) -> float:
        """Central difference of the transforms along a direction over columns."""
        plus, minus = self.tr.copy(), self.tr.copy()
        for c, d in zip(cols, direction):
            plus[index_row, c] += np.float32(eps * d)
            minus[index_row, c] -= np.float32(eps * d)
        return (self.loss(plus, self.sh, self.opac) - self.loss(minus, self.sh, self.opac)) / (2.0 * eps)


def _close(num, an, rel_tol, abs_tol) -> bool:
    scale = max(abs(num), abs(an), 1e-8)
    return abs(num - an) <= abs_tol + rel_tol * scale


# transforms columns: means 0-2, quaternion w x y z 3-6, log-scales 7-9
_LANES = {"means": 0, "rots": 3, "log_scales": 7}


def _analytic(grads, lane, splat, comp):
    vt, vcoef, vo, _ = grads
    if lane == "sh_dc":
        return float(vcoef[splat, 0, comp])
    if lane == "raw_opac":
        return float(vo[splat])
    return float(vt[splat, _LANES[lane] + comp])


def _numeric(p: _Problem, lane, splat, comp, eps):
    if lane == "sh_dc":
        return p.fd("c", (splat, 0, comp), eps)
    if lane == "raw_opac":
        return p.fd("o", (splat,), eps)
    return p.fd("t", (splat, _LANES[lane] + comp), eps)


def test_finite_difference_gradient_broad():
    """finite_diff.rs:530-595: a few indices of every parameter category,
    eps 3e-4, 1 % relative + 5e-5 absolute."""
    tr, sh, opac = _reference_base_scene()
    p = _Problem(_std_cam(), (32, 32), tr, sh, opac)
    fwd, grads = p.grads()
    assert fwd.num_visible == 4
    cases = [("means", 0, 0), ("means", 0, 2), ("means", 1, 1), ("rots", 0, 0), ("rots", 1, 2),
             ("log_scales", 0, 0), ("log_scales", 1, 1), ("sh_dc", 0, 0), ("sh_dc", 1, 1), ("sh_dc", 2, 2),
             ("raw_opac", 0, 0), ("raw_opac", 2, 0)]
    bad = []
    for lane, s, c in cases:
        num, an = _numeric(p, lane, s, c, 3e-4), _analytic(grads, lane, s, c)
        if not _close(num, an, 0.01, 5e-5):
            bad.append(f"{lane}[{s},{c}]: numerical {num:.6g} vs analytical {an:.6g}")
    assert not bad, "\n".join(bad)


def test_finite_diff_tangential_quat():
    """finite_diff.rs:600-673: the radial direction of the quaternion has ~0
    gradient (normalisation projects it out); tangent directions agree with
    central differences at 1 % + 5e-5."""
    tr, sh, opac = _reference_base_scene()
    tr[0, 3:7] = [1.0, 0.0, 0.0, 0.0]
    tr[0, 7:10] = [-1.0, -2.8, -1.5]
    p = _Problem(_std_cam(), (64, 64), tr, sh, opac)
    _, (vt, _, _, _) = p.grads()
    q_grad = vt[0, 3:7].astype(np.float64)
    assert abs(q_grad[0]) < 1e-4, f"radial quaternion gradient {q_grad[0]}"
    bad = []
    for t in ([0.0, 1.0, 0.0, 0.0], [0.0, 0.0, 1.0, 0.0], [0.0, 0.0, 0.0, 1.0], [0.0, 0.6, 0.0, 0.8]):
        num = p.fd_dir(0, range(3, 7), t, 3e-4)
        an = float(np.dot(q_grad, t))
        if not _close(num, an, 0.01, 5e-5):
            bad.append(f"{t}: numerical {num:.6g} vs analytical {an:.6g}")
    assert not bad, "\n".join(bad)


def test_finite_diff_broad_mip_mode():
    """finite_diff.rs:677-792: SplatRenderMode::Mip on the same scene, 3 %
    relative + 1e-4 absolute.  The reference's Mip backward keeps the
    compensation factor as a constant in the covariance VJP (its derivative
    with respect to the covariance is not propagated, project_backwards.rs:
    188-190); on splats of this size that term is below the tolerance."""
    tr, sh, opac = _reference_base_scene()
    p = _Problem(_std_cam(), (32, 32), tr, sh, opac, SMOOTH | O.FLAG_MIP)
    fwd, grads = p.grads()
    assert fwd.num_visible == 4
    bad = []
    for lane, s, c in [("means", 0, 0), ("means", 1, 1), ("log_scales", 0, 0), ("log_scales", 1, 1),
                       ("sh_dc", 0, 0), ("raw_opac", 0, 0)]:
        num, an = _numeric(p, lane, s, c, 3e-4), _analytic(grads, lane, s, c)
        if not _close(num, an, 0.03, 1e-4):
            bad.append(f"{lane}[{s},{c}]: numerical {num:.6g} vs analytical {an:.6g}")
    assert not bad, "\n".join(bad)


def test_mip_mode_changes_the_gradients():
    """The Mip forward and backward are a different computation (a blur of 0.1
    instead of 0.3, and the opacity compensation): its gradients must not be
    the Default mode's, so the test above cannot pass on a path that ignores
    the flag."""
    tr, sh, opac = _reference_base_scene()
    _, g_def = _Problem(_std_cam(), (32, 32), tr, sh, opac).grads()
    _, g_mip = _Problem(_std_cam(), (32, 32), tr, sh, opac, SMOOTH | O.FLAG_MIP).grads()
    assert np.max(np.abs(g_def[0] - g_mip[0])) > 1e-3 * np.max(np.abs(g_def[0]))
    assert np.max(np.abs(g_def[2] - g_mip[2])) > 1e-3 * np.max(np.abs(g_def[2]))


def _high_sh_scene(degree: int):
    """finite_diff.rs:1659-1690 generalised to any degree: two splats off
    axis, log-scales -1, DC 0.5, higher bands 0.4 sin(splat + coef + ch)."""
    nc = (degree + 1) ** 2
    tr = np.zeros((2, 10), np.float32)
    tr[0, :3] = [0.4, -0.2, 0.0]
    tr[1, :3] = [-0.3, 0.3, 0.2]
    tr[:, 3] = 1.0
    tr[:, 7:10] = -1.0
    sh = np.zeros((2, nc, 3), np.float32)
    sh[:, 0, :] = 0.5
    for s in range(2):
        for c in range(1, nc):
            for ch in range(3):
                sh[s, c, ch] = np.float32(0.4 * math.sin(s + c + ch))
    return tr, sh, np.array([2.0, 2.0], np.float32)


@pytest.mark.parametrize("degree", [2, 3, 4])
def test_finite_diff_means_through_high_sh(degree):
    """finite_diff.rs:1659-1745 (degree 2 in the reference; also 3 and 4 here):
    the colour depends on the view direction, which depends on the mean, so the
    mean gradient carries the SH view-direction VJP.  Best of an eps sweep per
    component, 5 % relative + 5e-4 absolute."""
    tr, sh, opac = _high_sh_scene(degree)
    p = _Problem(_std_cam(), (48, 48), tr, sh, opac)
    fwd, grads = p.grads()
    assert fwd.num_visible == 2
    bad = []
    for s in range(2):
        for comp in range(3):
            an = float(grads[0][s, comp])
            best = None
            for eps in (3e-2, 3e-3, 1e-3, 3e-4, 1e-4):
                num = p.fd("t", (s, comp), eps)
                rel = abs(num - an) / max(abs(num), abs(an), 1e-8)
                if best is None or rel < best[0]:
                    best = (rel, num)
            if not _close(best[1], an, 0.05, 5e-4):
                bad.append(f"deg {degree} means[{s},{comp}]: numerical {best[1]:.6g} vs analytical {an:.6g}")
    assert not bad, "\n".join(bad)


@pytest.mark.parametrize("degree", [2, 3, 4])
def test_high_sh_view_direction_term_exceeds_the_tolerance(degree):
    """The finite-difference test above has the power to catch a missing
    view-direction VJP (the bug finite_diff.rs:1650-1658 documents): the part
    of the mean gradient that flows through the colour, sum_k dL/drgb_k
    drgb_k/dmean, is many times that test's tolerance for some component.
    dL/drgb is lanes 5-7 of v_combined; drgb/dmean is a central difference of
    the forward's SH colours (projected lanes 6-8, pinned by the gsplat SH3
    goldens)."""
    tr, sh, opac = _high_sh_scene(degree)
    p = _Problem(_std_cam(), (48, 48), tr, sh, opac)
    fwd = O.render_forward(p.u, tr, sh, opac, p.flags)
    vc = O.rasterize_backward(fwd, np.full(fwd.out_img.shape, p.weight, np.float32), O.FLAG_SMOOTH_CUTOFF)
    grads = O.project_backward(fwd, tr, sh, opac, vc)[0]
    worst = 0.0
    for c in range(fwd.num_visible):
        g = int(fwd.global_from_compact_gid[c])
        for comp in range(3):
            eps = 1e-3
            plus, minus = tr.copy(), tr.copy()
            plus[g, comp] += np.float32(eps)
            minus[g, comp] -= np.float32(eps)
            rp = O.render_forward(p.u, plus, sh, opac, p.flags)
            rm = O.render_forward(p.u, minus, sh, opac, p.flags)
            cp = rp.projected[list(rp.global_from_compact_gid).index(g), 6:9].astype(np.float64)
            cm = rm.projected[list(rm.global_from_compact_gid).index(g), 6:9].astype(np.float64)
            term = float(np.dot(vc[c, 5:8], (cp - cm) / (float(plus[g, comp]) - float(minus[g, comp]))))
            an = float(grads[g, comp])
            tol = 5e-4 + 0.05 * abs(an)
            worst = max(worst, abs(term) / tol)
    assert worst > 3.0, f"view-direction term at most {worst:.2f}x the tolerance"


@pytest.mark.parametrize("degree", [3, 4])
def test_finite_diff_high_band_sh_coefficients(degree):
    """finite_diff.rs:1748-1831 (degree 4 in the reference; also 3 here):
    an offscreen splat first, so the visible splat is compact id 0 at global
    row 1; the offscreen row's SH gradient is exactly zero; every band checked
    by central differences at eps 3e-2, 4 % relative + 2e-5 absolute."""
    nc = (degree + 1) ** 2
    cam = Camera((-0.8, 0.6, -2.0), (0.0, 0.0, 0.0, 1.0), 0.9, 0.9)
    tr = np.array([[100.0, 100.0, 0.1, 0.9, 0.1, 0.05, 0.02, -0.8, -0.9, -1.0],
                   [0.4, -0.3, 0.1, 0.9, 0.1, 0.05, 0.02, -0.8, -0.9, -1.0]], np.float32)
    sh = np.zeros((2, nc, 3), np.float32)
    for ch in range(3):
        sh[1, 0, ch] = 0.25 + ch * 0.05
    for c in range(1, nc):
        for ch in range(3):
            sh[1, c, ch] = 0.02 * (c + ch + 1)
    opac = np.array([2.0, 2.0], np.float32)
    p = _Problem(cam, (48, 48), tr, sh, opac)
    fwd, (_, vcoef, _, _) = p.grads()
    assert fwd.num_visible == 1 and int(fwd.global_from_compact_gid[0]) == 1
    assert np.all(vcoef[0] == 0.0), "offscreen SH gradient row must be exactly zero"
    cases = [c * 3 + c % 3 for c in range(nc)] + ([32, 64, 74] if degree == 4 else [32, 47])
    bad = []
    for flat in cases:
        c, ch = flat // 3, flat % 3
        num = p.fd("c", (1, c, ch), 3e-2)
        an = float(vcoef[1, c, ch])
        if not _close(num, an, 0.04, 2e-5):
            bad.append(f"deg {degree} SH[{c},{ch}]: numerical {num:.6g} vs analytical {an:.6g}")
    assert not bad, "\n".join(bad)


@pytest.mark.parametrize("degree", [1, 2, 3, 4])
def test_sh_vjps_against_differences_of_the_forward_colour(degree):
    """The SH VJPs in isolation, at view directions far from the axis (a wide
    camera close to the splats): with only the colour lanes 5-7 of v_combined
    set to w, project_backward's mean gradient is exactly the view-direction
    term sum_k w_k drgb_k/dmean (the geometric lanes are zero) and its
    coefficient gradient is w_ch drgb_ch/dcoef (sh.rs:249-466).  Both are
    compared with central differences of the forward's SH colour (projected
    lanes 6-8, pinned by the gsplat SH3 goldens) at 2e-3 relative."""
    rng = np.random.default_rng(100 + degree)
    nc = (degree + 1) ** 2
    n = 10
    tr = np.zeros((n, 10), np.float32)
    tr[:, 0:2] = rng.uniform(-0.9, 0.9, (n, 2))
    tr[:, 2] = np.linspace(-0.4, 0.4, n)
    tr[:, 3] = 1.0
    tr[:, 7:10] = -2.5
    sh = (rng.standard_normal((n, nc, 3)) * 0.25).astype(np.float32)
    opac = np.zeros(n, np.float32)
    cam = Camera((0.0, 0.0, -1.6), (0.0, 0.0, 0.0, 1.0), 1.7, 1.7)
    u = uniforms_for(cam, 64, 64, n, degree)
    fwd = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    assert fwd.num_visible == n
    gfc = list(fwd.global_from_compact_gid)
    w = rng.standard_normal((n, 3)).astype(np.float32)
    vc = np.zeros((n, 11), np.float32)
    for c, g in enumerate(gfc):
        vc[c, 5:8] = w[g]
    vt, vcoef, _, _ = O.project_backward(fwd, tr, sh, opac, vc)

    def colour(t, s, g):
        r = O.render_forward(u, t, s, opac, O.FLAG_BWD_INFO)
        return r.projected[list(r.global_from_compact_gid).index(g), 6:9].astype(np.float64)

    bad = []
    for g in range(n):
        for comp in range(3):
            eps = 2e-3
            plus, minus = tr.copy(), tr.copy()
            plus[g, comp] += np.float32(eps)
            minus[g, comp] -= np.float32(eps)
            d = (colour(plus, sh, g) - colour(minus, sh, g)) / (float(plus[g, comp]) - float(minus[g, comp]))
            num, an = float(np.dot(w[g], d)), float(vt[g, comp])
            if not _close(num, an, 2e-3, 2e-5):
                bad.append(f"deg {degree} splat {g} mean[{comp}]: numerical {num:.6g} vs analytical {an:.6g}")
        for k in range(nc):
            for ch in range(3):
                eps = 0.05
                plus, minus = sh.copy(), sh.copy()
                plus[g, k, ch] += np.float32(eps)
                minus[g, k, ch] -= np.float32(eps)
                d = (colour(tr, plus, g)[ch] - colour(tr, minus, g)[ch]) / (float(plus[g, k, ch]) - float(minus[g, k, ch]))
                num, an = float(w[g, ch] * d), float(vcoef[g, k, ch])
                if not _close(num, an, 2e-3, 2e-6):
                    bad.append(f"deg {degree} splat {g} coef[{k},{ch}]: numerical {num:.6g} vs analytical {an:.6g}")
    assert not bad, "\n".join(bad[:20])
    assert np.all(vt[:, 3:] == 0.0)


def _row_jacobian(u, tr, sh, opac, flags, g, which, index, eps):
    """Central difference of splat g's projected row (x y c00 c01 c11 opac r g
    b depth) along one parameter scalar, found by global id in each render."""
    arrs = {"t": tr, "c": sh, "o": opac}
    plus, minus = arrs[which].copy(), arrs[which].copy()
    plus[index] += np.float32(eps)
    minus[index] -= np.float32(eps)
    step = float(plus[index]) - float(minus[index])
    rows = []
    for a in (plus, minus):
        args = {"t": (a, sh, opac), "c": (tr, a, opac), "o": (tr, sh, a)}[which]
        r = O.render_forward(u, *args, flags)
        rows.append(r.projected[list(r.global_from_compact_gid).index(g)].astype(np.float64))
    return (rows[0] - rows[1]) / step


# v_combined lane -> projected lane it is the gradient of (rasterize_backwards.rs:28-40,
# helpers.rs:192-196); lane 9 (refine) is not a derivative and is pinned separately
_LANE_OF_ROW = {0: 0, 1: 1, 2: 2, 3: 3, 4: 4, 5: 6, 6: 7, 7: 8, 8: 5, 10: 9}


@pytest.mark.parametrize("mip", [False, True])
@pytest.mark.parametrize("group", [(0, 1), (2, 3, 4), (5, 6, 7), (8,), (10,)])
def test_project_backward_lanes_against_forward_differences(mip, group):
    """project_backward in isolation (project_backwards.rs:101-263): with only
    one group of v_combined lanes set (2D mean, conic, colour, opacity, depth)
    every dense gradient equals sum_lane v_lane dprojected_lane/dparam, with
    the derivative a central difference of the forward's projected row, on
    small splats (0.3-3 px) seen from wide angles, where the blur (0.3, or 0.1
    with Mip) and the view direction matter, at 4e-3 relative.  The one term
    the reference leaves out is asserted as left out: in Mip mode the opacity
    row depends on the covariance through the compensation factor, and the
    reference propagates no gradient along it (project_backwards.rs:188-190),
    so the opacity lane gives exactly zero transform gradients."""
    rng = np.random.default_rng(7 + 31 * len(group) + (1000 if mip else 0))
    n, degree = 6, 2
    nc = (degree + 1) ** 2
    tr = np.zeros((n, 10), np.float32)
    tr[:, 0:2] = rng.uniform(-0.8, 0.8, (n, 2))
    tr[:, 2] = np.linspace(-0.3, 0.3, n)
    q = rng.standard_normal((n, 4))
    tr[:, 3:7] = q / np.linalg.norm(q, axis=1, keepdims=True)
    tr[:, 7:10] = rng.uniform(-5.2, -3.6, (n, 3))
    sh = (rng.standard_normal((n, nc, 3)) * 0.2).astype(np.float32)
    sh[:, 0, :] += 1.0
    opac = rng.uniform(-0.5, 1.0, n).astype(np.float32)
    cam = Camera((0.1, -0.05, -1.8), (0.0, 0.0, 0.0, 1.0), 1.6, 1.4)
    flags = O.FLAG_BWD_INFO | (O.FLAG_MIP if mip else 0)
    u = uniforms_for(cam, 96, 80, n, degree)
    fwd = O.render_forward(u, tr, sh, opac, flags)
    assert fwd.num_visible == n
    gfc = list(fwd.global_from_compact_gid)
    v = rng.standard_normal((n, 11)).astype(np.float32)
    vc = np.zeros((n, 11), np.float32)
    for c, g in enumerate(gfc):
        for lane in group:
            vc[c, lane] = v[g, lane]
    vt, vcoef, vo, _ = O.project_backward(fwd, tr, sh, opac, vc, mip=mip)
    params = [("t", (g, k)) for g in range(n) for k in range(10)] + \
             [("c", (g, k, ch)) for g in range(n) for k in range(nc) for ch in range(3)] + \
             [("o", (g,)) for g in range(n)]
    got = {"t": vt, "c": vcoef, "o": vo}
    scale = max(float(np.max(np.abs(a))) for a in (vt, vcoef, vo)) or 1.0
    bad = []
    for which, idx in params:
        g = idx[0]
        an = float(got[which][idx])
        if mip and group == (8,) and which == "t":
            assert an == 0.0
            continue
        # f32 rows: steps below ~1e-2 leave rounding noise in the quotient
        # (the truncation error at 1e-2 is ~1e-4 relative)
        eps = 0.05 if which == "c" else 1e-2
        d = _row_jacobian(u, tr, sh, opac, flags, g, which, idx, eps)
        num = sum(float(v[g, lane]) * d[_LANE_OF_ROW[lane]] for lane in group)
        if abs(num - an) > 4e-3 * max(abs(num), abs(an)) + 2e-5 * scale:
            bad.append(f"{which}{idx}: numerical {num:.6g} vs analytical {an:.6g}")
    assert not bad, f"{len(bad)} mismatches:\n" + "\n".join(bad[:20])


# ---- closed forms: refine weight and depth lane ---------------------------------------------------

def _single_splat(img=(24, 20)):
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 40.0, *img)
    tr = np.array([[0.03, -0.02, 0.0, 0.95, 0.2, -0.1, 0.15, -1.6, -1.9, -1.7]], np.float32)
    sh = np.full((1, 1, 3), 0.6, np.float32)
    opac = np.array([0.8], np.float32)
    return cam, tr, sh, opac


def test_refine_weight_closed_form_one_pixel():
    """rasterize_backwards.rs:412-427: with the upstream gradient on one pixel,
    lane 9 = |(v_x W, v_y H)| / max(A, 1e-5), where (v_x, v_y) = lanes 0-1
    (the pixel's 2D-mean gradient, pinned by the finite differences above)
    and A the pixel's final alpha."""
    cam, tr, sh, opac = _single_splat()
    w, h = 24, 20
    u = uniforms_for(cam, w, h, 1, 0)
    fwd = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    assert fwd.num_visible == 1
    checked = 0
    for (py, px) in [(10, 12), (8, 14), (12, 9), (9, 11)]:
        a = float(fwd.out_img[py, px, 3])
        if a < 2.0 / 255.0:
            continue
        v = np.zeros((h, w, 4), np.float32)
        v[py, px] = [0.7, -1.3, 0.4, 0.9]
        vc = O.rasterize_backward(fwd, v, O.FLAG_REFINE_WEIGHT)
        vx, vy = float(vc[0, 0]), float(vc[0, 1])
        assert vx != 0.0 or vy != 0.0
        want = math.hypot(vx * w, vy * h) / max(a, 1e-5)
        assert abs(float(vc[0, 9]) - want) <= 1e-5 * want
        checked += 1
    assert checked >= 3


def test_refine_weight_sums_per_pixel_norms():
    """The refine lane adds one norm per contributing pixel (not the norm of
    the summed gradient): with two weighted pixels it equals the sum of the
    two one-pixel values; lanes 0-8 are linear in the upstream gradient."""
    cam, tr, sh, opac = _single_splat()
    w, h = 24, 20
    u = uniforms_for(cam, w, h, 1, 0)
    fwd = O.render_forward(u, tr, sh, opac, O.FLAG_BWD_INFO)
    va = np.zeros((h, w, 4), np.float32)
    vb = np.zeros((h, w, 4), np.float32)
    va[10, 12] = [0.7, -1.3, 0.4, 0.9]
    vb[9, 10] = [-0.5, 0.2, 1.1, -0.3]
    ga = O.rasterize_backward(fwd, va, O.FLAG_REFINE_WEIGHT)
    gb = O.rasterize_backward(fwd, vb, O.FLAG_REFINE_WEIGHT)
    gab = O.rasterize_backward(fwd, va + vb, O.FLAG_REFINE_WEIGHT)
    np.testing.assert_allclose(gab[0, 9], ga[0, 9] + gb[0, 9], rtol=1e-6)
    np.testing.assert_allclose(gab[0, :9], ga[0, :9] + gb[0, :9], rtol=1e-5, atol=1e-9)
    norm_of_sum = math.hypot(float(gab[0, 0]) * w, float(gab[0, 1]) * h)
    assert abs(norm_of_sum - float(ga[0, 9] * fwd.out_img[10, 12, 3])) > 1e-6  # the lanes are not one norm


def test_refine_weight_cleanup_in_project_backward():
    """project_backwards.rs:194-195: the refine lane passes through NaN -> 0
    and clamp(., 0, 1e32), written at the splat's global id."""
    rng = np.random.default_rng(4)
    n = 6
    tr = np.zeros((n, 10), np.float32)
    tr[:, 0] = np.linspace(-0.4, 0.4, n)
    tr[:, 2] = np.linspace(-0.2, 0.2, n)[::-1]
    tr[:, 3] = 1.0
    tr[:, 7:10] = -2.0
    sh = np.full((n, 1, 3), 0.5, np.float32)
    opac = np.zeros(n, np.float32)
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 50.0, 48, 32)
    fwd = O.render_forward(uniforms_for(cam, 48, 32, n, 0), tr, sh, opac, O.FLAG_BWD_INFO)
    assert fwd.num_visible == n
    vc = np.zeros((n, 11), np.float32)
    lane9 = np.array([np.nan, np.inf, -5.0, 1e38, 3.0, -np.inf], np.float32)
    vc[:, 9] = lane9
    vc[:, 8] = rng.standard_normal(n).astype(np.float32)
    _, _, _, vr = O.project_backward(fwd, tr, sh, opac, vc)
    want = np.array([0.0, 0.0, 0.0, 1e32, 3.0, 0.0], np.float32)
    np.testing.assert_array_equal(vr[fwd.global_from_compact_gid], want)


def _blend_weights_f64(projected, img_w, img_h):
    """Front-to-back blending weights w[c, y, x] = alpha T of every splat at
    every pixel (hard cutoff, depth order = compact order), in float64: an
    independent walk with the reference's rules (rasterize.rs:120-170)."""
    v = projected.shape[0]
    ys, xs = np.mgrid[0:img_h, 0:img_w]
    px, py = xs + 0.5, ys + 0.5
    T = np.ones((img_h, img_w))
    done = np.zeros((img_h, img_w), bool)
    wts = np.zeros((v, img_h, img_w))
    for c in range(v):
        x, y, c00, c01, c11, o = (float(t) for t in projected[c, :6])
        dx, dy = x - px, y - py
        sigma = 0.5 * (c00 * dx * dx + c11 * dy * dy) + c01 * dx * dy
        alpha = np.minimum(0.999, o * np.exp(-sigma))
        ok = (~done) & (sigma >= 0) & (alpha >= 1.0 / 255.0)
        nt = T * (1 - alpha)
        sat = ok & (nt <= 1e-4)
        con = ok & ~sat
        wts[c] = np.where(con, alpha * T, 0.0)
        T = np.where(con, nt, T)
        done |= sat
    return wts


def test_depth_lane_is_detached_from_the_blend_weights():
    """rasterize_backwards.rs:379-396: with an upstream gradient on the depth
    channel only, lanes 0-8 are exactly zero (depth does not flow into alpha,
    colour or shape) and lane 10 = sum over pixels of (alpha T) v_d, the
    blending weight from an independent float64 walk (1e-5 relative)."""
    rng = np.random.default_rng(12)
    n = 7
    tr = np.zeros((n, 10), np.float32)
    tr[:, 0:2] = rng.uniform(-0.25, 0.25, (n, 2))
    tr[:, 2] = np.linspace(-0.3, 0.3, n)
    q = rng.standard_normal((n, 4))
    tr[:, 3:7] = q / np.linalg.norm(q, axis=1, keepdims=True)
    tr[:, 7:10] = rng.uniform(-2.0, -1.5, (n, 3))
    sh = rng.uniform(0.1, 0.9, (n, 1, 3)).astype(np.float32)
    opac = rng.uniform(-0.5, 1.5, n).astype(np.float32)
    cam = Camera.from_focal((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 45.0, 40, 36)
    flags = O.FLAG_BWD_INFO | O.FLAG_RENDER_DEPTH
    fwd = O.render_forward(uniforms_for(cam, 40, 36, n, 0), tr, sh, opac, flags)
    assert fwd.num_visible == n and fwd.out_img.shape == (36, 40, 5)
    v_d = rng.standard_normal((36, 40)).astype(np.float32)
    v = np.zeros((36, 40, 5), np.float32)
    v[..., 4] = v_d
    vc = O.rasterize_backward(fwd, v, O.FLAG_RENDER_DEPTH | O.FLAG_REFINE_WEIGHT)
    assert np.all(vc[:, :9] == 0.0)
    wts = _blend_weights_f64(fwd.projected[:n], 40, 36)
    want = np.einsum("cyx,yx->c", wts, v_d.astype(np.float64))
    np.testing.assert_allclose(vc[:, 10], want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
    # the depth image itself is sum_c w_c depth_c
    np.testing.assert_allclose(fwd.out_img[..., 4], np.einsum("cyx,c->yx", wts, fwd.projected[:n, 9]),
                               rtol=2e-5, atol=1e-5)
    # adding an RGBA upstream gradient leaves the depth lane as it was and
    # gives lanes 0-8 exactly as without the depth channel
    v_rgba = rng.standard_normal((36, 40, 4)).astype(np.float32)
    v2 = v.copy()
    v2[..., :4] = v_rgba
    vc2 = O.rasterize_backward(fwd, v2, O.FLAG_RENDER_DEPTH)
    v3 = np.zeros_like(v)
    v3[..., :4] = v_rgba
    vc3 = O.rasterize_backward(fwd, v3, O.FLAG_RENDER_DEPTH)
    np.testing.assert_array_equal(vc2[:, :9], vc3[:, :9])
    np.testing.assert_allclose(vc2[:, 10], vc[:, 10], rtol=1e-6, atol=1e-9)
