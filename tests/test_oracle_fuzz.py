"""The reference's finite-difference fuzz suites, run on the CPU restatement.

crates/brush-bench-test/tests/finite_diff.rs drives random scenes, cameras
and parameter picks through the differentiable render and compares each
analytic gradient with a central difference of mean(image) (or of a
weighted sum), under the smooth alpha cutoff (RasterPass::
BackwardSmoothCutoff, :32).  Here the same generators (SplitMix64 streams
seeded as the reference seeds them, :955-982), the same scene and camera
distributions, the same parameter picks and the same tolerances drive the
restatement: its forward gives the loss (summed in float64, the quotient
divided by the step actually taken in f32), its rasterize + project backward
the analytic gradient.

Suites (finite_diff.rs line of each):
  random scenes :1003, camera models :1143, non-identity camera rotation
  :1256, off-centre principal point and asymmetric focal :1303, asymmetric
  images :1342, anisotropic scales :1396, near-camera splats :1442, depth
  extremes :1490, heavy distortion :1532, SH degree 3 :1606, kitchen sink
  :1834, weighted loss :794, the transmittance early-out :1019.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from brush_amd import camera as C
from brush_amd.camera import Camera, quat_to_mat3
from oracle import oracle as O
from tests.helpers import uniforms_for

MASK64 = (1 << 64) - 1
FLAGS = O.FLAG_BWD_INFO | O.FLAG_SMOOTH_CUTOFF
FUZZ_EPS = 3e-4  # finite_diff.rs:1210


class Sm64:
    """finite_diff.rs:955-982: SplitMix64 with f32 draws."""

    def __init__(self, seed: int):
        self.state = seed & MASK64

    def u64(self) -> int:
        self.state = (self.state + 0x9E3779B97F4A7C15) & MASK64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        return z ^ (z >> 31)

    def f01(self) -> np.float32:
        return np.float32(self.u64() / float(MASK64))

    def uniform(self, lo: float, hi: float) -> np.float32:
        lo, hi = np.float32(lo), np.float32(hi)
        return np.float32(lo + self.f01() * np.float32(hi - lo))

    def usize_in(self, lo: int, hi: int) -> int:
        return lo + self.u64() % (hi - lo)


def wmul(a: int, b: int) -> int:
    return (a * b) & MASK64


class Scene:
    """finite_diff.rs:34-46: flat arrays as the reference builds them; the
    rotations are raw (not normalised) wxyz quaternions."""

    def __init__(self, means, rots, log_scales, sh, raw_opac):
        self.means = np.asarray(means, np.float32).reshape(-1, 3)
        self.rots = np.asarray(rots, np.float32).reshape(-1, 4)
        self.log_scales = np.asarray(log_scales, np.float32).reshape(-1, 3)
        n = self.means.shape[0]
        self.sh = np.asarray(sh, np.float32).reshape(n, -1, 3)
        self.raw_opac = np.asarray(raw_opac, np.float32).reshape(n)

    @property
    def n(self) -> int:
        return self.means.shape[0]

    def arrays(self):
        tr = np.concatenate([self.means, self.rots, self.log_scales], 1).astype(np.float32)
        return tr, self.sh.copy(), self.raw_opac.copy()


def random_scene(seed: int, n: int) -> Scene:
    """finite_diff.rs:984-999."""
    rng = Sm64(wmul(seed, 0x517CC1B727220A95))
    means = [rng.uniform(-1.0, 1.0) for _ in range(n * 3)]
    rots = [rng.uniform(-1.0, 1.0) for _ in range(n * 4)]
    log_scales = [rng.uniform(-2.5, 0.0) for _ in range(n * 3)]
    sh_dc = [rng.uniform(0.2, 0.8) for _ in range(n * 3)]
    raw_opac = [rng.uniform(0.5, 3.0) for _ in range(n)]
    return Scene(means, rots, log_scales, sh_dc, raw_opac)


def random_camera(seed: int) -> Camera:
    """finite_diff.rs:1001-1016."""
    rng = Sm64(wmul(seed, 0xBF58476D1CE4E5B9) ^ 0xCAFE)
    dist = rng.uniform(2.5, 5.0)
    pos = (float(rng.uniform(-0.3, 0.3)), float(rng.uniform(-0.3, 0.3)), -float(dist))
    fov = float(rng.uniform(0.4, 0.9))
    return Camera(pos, (0.0, 0.0, 0.0, 1.0), fov, fov, (0.5, 0.5), C.PINHOLE)


LANES = ("means", "rots", "log_scales", "sh_dc", "raw_opac")


def random_param(rng: Sm64, n: int):
    """finite_diff.rs:1018-1034."""
    lane = LANES[min(rng.usize_in(0, 5), 4)]
    splat = rng.usize_in(0, n)
    comp = {"means": lambda: rng.usize_in(0, 3), "log_scales": lambda: rng.usize_in(0, 3),
            "sh_dc": lambda: rng.usize_in(0, 3), "rots": lambda: rng.usize_in(0, 4),
            "raw_opac": lambda: 0}[lane]()
    return lane, splat, comp


def random_param_no_sh(rng: Sm64, n: int):
    """finite_diff.rs:1036-1056."""
    lane = ("means", "rots", "log_scales", "raw_opac")[rng.usize_in(0, 4)]
    splat = rng.usize_in(0, n)
    comp = {"means": lambda: rng.usize_in(0, 3), "log_scales": lambda: rng.usize_in(0, 3),
            "rots": lambda: rng.usize_in(0, 4), "raw_opac": lambda: 0}[lane]()
    return lane, splat, comp


def quat_axis_angle(axis, angle) -> tuple:
    """glam Quat::from_axis_angle, (x, y, z, w); a zero axis gives identity."""
    a = np.asarray(axis, np.float64)
    nrm = float(np.linalg.norm(a))
    if nrm == 0.0:
        return (0.0, 0.0, 0.0, 1.0)
    a = a / nrm
    s, c = math.sin(float(angle) / 2.0), math.cos(float(angle) / 2.0)
    return (a[0] * s, a[1] * s, a[2] * s, c)


def rotate(q, v) -> tuple:
    return tuple(float(x) for x in quat_to_mat3(q).astype(np.float64) @ np.asarray(v, np.float64))


class Problem:
    """sum(weights * image) (weights None: mean(image), finite_diff.rs:102-131)
    of a scene through the restatement, and its analytic gradient."""

    def __init__(self, scene: Scene, cam: Camera, size, weights=None):
        self.scene, self.cam, self.size = scene, cam, size
        w, h = size
        deg = int(round(math.sqrt(scene.sh.shape[1]))) - 1
        self.u = uniforms_for(cam, w, h, scene.n, deg)
        self.weights = weights if weights is not None else np.full((h, w, 4), 1.0 / (w * h * 4), np.float64)

    def loss(self, tr, sh, opac) -> float:
        r = O.render_forward(self.u, tr, sh, opac, FLAGS)
        return float(np.sum(r.out_img.astype(np.float64) * self.weights))

    def analytic(self):
        tr, sh, opac = self.scene.arrays()
        fwd = O.render_forward(self.u, tr, sh, opac, FLAGS)
        vc = O.rasterize_backward(fwd, self.weights.astype(np.float32), O.FLAG_SMOOTH_CUTOFF)
        return O.project_backward(fwd, tr, sh, opac, vc)

    @staticmethod
    def pick(grads, lane, splat, comp) -> float:
        vt, vcoef, vo, _ = grads
        col = {"means": 0, "rots": 3, "log_scales": 7}
        if lane == "sh_dc":
            return float(vcoef[splat, 0, comp])
        if lane == "raw_opac":
            return float(vo[splat])
        return float(vt[splat, col[lane] + comp])

    def numeric(self, lane, splat, comp, eps=FUZZ_EPS) -> float:
        tr, sh, opac = self.scene.arrays()
        arr, idx = {"means": (tr, (splat, comp)), "rots": (tr, (splat, 3 + comp)),
                    "log_scales": (tr, (splat, 7 + comp)), "sh_dc": (sh, (splat, 0, comp)),
                    "raw_opac": (opac, (splat,))}[lane]
        plus, minus = arr.copy(), arr.copy()
        plus[idx] += np.float32(eps)
        minus[idx] -= np.float32(eps)
        step = float(plus[idx]) - float(minus[idx])

        def args(a):
            if arr is tr:
                return a, sh, opac
            if arr is sh:
                return tr, a, opac
            return tr, sh, a

        return (self.loss(*args(plus)) - self.loss(*args(minus))) / step


def run_fuzz(size, n_iter, scene_fn, cam_fn, param_fn=random_param):
    """finite_diff.rs:1212-1262 (run_obscure_fuzz_with): per seed one scene,
    one camera, one random parameter."""
    rows = []
    for seed in range(n_iter):
        scene, n, tag = scene_fn(seed)
        cam = cam_fn(seed)
        p = Problem(scene, cam, size)
        grads = p.analytic()
        rng = Sm64((wmul(seed, 0xA5A55A5A) + 0x1234) & MASK64)
        lane, splat, comp = param_fn(rng, n)
        rows.append((seed, tag, lane, splat, comp, p.numeric(lane, splat, comp), p.pick(grads, lane, splat, comp)))
    return rows


def assert_fuzz_clean(rows, rel_tol, abs_tol, label):
    """finite_diff.rs:1264-1291: |num - an| <= abs_tol + rel_tol max(|num|, |an|)."""
    bad = []
    worst = 0.0
    for seed, tag, lane, splat, comp, num, an in rows:
        err = abs(num - an)
        tol = abs_tol + rel_tol * max(abs(num), abs(an), 1e-8)
        worst = max(worst, err / tol)
        if err > tol:
            bad.append(f"seed {seed} {tag} {lane}[{splat},{comp}]: num {num:.6g} an {an:.6g}")
    live = sum(abs(an) > abs_tol for *_, an in rows)
    print(f"[fuzz] {label}: {len(rows)} probes ({live} with |gradient| above abs_tol), worst |err|/tol {worst:.3f}")
    assert not bad, f"[{label}] {len(bad)} mismatches:\n  " + "\n  ".join(bad)
    assert live >= len(rows) // 2, f"[{label}] most probes have no gradient to check"



# ---- the suites --------------------------------------------------------------------------------------

def test_fuzz_random_scenes():
    def scene_fn(seed):
        n = Sm64((seed + 0xDEADBEEF) & MASK64).usize_in(3, 9)
        return random_scene(seed, n), n, "rng"

    assert_fuzz_clean(run_fuzz((32, 32), 5, scene_fn, random_camera), 0.02, 2e-4, "rng")


def random_camera_with_model(seed: int):
    """finite_diff.rs:1080-1139."""
    rng = Sm64(wmul(seed, 0xBF58476D1CE4E5B9) ^ 0xC0DE)
    dist = rng.uniform(2.5, 5.0)
    pos = (float(rng.uniform(-0.2, 0.2)), float(rng.uniform(-0.2, 0.2)), -float(dist))
    fov = float(rng.uniform(0.5, 1.0))
    kind = rng.usize_in(0, 4)
    if kind == 0:
        model, label = C.PINHOLE, "Pinhole"
    elif kind == 1:
        model = C.KannalaBrandt4(k1=float(rng.uniform(-0.05, 0.05)), k2=float(rng.uniform(-0.02, 0.02)),
                                 k3=float(rng.uniform(-0.01, 0.01)), k4=float(rng.uniform(-0.005, 0.005)))
        label = "KB4"
    elif kind == 2:
        k1, k2, k3 = (float(rng.uniform(-a, a)) for a in (0.1, 0.05, 0.01))
        p1, p2 = float(rng.uniform(-0.01, 0.01)), float(rng.uniform(-0.01, 0.01))
        model, label = C.RadialTangential8(k1=k1, k2=k2, k3=k3, p1=p1, p2=p2), "RT8"
    else:
        kb = C.KannalaBrandt4(k1=float(rng.uniform(-0.05, 0.05)), k2=float(rng.uniform(-0.02, 0.02)),
                              k3=float(rng.uniform(-0.005, 0.005)), k4=float(rng.uniform(-0.001, 0.001)))
        model = C.ThinPrismFisheye(kb4=kb, p1=float(rng.uniform(-0.01, 0.01)), p2=float(rng.uniform(-0.01, 0.01)),
                                   sx1=float(rng.uniform(-0.005, 0.005)), sy1=float(rng.uniform(-0.005, 0.005)))
        label = "TPF"
    return Camera(pos, (0.0, 0.0, 0.0, 1.0), fov, fov, (0.5, 0.5), model), label


def test_fuzz_camera_models():
    def scene_fn(seed):
        n = Sm64((seed + 0xC0DEBEEF) & MASK64).usize_in(3, 9)
        return random_scene(seed, n), n, random_camera_with_model(seed)[1]

    rows = run_fuzz((32, 32), 20, scene_fn, lambda s: random_camera_with_model(s)[0])
    assert_fuzz_clean(rows, 0.02, 2e-4, "cam-models")


def test_fuzz_obscure_rotated_cameras():
    def cam_fn(seed):
        rng = Sm64(wmul(seed, 0xCAFEC0DE) ^ 0x12345678)
        axis = (rng.uniform(-1.0, 1.0), rng.uniform(-1.0, 1.0), rng.uniform(-1.0, 1.0))
        rot = quat_axis_angle(axis, rng.uniform(-1.0, 1.0))
        fov = float(rng.uniform(0.5, 0.9))
        return Camera(rotate(rot, (0.0, 0.0, -4.0)), rot, fov, fov, (0.5, 0.5), C.PINHOLE)

    def scene_fn(seed):
        n = Sm64((seed + 0xCAFE) & MASK64).usize_in(3, 8)
        return random_scene(seed, n), n, "rot"

    # the rotation is not the identity in every camera
    assert sum(abs(cam_fn(s).rotation[3]) < 0.999 for s in range(20)) > 10
    assert_fuzz_clean(run_fuzz((32, 32), 20, scene_fn, cam_fn), 0.03, 5e-4, "rot-cam")


def test_fuzz_obscure_off_center_principal_and_asymmetric_focal():
    def cam_fn(seed):
        rng = Sm64(wmul(seed, 0xBEEFFEED))
        dist = rng.uniform(3.0, 5.0)
        cx, cy = float(rng.uniform(0.2, 0.8)), float(rng.uniform(0.2, 0.8))
        fx, fy = float(rng.uniform(0.4, 1.0)), float(rng.uniform(0.4, 1.0))
        return Camera((0.0, 0.0, -float(dist)), (0.0, 0.0, 0.0, 1.0), fx, fy, (cx, cy), C.PINHOLE)

    def scene_fn(seed):
        n = Sm64((seed + 0xFEEB) & MASK64).usize_in(3, 8)
        return random_scene(seed, n), n, "offc"

    assert_fuzz_clean(run_fuzz((48, 48), 20, scene_fn, cam_fn), 0.03, 5e-4, "off-center")


def test_fuzz_obscure_asymmetric_images():
    rows = []
    for w, h in ((15, 47), (63, 16), (17, 17), (81, 33), (128, 64), (32, 95)):
        def scene_fn(seed, w=w, h=h):
            n = Sm64((seed + 0xC0DEF00D) & MASK64).usize_in(3, 7)
            return random_scene(seed, n), n, f"{w}x{h}"

        def cam_fn(seed, w=w, h=h):
            fov = float(Sm64(wmul(seed, 0xABCD)).uniform(0.5, 0.9))
            return Camera((0.0, 0.0, -3.5), (0.0, 0.0, 0.0, 1.0), fov, fov * h / w, (0.5, 0.5), C.PINHOLE)

        rows += run_fuzz((w, h), 5, scene_fn, cam_fn)
    assert_fuzz_clean(rows, 0.03, 5e-4, "asym-img")


def test_fuzz_obscure_anisotropic_scales():
    def scene_fn(seed):
        rng = Sm64(wmul(seed, 0xDEADF00D))
        n = rng.usize_in(3, 8)
        scene = random_scene(seed, n)
        for i in range(n):
            big, a, b = rng.uniform(-0.5, 0.5), rng.uniform(-3.5, -2.5), rng.uniform(-3.5, -2.5)
            scene.log_scales[i] = ((big, a, b), (a, big, b), (a, b, big))[i % 3]
        return scene, n, "aniso"

    assert_fuzz_clean(run_fuzz((48, 48), 20, scene_fn, random_camera), 0.03, 5e-4, "aniso")


def test_fuzz_obscure_near_camera_splats():
    def scene_fn(seed):
        rng = Sm64(wmul(seed, 0xCAB005E0))
        n = rng.usize_in(3, 7)
        scene = random_scene(seed, n)
        for i in range(n):
            z = np.float32(np.float32(0.1) + rng.uniform(0.0, 0.9))
            x = np.float32(rng.uniform(-0.3, 0.3) * z)
            y = np.float32(rng.uniform(-0.3, 0.3) * z)
            scene.means[i] = (x, y, np.float32(z - np.float32(3.0)))
        scene.log_scales -= np.float32(2.5)
        return scene, n, random_camera_with_model(seed)[1]

    def cam_fn(seed):
        model = random_camera_with_model(seed)[0].camera_model
        return Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.8, 0.8, (0.5, 0.5), model)

    assert_fuzz_clean(run_fuzz((48, 48), 20, scene_fn, cam_fn), 0.03, 5e-4, "near-cam")


def test_fuzz_obscure_depth_extremes():
    def scene_fn(seed):
        rng = Sm64(wmul(seed, 0xC001D00D))
        n = rng.usize_in(4, 9)
        scene = random_scene(seed, n)
        for i in range(n):
            x, y = rng.uniform(-0.4, 0.4), rng.uniform(-0.4, 0.4)
            t = np.float32(i / max(n - 1, 1))
            z = np.float32(np.float32(-2.5) + t * np.float32(29.5) + rng.uniform(-0.3, 0.3))
            scene.means[i] = (x, y, z)
        return scene, n, "depth"

    cam = Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.7, 0.7, (0.5, 0.5), C.PINHOLE)
    assert_fuzz_clean(run_fuzz((48, 48), 15, scene_fn, lambda s: cam), 0.03, 5e-4, "depth-ext")


def test_fuzz_obscure_heavy_distortion():
    def cam_fn(seed):
        rng = Sm64(wmul(seed, 0xF15EBEEF))
        dist = rng.uniform(3.0, 5.0)
        fov = float(rng.uniform(0.5, 0.9))
        u = lambda a: float(rng.uniform(-a, a))  # noqa: E731
        if seed % 3 == 0:
            model = C.KannalaBrandt4(k1=u(0.3), k2=u(0.15), k3=u(0.05), k4=u(0.02))
        elif seed % 3 == 1:
            k1, k2, k3, k4, k5 = u(0.4), u(0.2), u(0.05), u(0.01), u(0.005)
            model = C.RadialTangential8(k1=k1, k2=k2, k3=k3, k4=k4, k5=k5, p1=u(0.05), p2=u(0.05))
        else:
            kb = C.KannalaBrandt4(k1=u(0.2), k2=u(0.1), k3=u(0.02), k4=u(0.005))
            model = C.ThinPrismFisheye(kb4=kb, p1=u(0.03), p2=u(0.03), sx1=u(0.02), sy1=u(0.02))
        return Camera((0.0, 0.0, -float(dist)), (0.0, 0.0, 0.0, 1.0), fov, fov, (0.5, 0.5), model)

    def scene_fn(seed):
        rng = Sm64(wmul(seed, 0xB1B1))
        n = rng.usize_in(3, 8)
        scene = random_scene(seed, n)
        for i in range(n):
            scene.means[i] = (rng.uniform(-0.5, 0.5), rng.uniform(-0.5, 0.5), rng.uniform(-0.5, 0.5))
        return scene, n, "KB4" if seed % 2 == 0 else "RT8"

    assert_fuzz_clean(run_fuzz((48, 48), 20, scene_fn, cam_fn), 0.03, 5e-4, "heavy-dist")


def test_fuzz_obscure_sh_degree3():
    def scene_fn(seed):
        rng = Sm64(wmul(seed, 0x5417BABE))
        n = rng.usize_in(3, 7)
        base = random_scene(seed, n)
        sh = np.zeros((n, 16, 3), np.float32)
        for s in range(n):
            sh[s, 0] = base.sh[s, 0]
            for k in range(1, 16):
                for ch in range(3):
                    sh[s, k, ch] = rng.uniform(-0.1, 0.1)
        return Scene(base.means, base.rots, base.log_scales, sh, base.raw_opac), n, "sh3"

    rows = run_fuzz((32, 32), 25, scene_fn, random_camera, random_param_no_sh)
    assert_fuzz_clean(rows, 0.03, 5e-4, "sh3")


def test_fuzz_obscure_kitchen_sink():
    rows = []
    for idx, size in enumerate(((32, 32), (48, 33), (17, 65))):
        def scene_fn(seed, idx=idx):
            rng = Sm64(wmul(seed, 0xC11ABAD0))
            n = rng.usize_in(3, 8)
            scene = random_scene(seed, n)
            for i in range(n):
                big, small = rng.uniform(-1.0, 0.0), rng.uniform(-2.5, -1.5)
                scene.log_scales[i] = [big if c == i % 3 else small for c in range(3)]
            return scene, n, f"img{idx}"

        def cam_fn(seed):
            rng = Sm64(wmul(seed, 0x9999AAAA) ^ 0x55)
            axis = (rng.uniform(-1.0, 1.0), rng.uniform(-1.0, 1.0), rng.uniform(-1.0, 1.0))
            rot = quat_axis_angle(axis, rng.uniform(-0.6, 0.6))
            dist = rng.uniform(3.0, 5.0)
            fx, fy = float(rng.uniform(0.5, 0.9)), float(rng.uniform(0.5, 0.9))
            cx, cy = float(rng.uniform(0.3, 0.7)), float(rng.uniform(0.3, 0.7))
            u = lambda a: float(rng.uniform(-a, a))  # noqa: E731
            kind = seed % 4
            if kind == 0:
                model = C.PINHOLE
            elif kind == 1:
                model = C.KannalaBrandt4(k1=u(0.05), k2=u(0.02), k3=u(0.005), k4=u(0.001))
            elif kind == 2:
                k1, k2 = u(0.1), u(0.03)
                model = C.RadialTangential8(k1=k1, k2=k2, p1=u(0.01), p2=u(0.01))
            else:
                kb = C.KannalaBrandt4(k1=u(0.05), k2=u(0.02), k3=u(0.005), k4=u(0.001))
                model = C.ThinPrismFisheye(kb4=kb, p1=u(0.01), p2=u(0.01), sx1=u(0.005), sy1=u(0.005))
            return Camera(rotate(rot, (0.0, 0.0, -float(dist))), rot, fx, fy, (cx, cy), model)

        rows += run_fuzz(size, 10, scene_fn, cam_fn)
    assert_fuzz_clean(rows, 0.03, 5e-4, "kitchen-sink")


def _base_scene() -> Scene:
    """finite_diff.rs:48-77."""
    from tests.test_oracle_backward import _reference_base_scene

    tr, sh, opac = _reference_base_scene()
    return Scene(tr[:, 0:3], tr[:, 3:7], tr[:, 7:10], sh, opac)


def test_finite_diff_weighted_loss():
    """finite_diff.rs:794-904: sum(W * image) with a fixed [0, 1) weight map
    from a 64-bit LCG, so per-pixel asymmetries of the backward show;
    tolerance 0.5 + 2 % (sum losses are O(100))."""
    w, h = 32, 32
    state = 0xCAFEF00D
    vals = np.empty(h * w * 4, np.float64)
    for i in range(vals.size):
        state = (state * 6364136223846793005 + 1442695040888963407) & MASK64
        vals[i] = np.float32(np.float32((state >> 33) & 0xFFFFFFFF) / np.float32(4294967295.0))
    weights = vals.reshape(h, w, 4)
    p = Problem(_base_scene(), Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.6, 0.6), (w, h), weights)
    grads = p.analytic()
    rows = []
    for lane, splat, comp in (("means", 0, 0), ("means", 1, 1), ("log_scales", 0, 0), ("sh_dc", 1, 1),
                              ("raw_opac", 0, 0), ("raw_opac", 2, 0)):
        rows.append((0, "weighted", lane, splat, comp, p.numeric(lane, splat, comp), p.pick(grads, lane, splat, comp)))
    assert_fuzz_clean(rows, 0.02, 0.5, "weighted")
    # the weighting matters: the same probes under mean(image) differ
    plain = Problem(_base_scene(), p.cam, (w, h))
    g2 = plain.analytic()
    assert any(abs(Problem.pick(g2, *r[2:5]) * (w * h * 4) * 0.5 - r[6]) > 1e-3 * abs(r[6]) for r in rows)


def test_finite_diff_t_early_out_back_splats():
    """finite_diff.rs:1019-1074: 30 opaque splats stacked in depth; the ones
    behind the transmittance early-out get zero gradient, and every probe
    agrees with its central difference to 5e-4."""
    n = 30
    means = [[0.0, 0.0, i * 0.3] for i in range(n)]
    rots = [[1.0, 0.0, 0.0, 0.0]] * n
    log_scales = [[-0.3, -0.3, -0.3]] * n
    sh = [[0.3 + 0.4 * (i / n)] * 3 for i in range(n)]
    scene = Scene(means, rots, log_scales, sh, [4.0] * n)
    p = Problem(scene, Camera((0.0, 0.0, -3.0), (0.0, 0.0, 0.0, 1.0), 0.6, 0.6), (32, 32))
    grads = p.analytic()
    for s in (1, 5, 10, 15, 20, 25, 29):
        num = p.numeric("raw_opac", s, 0, eps=1e-3)
        an = Problem.pick(grads, "raw_opac", s, 0)
        assert abs(num - an) < 5e-4, (s, num, an)
    # behind the early-out the far splats only blend where the stack is thin
    # (its edges): their gradients are orders of magnitude below the front's
    front = abs(Problem.pick(grads, "raw_opac", 1, 0))
    assert abs(Problem.pick(grads, "raw_opac", 29, 0)) < 1e-4 * front
