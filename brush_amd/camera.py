"""Camera, camera models and ProjectUniforms construction.

Restates the host side of the reference's projection setup:
``Camera`` (brush-render/src/camera.rs:11-82), ``fov_to_focal`` /
``focal_to_fov`` (camera.rs:84-195, every model),
``calculate_jacobian_clamp_limits`` (camera.rs:197-254),
``calc_tile_bounds`` (render.rs:30-47) and the uniform packing of
``render_with_rasterizer`` (render.rs:116-136).  The camera models
(kernels/camera_model/mod.rs:34-41) are ``Pinhole``, ``KannalaBrandt4``,
``RadialTangential8`` and ``ThinPrismFisheye``; the kernels receive the model
id and its coefficients through the uniforms.  Scalar arithmetic follows the
reference's types: f64 for fov/focal conversion and the distortion inverses,
f32 elsewhere (numpy float32 scalars give IEEE single-precision rounding per
operation).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

TILE_WIDTH = 16

f32 = np.float32


@dataclass(frozen=True)
class Pinhole:
    """camera_model/pinhole.rs."""

    model_id = 0

    def params(self):
        return [0.0] * 8


@dataclass(frozen=True)
class KannalaBrandt4:
    """camera_model/kannala_brandt_4.rs:11-16: d(theta) = theta (1 + k1 theta^2 + ... + k4 theta^8)."""

    k1: float = 0.0
    k2: float = 0.0
    k3: float = 0.0
    k4: float = 0.0
    model_id = 1

    def params(self):
        return [self.k1, self.k2, self.k3, self.k4, 0.0, 0.0, 0.0, 0.0]


@dataclass(frozen=True)
class RadialTangential8:
    """camera_model/radial_tangential_8.rs:12-21: rational radial (k1..k3 over
    k4..k6) plus tangential p1, p2."""

    k1: float = 0.0
    k2: float = 0.0
    k3: float = 0.0
    k4: float = 0.0
    k5: float = 0.0
    k6: float = 0.0
    p1: float = 0.0
    p2: float = 0.0
    model_id = 2

    def params(self):
        return [self.k1, self.k2, self.k3, self.k4, self.k5, self.k6, self.p1, self.p2]


@dataclass(frozen=True)
class ThinPrismFisheye:
    """camera_model/thin_prism_fisheye.rs:23-30: KB4 plus tangential (p1, p2)
    and thin prism (sx1, sy1)."""

    kb4: KannalaBrandt4 = KannalaBrandt4()
    p1: float = 0.0
    p2: float = 0.0
    sx1: float = 0.0
    sy1: float = 0.0
    model_id = 3

    def params(self):
        k = self.kb4
        return [k.k1, k.k2, k.k3, k.k4, self.p1, self.p2, self.sx1, self.sy1]


PINHOLE = Pinhole()


def _f32_coeffs(model):
    """The model's coefficients as the f32 values the reference stores, in f64."""
    return [float(f32(v)) for v in model.params()]


def kb4_d(theta: float, model) -> float:
    """camera.rs:121-130: theta + k1 theta^3 + k2 theta^5 + k3 theta^7 + k4 theta^9 (f64)."""
    k1, k2, k3, k4 = _f32_coeffs(model)[:4]
    t2 = theta * theta
    t3 = t2 * theta
    t5 = t3 * t2
    t7 = t5 * t2
    t9 = t7 * t2
    return theta + k1 * t3 + k2 * t5 + k3 * t7 + k4 * t9


def kb4_dd_dtheta(theta: float, model) -> float:
    """camera.rs:132-143."""
    k1, k2, k3, k4 = _f32_coeffs(model)[:4]
    t2 = theta * theta
    t4 = t2 * t2
    t6 = t4 * t2
    t8 = t6 * t2
    return 1.0 + 3.0 * k1 * t2 + 5.0 * k2 * t4 + 7.0 * k3 * t6 + 9.0 * k4 * t8


def kb4_invert_d(target: float, model) -> float:
    """camera.rs:145-168: Newton on d(theta) = target over [0, pi]."""
    if target <= 0.0:
        return 0.0
    theta = min(target, math.pi - 1e-6)
    for _ in range(50):
        fv = kb4_d(theta, model) - target
        fp = kb4_dd_dtheta(theta, model)
        if abs(fp) < 1e-12:
            break
        nxt = min(max(theta - fv / fp, 0.0), math.pi)
        if abs(nxt - theta) < 1e-12:
            theta = nxt
            break
        theta = nxt
    return theta


def rt8_radial(r: float, model: RadialTangential8) -> float:
    """camera.rs:170-179: (1 + k1 r^2 + k2 r^4 + k3 r^6) / (1 + k4 r^2 + k5 r^4 + k6 r^6)."""
    k1, k2, k3, k4, k5, k6 = _f32_coeffs(model)[:6]
    r2 = r * r
    r4 = r2 * r2
    r6 = r4 * r2
    return (1.0 + k1 * r2 + k2 * r4 + k3 * r6) / (1.0 + k4 * r2 + k5 * r4 + k6 * r6)


def rt8_undistort_radius(r_d: float, model: RadialTangential8) -> float:
    """camera.rs:181-195: fixed point r = r_d / radial(r)."""
    r = r_d
    for _ in range(30):
        factor = rt8_radial(r, model)
        if abs(factor) < 1e-12:
            break
        r_new = r_d / factor
        if abs(r_new - r) < 1e-12:
            r = r_new
            break
        r = r_new
    return r


def fov_to_focal(fov: float, pixels: int, model=PINHOLE) -> float:
    """camera.rs:84-101: r_pix / projection(fov / 2), in f64."""
    half = fov / 2.0
    r_pix = pixels / 2.0
    if isinstance(model, KannalaBrandt4):
        proj = kb4_d(half, model)
    elif isinstance(model, ThinPrismFisheye):
        proj = kb4_d(half, model.kb4)
    elif isinstance(model, RadialTangential8):
        r = math.tan(half)
        proj = r * rt8_radial(r, model)
    else:
        proj = math.tan(half)
    return r_pix / proj


def focal_to_fov(focal: float, pixels: int, model=PINHOLE) -> float:
    """camera.rs:103-119, in f64."""
    r_norm = (pixels / 2.0) / focal
    if isinstance(model, KannalaBrandt4):
        half = kb4_invert_d(r_norm, model)
    elif isinstance(model, ThinPrismFisheye):
        half = kb4_invert_d(r_norm, model.kb4)
    elif isinstance(model, RadialTangential8):
        half = math.atan(rt8_undistort_radius(r_norm, model))
    else:
        half = math.atan(r_norm)
    return 2.0 * half


def quat_to_mat3(q_xyzw) -> np.ndarray:
    """Rotation matrix of a unit quaternion (glam ``Mat3::from_quat``), f32.

    Returns a row-major 3x3 array M with M @ v the rotated vector.
    """
    x, y, z, w = (f32(c) for c in q_xyzw)
    x2, y2, z2 = x + x, y + y, z + z
    xx, xy, xz = x * x2, x * y2, x * z2
    yy, yz, zz = y * y2, y * z2, z * z2
    wx, wy, wz = w * x2, w * y2, w * z2
    one = f32(1.0)
    cols = [
        [one - (yy + zz), xy + wz, xz - wy],
        [xy - wz, one - (xx + zz), yz + wx],
        [xz + wy, yz - wx, one - (xx + yy)],
    ]
    return np.array(cols, dtype=np.float32).T


def _cross(a, b):
    return np.array(
        [a[1] * b[2] - b[1] * a[2], a[2] * b[0] - b[2] * a[0], a[0] * b[1] - b[0] * a[1]],
        dtype=np.float32,
    )


def affine_inverse(rot: np.ndarray, trans: np.ndarray):
    """Inverse of the affine map v -> rot @ v + trans (glam ``Affine3A::inverse``:
    cofactor inverse of the 3x3 part, translation -(inv @ trans)), in f32."""
    x_axis, y_axis, z_axis = rot[:, 0], rot[:, 1], rot[:, 2]
    tmp0 = _cross(y_axis, z_axis)
    tmp1 = _cross(z_axis, x_axis)
    tmp2 = _cross(x_axis, y_axis)
    det = f32(z_axis[0] * tmp2[0] + z_axis[1] * tmp2[1] + z_axis[2] * tmp2[2])
    inv_det = f32(1.0) / det
    inv = np.stack([tmp0 * inv_det, tmp1 * inv_det, tmp2 * inv_det], axis=1).T.astype(np.float32)
    t = -(inv[:, 0] * trans[0] + inv[:, 1] * trans[1] + inv[:, 2] * trans[2])
    return inv, t.astype(np.float32)


@dataclass
class Camera:
    """camera.rs:11-19.  ``rotation`` is a quaternion in (x, y, z, w) order like
    glam; the camera looks down its local +z axis."""

    position: tuple = (0.0, 0.0, 0.0)
    rotation: tuple = (0.0, 0.0, 0.0, 1.0)
    fov_x: float = 0.5
    fov_y: float = 0.5
    center_uv: tuple = (0.5, 0.5)
    camera_model: object = PINHOLE

    @staticmethod
    def from_focal(position, rotation, focal: float, img_w: int, img_h: int, center_uv=(0.5, 0.5),
                   camera_model=PINHOLE):
        """A camera whose focal length is ``focal`` pixels on both axes."""
        return Camera(
            tuple(position),
            tuple(rotation),
            focal_to_fov(focal, img_w, camera_model),
            focal_to_fov(focal, img_h, camera_model),
            tuple(center_uv),
            camera_model,
        )

    def focal(self, img_w: int, img_h: int):
        """camera.rs:49-54: f64 focal cast to f32."""
        return (f32(fov_to_focal(self.fov_x, img_w, self.camera_model)),
                f32(fov_to_focal(self.fov_y, img_h, self.camera_model)))

    def center(self, img_w: int, img_h: int):
        """camera.rs:56-61."""
        return f32(self.center_uv[0]) * f32(img_w), f32(self.center_uv[1]) * f32(img_h)

    def world_to_local(self):
        """camera.rs:75-81: inverse of the local-to-world rigid transform."""
        rot = quat_to_mat3(self.rotation)
        return affine_inverse(rot, np.asarray(self.position, dtype=np.float32))


def tile_bounds(img_w: int, img_h: int, tile_h: int = TILE_WIDTH):
    """render.rs:30-47 (calc_tile_bounds_for_dims) for 16 x tile_h tiles."""
    return (img_w + TILE_WIDTH - 1) // TILE_WIDTH, (img_h + tile_h - 1) // tile_h


def jacobian_clamp_limits(img_w: int, img_h: int, fx, fy, cx, cy, model=PINHOLE):
    """camera.rs:197-254, f32: the pinhole margins (1.15 W - c) / f and
    (-0.15 W - c) / f; for RT8 each edge is undistorted (in f64) to the bound
    on the undistorted coordinate; the fisheye models are not clamped (zeros)."""
    if isinstance(model, (KannalaBrandt4, ThinPrismFisheye)):
        z = f32(0.0)
        return z, z, z, z
    w, h = f32(img_w), f32(img_h)
    edges = ((f32(1.15) * w - cx) / fx, (f32(1.15) * h - cy) / fy,
             (f32(-0.15) * w - cx) / fx, (f32(-0.15) * h - cy) / fy)
    if isinstance(model, RadialTangential8):
        def undistort(edge):
            mag = f32(rt8_undistort_radius(abs(float(edge)), model))
            return mag * (f32(1.0) if edge >= 0 else f32(-1.0))
        edges = tuple(undistort(e) for e in edges)
    return edges


def project_uniforms(camera: Camera, img_w: int, img_h: int, total_splats: int, sh_degree: int) -> dict:
    """The ProjectUniforms of render.rs:116-136 as a dict of numpy scalars.

    ``viewmat`` holds the top three rows of the world-to-camera matrix,
    column-major (12 floats: three rotation columns, then translation).
    """
    if img_w <= 0 or img_h <= 0:
        raise ValueError("Can't render images with 0 size.")
    fx, fy = camera.focal(img_w, img_h)
    cx, cy = camera.center(img_w, img_h)
    rot, trans = camera.world_to_local()
    viewmat = np.concatenate([rot[:, 0], rot[:, 1], rot[:, 2], trans]).astype(np.float32)
    hyp = f32(math.hypot(float(f32(camera.fov_x)), float(f32(camera.fov_y))))
    half_fov = min(hyp * f32(1.05), f32(2.0 * math.pi - 1e-6)) * f32(0.5)
    lims = jacobian_clamp_limits(img_w, img_h, fx, fy, cx, cy, camera.camera_model)
    tbw, tbh = tile_bounds(img_w, img_h)
    return dict(
        viewmat=viewmat,
        half_max_render_fov=f32(half_fov),
        fx=fx, fy=fy, cx=cx, cy=cy,
        lim_pos_x=lims[0], lim_pos_y=lims[1], lim_neg_x=lims[2], lim_neg_y=lims[3],
        camera_pos=np.asarray(camera.position, dtype=np.float32),
        img_w=int(img_w), img_h=int(img_h),
        tile_bw=int(tbw), tile_bh=int(tbh),
        sh_degree=int(sh_degree),
        total_splats=int(total_splats),
        num_visible=0,
        camera_model=int(camera.camera_model.model_id),
        camera_params=[float(f32(v)) for v in camera.camera_model.params()],
    )


def look_at_rotation(eye, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0)):
    """Quaternion (x, y, z, w) of a camera at ``eye`` whose local +z axis points
    at ``target`` (local +y roughly along ``up``), computed in float64."""
    eye = np.asarray(eye, dtype=np.float64)
    fwd = np.asarray(target, dtype=np.float64) - eye
    fwd /= np.linalg.norm(fwd)
    right = np.cross(np.asarray(up, dtype=np.float64), fwd)
    if np.linalg.norm(right) < 1e-9:
        right = np.cross(np.array([1.0, 0.0, 0.0]), fwd)
    right /= np.linalg.norm(right)
    down = np.cross(fwd, right)
    m = np.stack([right, down, fwd], axis=1)  # columns: local x, y, z in world
    tr = m[0, 0] + m[1, 1] + m[2, 2]
    if tr > 0:
        s = math.sqrt(tr + 1.0) * 2
        w = 0.25 * s
        x = (m[2, 1] - m[1, 2]) / s
        y = (m[0, 2] - m[2, 0]) / s
        z = (m[1, 0] - m[0, 1]) / s
    elif m[0, 0] > m[1, 1] and m[0, 0] > m[2, 2]:
        s = math.sqrt(1.0 + m[0, 0] - m[1, 1] - m[2, 2]) * 2
        w = (m[2, 1] - m[1, 2]) / s
        x = 0.25 * s
        y = (m[0, 1] + m[1, 0]) / s
        z = (m[0, 2] + m[2, 0]) / s
    elif m[1, 1] > m[2, 2]:
        s = math.sqrt(1.0 + m[1, 1] - m[0, 0] - m[2, 2]) * 2
        w = (m[0, 2] - m[2, 0]) / s
        x = (m[0, 1] + m[1, 0]) / s
        y = 0.25 * s
        z = (m[1, 2] + m[2, 1]) / s
    else:
        s = math.sqrt(1.0 + m[2, 2] - m[0, 0] - m[1, 1]) * 2
        w = (m[1, 0] - m[0, 1]) / s
        x = (m[0, 2] + m[2, 0]) / s
        y = (m[1, 2] + m[2, 1]) / s
        z = 0.25 * s
    q = np.array([x, y, z, w])
    return tuple(float(c) for c in q / np.linalg.norm(q))
