"""Pinhole camera and ProjectUniforms construction.

Restates the host side of the reference's projection setup:
``Camera`` (brush-render/src/camera.rs:11-82), ``fov_to_focal`` /
``focal_to_fov`` (camera.rs:84-119, pinhole branch),
``calculate_jacobian_clamp_limits`` (camera.rs:200-254, pinhole branch),
``calc_tile_bounds`` (render.rs:30-47) and the uniform packing of
``render_with_rasterizer`` (render.rs:116-136).  Scalar arithmetic follows the
reference's types: f64 for fov/focal conversion, f32 elsewhere (numpy float32
scalars give IEEE single-precision rounding per operation).

Other camera models (Kannala-Brandt, radial-tangential, thin-prism fisheye)
are not part of this build.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

TILE_WIDTH = 16

f32 = np.float32


def fov_to_focal(fov: float, pixels: int) -> float:
    """camera.rs:84-101 (pinhole): r_pix / tan(fov / 2), in f64."""
    return (pixels / 2.0) / math.tan(fov / 2.0)


def focal_to_fov(focal: float, pixels: int) -> float:
    """camera.rs:103-119 (pinhole): 2 atan(r_pix / focal), in f64."""
    return 2.0 * math.atan((pixels / 2.0) / focal)


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

    @staticmethod
    def from_focal(position, rotation, focal: float, img_w: int, img_h: int, center_uv=(0.5, 0.5)):
        """A camera whose pinhole focal length is ``focal`` pixels on both axes."""
        return Camera(
            tuple(position),
            tuple(rotation),
            focal_to_fov(focal, img_w),
            focal_to_fov(focal, img_h),
            tuple(center_uv),
        )

    def focal(self, img_w: int, img_h: int):
        """camera.rs:49-54: f64 focal cast to f32."""
        return f32(fov_to_focal(self.fov_x, img_w)), f32(fov_to_focal(self.fov_y, img_h))

    def center(self, img_w: int, img_h: int):
        """camera.rs:56-61."""
        return f32(self.center_uv[0]) * f32(img_w), f32(self.center_uv[1]) * f32(img_h)

    def world_to_local(self):
        """camera.rs:75-81: inverse of the local-to-world rigid transform."""
        rot = quat_to_mat3(self.rotation)
        return affine_inverse(rot, np.asarray(self.position, dtype=np.float32))


def tile_bounds(img_w: int, img_h: int):
    """render.rs:30-47 for 16x16 tiles."""
    return (img_w + TILE_WIDTH - 1) // TILE_WIDTH, (img_h + TILE_WIDTH - 1) // TILE_WIDTH


def jacobian_clamp_limits(img_w: int, img_h: int, fx, fy, cx, cy):
    """camera.rs:200-254, pinhole branch, f32."""
    w, h = f32(img_w), f32(img_h)
    lim_pos_x = (f32(1.15) * w - cx) / fx
    lim_pos_y = (f32(1.15) * h - cy) / fy
    lim_neg_x = (f32(-0.15) * w - cx) / fx
    lim_neg_y = (f32(-0.15) * h - cy) / fy
    return lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y


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
    lims = jacobian_clamp_limits(img_w, img_h, fx, fy, cx, cy)
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
