"""Seeded synthetic workloads for the benchmark configurations.

Generator contract (stable across releases, so fixtures stay valid):

* PRNG: SplitMix64, the generator of the reference's own tests
  (brush-render/src/tests/mod.rs:197-207, brush-bench-test/tests/fuzz.rs:33-58).
  Draw ``k`` (0-based) of a stream with seed ``s`` is
  ``mix(s + (k + 1) * 0x9E3779B97F4A7C15)``, so any draw can be computed
  directly and generation vectorises.
* Uniform in [0, 1): ``(u64 >> 40) * 2^-24``.  Box-Muller normals use two
  draws: ``u1 = ((a >> 40) + 1) * 2^-24`` in (0, 1], ``u2`` uniform,
  ``z = sqrt(-2 ln u1) cos(2 pi u2)`` in float64, then ``mu + sigma z`` cast to
  float32.
* Per-splat draw order: mean xyz, log-scale xyz, quaternion wxyz, opacity
  logit, then SH coefficients (coefficient-major, rgb inner).  Splat ``i`` owns
  draws ``[i * S, (i + 1) * S)`` with ``S = 3 + 2 * (3 + 4 + 1 + 3 C)``.
* Configuration ``k`` uses seed ``0xB5C00000 + k``; the upstream image
  gradient uses seed ``+ 1000``; the clustered configuration draws its 64
  centres from seed ``+ 2000``.
* Camera: identity rotation at (0, 0, -d) looking down +z at the origin,
  ``cx = W / 2``, ``cy = H / 2``, background (0, 0, 0).
"""
from __future__ import annotations

import math
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np

from .camera import Camera, look_at_rotation

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
BASE_SEED = 0xB5C00000


def splitmix64(seed: int, idx: np.ndarray) -> np.ndarray:
    """Draws ``idx`` (uint64 array of 0-based draw indices) of stream ``seed``."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (idx.astype(np.uint64) + np.uint64(1)) * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def _uniform(z: np.ndarray) -> np.ndarray:
    return (z >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)


def _normal(za: np.ndarray, zb: np.ndarray) -> np.ndarray:
    u1 = ((za >> np.uint64(40)).astype(np.float64) + 1.0) * (1.0 / 16777216.0)
    u2 = _uniform(zb)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * math.pi * u2)


@dataclass
class Workload:
    name: str
    n: int
    sh_degree: int
    img_w: int
    img_h: int
    focal: float
    distance: float
    mean_lo: float = -1.0
    mean_hi: float = 1.0
    log_scale_mu: float = -4.0
    log_scale_sigma: float = 0.5
    opac_mu: float = 0.0
    opac_sigma: float = 1.0
    dc_sigma: float = 0.5
    rest_sigma: float = 0.05
    clusters: int = 0
    cluster_sigma: float = 0.15
    forward_only: bool = False
    seed: int = BASE_SEED

    @property
    def num_coeffs(self) -> int:
        return (self.sh_degree + 1) ** 2

    @property
    def pixels(self) -> int:
        return self.img_w * self.img_h

    def camera(self, pose: int = 0, num_poses: int = 1) -> Camera:
        if num_poses <= 1:
            return Camera.from_focal((0.0, 0.0, -self.distance), (0.0, 0.0, 0.0, 1.0), self.focal,
                                     self.img_w, self.img_h)
        # golden-angle spiral of poses on a sphere of radius `distance`
        i = pose + 0.5
        y = 1.0 - 2.0 * i / num_poses
        r = math.sqrt(max(0.0, 1.0 - y * y))
        phi = i * math.pi * (3.0 - math.sqrt(5.0))
        eye = (self.distance * r * math.cos(phi), self.distance * y, self.distance * r * math.sin(phi))
        return Camera.from_focal(eye, look_at_rotation(eye), self.focal, self.img_w, self.img_h)


CONFIGS = {
    0: Workload("cfg0_100k_sh0_256", 100_000, 0, 256, 256, 300.0, 3.0, seed=BASE_SEED + 0),
    1: Workload("cfg1_1M_sh3_1080p", 1_000_000, 3, 1920, 1080, 1100.0, 4.0, seed=BASE_SEED + 1),
    2: Workload("cfg2_3M_clustered_sh3_720p", 3_000_000, 3, 1280, 720, 1100.0 * 1280 / 1920, 4.0,
                log_scale_mu=-3.0, log_scale_sigma=0.7, opac_mu=1.0, clusters=64,
                seed=BASE_SEED + 2),
    3: Workload("cfg3_6M_sh3_4k_fwd", 6_000_000, 3, 3840, 2160, 2200.0, 4.0, forward_only=True,
                seed=BASE_SEED + 3),
    4: Workload("cfg4_1M_sh3_1600x1064_train", 1_000_000, 3, 1600, 1064, 1100.0 * 1600 / 1920,
                4.0, seed=BASE_SEED + 4),
}


def generate_splats(w: Workload, n: int | None = None, chunk: int = 1 << 16):
    """Returns (transforms f32[N,10], sh_coeffs f32[N,C,3], raw_opacities f32[N])."""
    n = w.n if n is None else n
    c = w.num_coeffs
    per = 3 + 2 * (3 + 4 + 1 + 3 * c)
    transforms = np.empty((n, 10), dtype=np.float32)
    sh = np.empty((n, c, 3), dtype=np.float32)
    opac = np.empty((n,), dtype=np.float32)
    centres = None
    if w.clusters:
        zc = splitmix64(w.seed + 2000, np.arange(w.clusters * 3, dtype=np.uint64))
        centres = (w.mean_lo + _uniform(zc) * (w.mean_hi - w.mean_lo)).reshape(w.clusters, 3)
    sh_sigma = np.full((c, 3), w.rest_sigma)
    sh_sigma[0, :] = w.dc_sigma
    sh_sigma = sh_sigma.reshape(-1)
    def fill(s):
        e = min(n, s + chunk)
        m = e - s
        idx = (np.arange(s, e, dtype=np.uint64) * np.uint64(per))[:, None] + np.arange(per, dtype=np.uint64)[None, :]
        z = splitmix64(w.seed, idx)
        u = _uniform(z[:, 0:3])
        nrm = _normal(z[:, 3::2], z[:, 4::2])  # (m, 3 + 4 + 1 + 3c)
        if centres is not None:
            k = np.minimum((u[:, 0] * w.clusters).astype(np.int64), w.clusters - 1)
            # offsets reuse the two remaining mean uniforms and the first
            # log-scale normal draw pair as a second stream of normals
            zo = splitmix64(w.seed + 3000, idx[:, :6])
            off = _normal(zo[:, 0::2], zo[:, 1::2]) * w.cluster_sigma
            means = centres[k] + off
        else:
            means = w.mean_lo + u * (w.mean_hi - w.mean_lo)
        transforms[s:e, 0:3] = means
        log_scales = w.log_scale_mu + w.log_scale_sigma * nrm[:, 0:3]
        quat = nrm[:, 3:7]
        quat = quat / np.linalg.norm(quat, axis=1, keepdims=True)
        transforms[s:e, 3:7] = quat
        transforms[s:e, 7:10] = log_scales
        opac[s:e] = w.opac_mu + w.opac_sigma * nrm[:, 7]
        sh[s:e] = (nrm[:, 8:] * sh_sigma[None, :]).reshape(m, c, 3)

    # every chunk depends only on its own indices: fill them on a thread pool
    # (numpy releases the GIL in these array operations)
    starts = list(range(0, n, chunk))
    workers = max(1, min(len(starts), os.cpu_count() or 1, 16))
    if workers == 1:
        for s in starts:
            fill(s)
    else:
        with ThreadPoolExecutor(max_workers=workers) as pool:
            list(pool.map(fill, starts))
    return transforms, sh, opac


def generate_v_output(w: Workload, channels: int = 4) -> np.ndarray:
    """Upstream dL/d(out_img) ~ N(0, 1), f32[H, W, channels], seed + 1000."""
    count = w.img_h * w.img_w * channels
    idx = np.arange(2 * count, dtype=np.uint64)
    z = splitmix64(w.seed + 1000, idx)
    return _normal(z[0::2], z[1::2]).astype(np.float32).reshape(w.img_h, w.img_w, channels)


def generate_target(w: Workload, block: int = 8) -> np.ndarray:
    """The training target of config 4: RGB uniform in [0, 1], constant over
    block x block pixel squares, drawn with SplitMix64 from seed + 2000 (one
    draw per block and channel, row-major over blocks), quantised like a
    decoded 8-bit image (round(x * 255)) and packed RGBA8 with alpha 255
    (r in the low byte).  Returns uint32 [H, W]."""
    bh, bw = (w.img_h + block - 1) // block, (w.img_w + block - 1) // block
    z = splitmix64(w.seed + 2000, np.arange(bh * bw * 3, dtype=np.uint64))
    rgb = _uniform(z).reshape(bh, bw, 3)
    q = np.round(rgb * 255.0).astype(np.uint32)
    q = np.repeat(np.repeat(q, block, axis=0), block, axis=1)[: w.img_h, : w.img_w]
    return (q[..., 0] | (q[..., 1] << 8) | (q[..., 2] << 16) | np.uint32(255 << 24)).astype(np.uint32)
