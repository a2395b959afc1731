"""ctypes wrapper and numpy orchestration of the CPU restatement (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, as the checker.  The product package
(brush_amd) never imports this module.

The forward pipeline mirrors render.rs:78-543: project_forward, compaction in
global-id order, stable depth sort, gather + inclusive scan of tile counts,
project_visible, map_gaussians_to_intersect, stable tile sort, tile offsets,
rasterize.  Compaction in global-id order followed by a stable sort resolves
equal depths by global id; the reference resolves them by atomic arrival
order, which is not reproducible (brush-render/src/tests/mod.rs:443-451).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# BH_ORACLE_LIB selects another build of the same sources (the sanitizer
# build, tests/test_sanitizers.py)
_LIB_PATH = os.environ.get("BH_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")

FLAG_BWD_INFO = 1
FLAG_SMOOTH_CUTOFF = 2
FLAG_RENDER_DEPTH = 4
FLAG_MIP = 8
FLAG_REFINE_WEIGHT = 16
FLAG_TILE_16X8 = 32


class Uniforms(ctypes.Structure):
    """bh_project_uniforms (include/brush_hip.h)."""

    _fields_ = [
        ("viewmat", ctypes.c_float * 12),
        ("half_max_render_fov", ctypes.c_float),
        ("fx", ctypes.c_float), ("fy", ctypes.c_float), ("cx", ctypes.c_float), ("cy", ctypes.c_float),
        ("lim_pos_x", ctypes.c_float), ("lim_pos_y", ctypes.c_float),
        ("lim_neg_x", ctypes.c_float), ("lim_neg_y", ctypes.c_float),
        ("camera_pos", ctypes.c_float * 3),
        ("img_w", ctypes.c_uint32), ("img_h", ctypes.c_uint32),
        ("tile_bw", ctypes.c_uint32), ("tile_bh", ctypes.c_uint32),
        ("sh_degree", ctypes.c_uint32),
        ("total_splats", ctypes.c_uint32),
        ("num_visible", ctypes.c_uint32),
        ("camera_model", ctypes.c_uint32),
        ("camera_params", ctypes.c_float * 8),
    ]


class LossConfig(ctypes.Structure):
    """bh_image_loss_config (include/brush_hip.h)."""

    _fields_ = [("l1_weight", ctypes.c_float), ("ssim_weight", ctypes.c_float), ("composite", ctypes.c_uint32),
                ("background", ctypes.c_float * 3), ("mask", ctypes.c_uint32)]


class AdamConfig(ctypes.Structure):
    """bh_adam_config (include/brush_hip.h)."""

    _fields_ = [("beta_1", ctypes.c_float), ("beta_2", ctypes.c_float), ("epsilon", ctypes.c_float)]


def loss_config(l1_weight: float, ssim_weight: float, composite_bg=None, mask: bool = False) -> LossConfig:
    c = LossConfig()
    c.l1_weight = l1_weight
    c.ssim_weight = ssim_weight
    c.composite = 0 if composite_bg is None else 1
    for i in range(3):
        c.background[i] = 0.0 if composite_bg is None else float(composite_bg[i])
    c.mask = 1 if mask else 0
    return c


def make_uniforms(d: dict) -> Uniforms:
    u = Uniforms()
    for i, v in enumerate(d["viewmat"]):
        u.viewmat[i] = float(v)
    for k in ("half_max_render_fov", "fx", "fy", "cx", "cy", "lim_pos_x", "lim_pos_y", "lim_neg_x", "lim_neg_y"):
        setattr(u, k, float(d[k]))
    for i in range(3):
        u.camera_pos[i] = float(d["camera_pos"][i])
    for k in ("img_w", "img_h", "tile_bw", "tile_bh", "sh_degree", "total_splats", "num_visible"):
        setattr(u, k, int(d[k]))
    u.camera_model = int(d.get("camera_model", 0))
    for i, v in enumerate(d.get("camera_params", ())):
        u.camera_params[i] = float(v)
    return u


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is missing: run `make -C oracle` or __graft_entry__.build()")
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        U32 = ctypes.c_uint32
        U64 = ctypes.c_uint64
        UP = ctypes.POINTER(Uniforms)
        L.or_set_threads.argtypes = [ctypes.c_int]
        L.or_expf.argtypes = [P, P, U64]
        L.or_exp2_neg.argtypes = [P, P, U64]
        L.or_div_by_recip.argtypes = [P, P, P, U64]
        L.or_power_log2.argtypes = [P, P, P, P, P, P, U64]
        L.or_logf.argtypes = [P, P, U64]
        L.or_atan2f.argtypes = [P, P, P, U64]
        L.or_camera_project.argtypes = [UP, P, U64, P, P]
        L.or_camera_jacobian.argtypes = [UP, P, U64, P]
        L.or_camera_vjp.argtypes = [UP, P, P, P, P, U64, P]
        L.or_get_max_threads.restype = ctypes.c_int
        L.or_project_forward.argtypes = [UP, P, P, U32, U32, U32, P, P, P, P]
        L.or_project_forward.restype = U64
        L.or_stable_sort.argtypes = [P, P, U64, U32]
        L.or_prefix_sum.argtypes = [P, P, U64]
        L.or_project_visible.argtypes = [UP, P, P, P, P, U32, U32, U32, P]
        L.or_map_intersects.argtypes = [U32, U32, U32, P, P, U32, P, P]
        L.or_tile_offsets.argtypes = [P, U64, U32, P]
        L.or_rasterize.argtypes = [U32, U32, U32, U32, P, P, P, P, P, U32, P, P, P]
        L.or_rasterize_reference.argtypes = [P, U32, U32, U32, P, U32, P]
        L.or_rasterize_backward.argtypes = [U32, U32, U32, U32, P, P, P, P, P, U32, P, U32, P]
        L.or_rasterize_backward_check.argtypes = [U32, U32, U32, U32, P, P, P, P, P, U32, P, U32, U32, P, P, P]
        L.or_rasterize_backward_f64.argtypes = [U32, U32, U32, U32, P, P, P, P, P, U32, P, U32, P]
        L.or_project_backward.argtypes = [UP, P, P, P, P, U32, U32, U32, U32, P, P, P, P, P]
        L.or_gauss_taps.argtypes = [P]
        L.or_image_loss_forward.argtypes = [P, U32, U32, P, U32, U32, ctypes.POINTER(LossConfig), P]
        L.or_image_loss_backward.argtypes = [P, U32, U32, P, U32, U32, ctypes.POINTER(LossConfig), P, P]
        L.or_adam_scaled_step.argtypes = [P, P, P, P, P, U32, U32, U32, ctypes.c_float, U32,
                                          ctypes.POINTER(AdamConfig)]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n: int):
    lib().or_set_threads(int(n))


def max_threads() -> int:
    return int(lib().or_get_max_threads())


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_expf(_p(x), _p(out), x.size)
    return out


def exp2_neg(x: np.ndarray) -> np.ndarray:
    """2^x as the blend kernels evaluate the splat Gaussian (bh_math.h
    bh_exp2_neg; arguments in [-126, 1])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_exp2_neg(_p(x), _p(out), x.size)
    return out


def div_by_recip(num, den) -> np.ndarray:
    """The tile walks' quotient from a rounded reciprocal (bh_tile_walk.h
    div_by_recip), for its pin against the division."""
    num, den = (np.ascontiguousarray(a, dtype=np.float32) for a in np.broadcast_arrays(num, den))
    out = np.empty_like(num)
    lib().or_div_by_recip(_p(num), _p(den), _p(out), out.size)
    return out


def power_log2(c00, c01, c11, dx, dy) -> np.ndarray:
    """sigma log2(e) of pixel offsets (dx, dy) = mean - pixel centre, from the
    conic scaled as the blend kernels scale it (bh_conic_log2, bh_power_log2);
    arguments broadcast."""
    arrs = np.broadcast_arrays(*[np.asarray(a, dtype=np.float32) for a in (c00, c01, c11, dx, dy)])
    arrs = [np.ascontiguousarray(a) for a in arrs]
    out = np.empty_like(arrs[0])
    lib().or_power_log2(*[_p(a) for a in arrs], _p(out), out.size)
    return out


def atan2f(y: np.ndarray, x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(y)
    lib().or_atan2f(_p(y), _p(x), _p(out), y.size)
    return out


def camera_project(uniforms: dict, pts: np.ndarray):
    """(screen points [n, 2], depth-culled mask [n]) of camera-space points
    through the uniforms' camera model."""
    u = make_uniforms(uniforms)
    pts = np.ascontiguousarray(pts, dtype=np.float32).reshape(-1, 3)
    out = np.empty((pts.shape[0], 2), np.float32)
    culled = np.empty(pts.shape[0], np.uint8)
    lib().or_camera_project(ctypes.byref(u), _p(pts), pts.shape[0], _p(out), _p(culled))
    return out, culled.astype(bool)


def camera_jacobian(uniforms: dict, pts: np.ndarray) -> np.ndarray:
    """[n, 2, 3] projection Jacobians (rows u, v; columns x, y, z)."""
    u = make_uniforms(uniforms)
    pts = np.ascontiguousarray(pts, dtype=np.float32).reshape(-1, 3)
    out = np.empty((pts.shape[0], 2, 3), np.float32)
    lib().or_camera_jacobian(ctypes.byref(u), _p(pts), pts.shape[0], _p(out))
    return out


def camera_vjp(uniforms: dict, mean_c, cov_c, v_cov2d, v_mean2d) -> np.ndarray:
    """[n, 3] projection VJP: cov_c [n, 6] (c00 c01 c02 c11 c12 c22), v_cov2d
    [n, 3] (c00 c01 c11), v_mean2d [n, 2]."""
    u = make_uniforms(uniforms)
    a = [np.ascontiguousarray(x, dtype=np.float32) for x in (mean_c, cov_c, v_cov2d, v_mean2d)]
    n = a[0].reshape(-1, 3).shape[0]
    out = np.empty((n, 3), np.float32)
    lib().or_camera_vjp(ctypes.byref(u), _p(a[0]), _p(a[1]), _p(a[2]), _p(a[3]), n, _p(out))
    return out


def logf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().or_logf(_p(x), _p(out), x.size)
    return out


# ---- primitives ---------------------------------------------------------------

def stable_sort(keys: np.ndarray, vals: np.ndarray, sorting_bits: int = 32):
    k = np.ascontiguousarray(keys, dtype=np.uint32).copy()
    v = np.ascontiguousarray(vals, dtype=np.uint32).copy()
    lib().or_stable_sort(_p(k), _p(v), k.size, sorting_bits)
    return k, v


def prefix_sum(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint32)
    out = np.empty_like(x)
    lib().or_prefix_sum(_p(x), _p(out), x.size)
    return out


def tile_offsets(tile_ids: np.ndarray, num_tiles: int) -> np.ndarray:
    ids = np.ascontiguousarray(tile_ids, dtype=np.uint32)
    out = np.empty((num_tiles * 2,), dtype=np.uint32)
    lib().or_tile_offsets(_p(ids), ids.size, num_tiles, _p(out))
    return out


def rasterize_reference(projected: np.ndarray, img_w: int, img_h: int, background, smooth: bool) -> np.ndarray:
    proj = np.ascontiguousarray(projected, dtype=np.float32).reshape(-1, 10)
    bg = np.asarray(background, dtype=np.float32)
    out = np.empty((img_h, img_w, 4), dtype=np.float32)
    lib().or_rasterize_reference(_p(proj), proj.shape[0], img_w, img_h, _p(bg), int(smooth), _p(out))
    return out


# ---- full forward / backward ----------------------------------------------------

@dataclass
class ForwardResult:
    num_visible: int
    num_intersections: int
    intersect_counts: np.ndarray
    max_radius: np.ndarray
    depths_sorted: np.ndarray
    global_from_compact_gid: np.ndarray
    cum_tiles_hit: np.ndarray
    projected: np.ndarray
    tile_id_from_isect: np.ndarray
    compact_gid_from_isect: np.ndarray
    tile_offsets_pre: np.ndarray
    tile_offsets: np.ndarray
    out_img: np.ndarray
    visible: np.ndarray
    uniforms: dict


def render_forward(uniforms: dict, transforms, sh_coeffs, raw_opac, flags: int = FLAG_BWD_INFO,
                   background=(0.0, 0.0, 0.0)) -> ForwardResult:
    L = lib()
    transforms = np.ascontiguousarray(transforms, dtype=np.float32).reshape(-1, 10)
    sh_coeffs = np.ascontiguousarray(sh_coeffs, dtype=np.float32)
    raw_opac = np.ascontiguousarray(raw_opac, dtype=np.float32).reshape(-1)
    n = transforms.shape[0]
    nc = sh_coeffs.shape[1] if sh_coeffs.ndim == 3 else 1
    deg = int(round(nc ** 0.5)) - 1
    ud = dict(uniforms)
    ud["total_splats"] = n
    ud["sh_degree"] = deg
    w, h = ud["img_w"], ud["img_h"]
    # calc_tile_bounds_for_dims (render.rs:36-47): 16x16 tiles, or 16x8
    th = 8 if flags & FLAG_TILE_16X8 else 16
    ud["tile_bw"], ud["tile_bh"], ud["tile_h"] = (w + 15) // 16, (h + th - 1) // th, th
    tbw, tbh = ud["tile_bw"], ud["tile_bh"]
    num_tiles = tbw * tbh
    mip = int((flags & FLAG_MIP) != 0)
    bwd_info = (flags & FLAG_BWD_INFO) != 0
    depth = bwd_info and (flags & FLAG_RENDER_DEPTH) != 0
    bg = np.asarray(background, dtype=np.float32)
    u = make_uniforms(ud)

    counts = np.zeros(n, np.uint32)
    radius = np.zeros(n, np.float32)
    depths = np.zeros(n, np.float32)
    mask = np.zeros(n, np.uint8)
    total = 0
    if n:
        total = L.or_project_forward(ctypes.byref(u), _p(transforms), _p(raw_opac), n, mip, th,
                                     _p(counts), _p(radius), _p(depths), _p(mask))
    vis_ids = np.nonzero(mask)[0].astype(np.uint32)
    num_visible = int(vis_ids.size)
    if total >= 2 ** 32:
        raise OverflowError("more than 2^32 intersections")
    dkeys = depths[vis_ids].view(np.uint32).copy()
    dkeys, gfc = stable_sort(dkeys, vis_ids, 32)
    depths_sorted = dkeys.view(np.float32)
    compact_counts = counts[gfc]
    cum = prefix_sum(compact_counts)
    ud["num_visible"] = num_visible
    u = make_uniforms(ud)
    projected = np.zeros((max(num_visible, 1), 10), np.float32)
    if num_visible:
        L.or_project_visible(ctypes.byref(u), _p(transforms), _p(sh_coeffs), _p(raw_opac), _p(gfc),
                             num_visible, deg, mip, _p(projected))
    m = int(total)
    tile_ids = np.zeros(max(m, 1), np.uint32)
    cgids = np.zeros(max(m, 1), np.uint32)
    if num_visible and m:
        L.or_map_intersects(tbw, tbh, th, _p(projected), _p(cum), num_visible, _p(tile_ids), _p(cgids))
    bits = int(num_tiles).bit_length()  # render.rs:392: 32 - leading_zeros(T)
    if m:
        tk, tv = stable_sort(tile_ids[:m], cgids[:m], bits)
        tile_ids[:m] = tk
        cgids[:m] = tv
    off_pre = tile_offsets(tile_ids[:m], num_tiles)
    off_post = np.zeros_like(off_pre)
    if bwd_info:
        out_img = np.zeros((h, w, 5 if depth else 4), np.float32)
        visible = np.zeros(n, np.float32)
    else:
        out_img = np.zeros((h, w), np.uint32)
        visible = np.zeros(1, np.float32)
    gfc_arg = gfc if gfc.size else np.zeros(1, np.uint32)
    L.or_rasterize(w, h, tbw, tbh, _p(bg), _p(projected), _p(cgids), _p(gfc_arg), _p(off_pre),
                   flags, _p(out_img), _p(visible), _p(off_post))
    return ForwardResult(num_visible, m, counts, radius, depths_sorted, gfc, cum, projected,
                         tile_ids, cgids, off_pre.reshape(tbh, tbw, 2), off_post.reshape(tbh, tbw, 2),
                         out_img, visible, ud)


def rasterize_backward(fwd: ForwardResult, v_output: np.ndarray, flags: int = FLAG_REFINE_WEIGHT,
                       background=(0.0, 0.0, 0.0)) -> np.ndarray:
    ud = fwd.uniforms
    bg = np.asarray(background, dtype=np.float32)
    v_output = np.ascontiguousarray(v_output, dtype=np.float32)
    v_comb = np.zeros((max(fwd.num_visible, 1), 11), np.float32)
    if ud.get("tile_h", 16) == 8:
        flags |= FLAG_TILE_16X8
    lib().or_rasterize_backward(ud["img_w"], ud["img_h"], ud["tile_bw"], ud["tile_bh"], _p(bg),
                                _p(np.ascontiguousarray(fwd.out_img)), _p(fwd.projected),
                                _p(fwd.compact_gid_from_isect),
                                _p(np.ascontiguousarray(fwd.tile_offsets).reshape(-1)),
                                fwd.num_visible, _p(v_output), flags, _p(v_comb))
    return v_comb


CHECK_DROP_LAST_BATCH = 1


def _raster_bwd_args(fwd: ForwardResult, v_output, flags, background):
    ud = fwd.uniforms
    if ud.get("tile_h", 16) == 8:
        flags |= FLAG_TILE_16X8
    bg = np.asarray(background, dtype=np.float32)
    v_output = np.ascontiguousarray(v_output, dtype=np.float32)
    keep = (bg, v_output, np.ascontiguousarray(fwd.out_img), np.ascontiguousarray(fwd.tile_offsets).reshape(-1))
    args = [ud["img_w"], ud["img_h"], ud["tile_bw"], ud["tile_bh"], _p(keep[0]), _p(keep[2]), _p(fwd.projected),
            _p(fwd.compact_gid_from_isect), _p(keep[3]), fwd.num_visible, _p(keep[1]), flags]
    return args, keep


def rasterize_backward_check(fwd: ForwardResult, v_output: np.ndarray, flags: int = FLAG_REFINE_WEIGHT,
                             background=(0.0, 0.0, 0.0), check: int = 0):
    """Test support for the gradient tolerance: the f32 backward (as
    rasterize_backward, or with a planted mistake: ``check`` =
    CHECK_DROP_LAST_BATCH) and, per lane, the sum of the magnitude bounds of
    the lane's per-pixel terms (or_rasterize_backward_check in
    bh_oracle.h).  Returns (v_combined, v_abs), both [max(V, 1), 11]."""
    args, keep = _raster_bwd_args(fwd, v_output, flags, background)
    rows = max(fwd.num_visible, 1)
    v_comb = np.zeros((rows, 11), np.float32)
    v_abs = np.zeros((rows, 11), np.float32)
    v_sq = np.zeros((rows, 11), np.float32)
    lib().or_rasterize_backward_check(*args, check, _p(v_comb), _p(v_abs), _p(v_sq))
    return v_comb, v_abs, np.sqrt(v_sq)


def rasterize_backward_f64(fwd: ForwardResult, v_output: np.ndarray, flags: int = FLAG_REFINE_WEIGHT,
                           background=(0.0, 0.0, 0.0)) -> np.ndarray:
    """The backward with every gradient quantity in double (the f32
    decisions and alpha): a second, more accurate evaluation of the same
    gradient, for calibrating tolerances."""
    args, keep = _raster_bwd_args(fwd, v_output, flags, background)
    v_comb = np.zeros((max(fwd.num_visible, 1), 11), np.float32)
    lib().or_rasterize_backward_f64(*args, _p(v_comb))
    return v_comb


def project_backward(fwd: ForwardResult, transforms, sh_coeffs, raw_opac, v_combined, mip: bool = False):
    ud = fwd.uniforms
    transforms = np.ascontiguousarray(transforms, dtype=np.float32).reshape(-1, 10)
    sh_coeffs = np.ascontiguousarray(sh_coeffs, dtype=np.float32)
    raw_opac = np.ascontiguousarray(raw_opac, dtype=np.float32).reshape(-1)
    n = transforms.shape[0]
    nc = sh_coeffs.shape[1]
    deg = ud["sh_degree"]
    v_t = np.empty((n, 10), np.float32)
    v_c = np.empty((n, nc, 3), np.float32)
    v_o = np.empty((n,), np.float32)
    v_r = np.empty((n,), np.float32)
    gfc = fwd.global_from_compact_gid if fwd.num_visible else np.zeros(1, np.uint32)
    u = make_uniforms(ud)
    lib().or_project_backward(ctypes.byref(u), _p(transforms), _p(sh_coeffs), _p(raw_opac), _p(gfc),
                              fwd.num_visible, n, deg, int(mip),
                              _p(np.ascontiguousarray(v_combined, dtype=np.float32)),
                              _p(v_t), _p(v_c), _p(v_o), _p(v_r))
    return v_t, v_c, v_o, v_r


# ---- training step: image loss and AdamScaled (bh_oracle_train.c) ----------------------------------

def gauss_taps() -> np.ndarray:
    t = np.zeros(6, np.float32)
    lib().or_gauss_taps(_p(t))
    return t


def image_loss_forward(pred: np.ndarray, channels: int, gt_packed: np.ndarray, cfg: LossConfig) -> np.ndarray:
    """pred f32 [H, W, stride], gt u32 [H, W] -> loss map f32 [H, W, channels]."""
    pred = np.ascontiguousarray(pred, dtype=np.float32)
    h, w, stride = pred.shape
    gt = np.ascontiguousarray(gt_packed, dtype=np.uint32)
    out = np.empty((h, w, channels), np.float32)
    lib().or_image_loss_forward(_p(pred), stride, channels, _p(gt), w, h, ctypes.byref(cfg), _p(out))
    return out


def image_loss_backward(pred: np.ndarray, channels: int, gt_packed: np.ndarray, cfg: LossConfig,
                        dl_dmap: np.ndarray) -> np.ndarray:
    """-> dl_dpred f32 [H, W, stride] (zeros past `channels`)."""
    pred = np.ascontiguousarray(pred, dtype=np.float32)
    h, w, stride = pred.shape
    gt = np.ascontiguousarray(gt_packed, dtype=np.uint32)
    dmap = np.ascontiguousarray(dl_dmap, dtype=np.float32)
    out = np.empty((h, w, stride), np.float32)
    lib().or_image_loss_backward(_p(pred), stride, channels, _p(gt), w, h, ctypes.byref(cfg), _p(dmap), _p(out))
    return out


def adam_scaled_step(param: np.ndarray, grad: np.ndarray, m1: np.ndarray, m2: np.ndarray, scaling, reduce: bool,
                     lr: float, time: int, beta_1: float = 0.9, beta_2: float = 0.999, epsilon: float = 1e-15):
    """In place on param, m1, m2 (f32, C-contiguous); param viewed as [rows, row_len]."""
    rows = param.shape[0]
    row_len = int(np.prod(param.shape[1:])) if param.ndim > 1 else 1
    cfg = AdamConfig()
    cfg.beta_1, cfg.beta_2, cfg.epsilon = beta_1, beta_2, epsilon
    sc = None if scaling is None else np.ascontiguousarray(scaling, dtype=np.float32).reshape(-1)
    g = np.ascontiguousarray(grad, dtype=np.float32)
    lib().or_adam_scaled_step(_p(param), _p(g), _p(m1), _p(m2), _p(sc) if sc is not None else None, rows, row_len,
                              int(reduce), float(lr), int(time), ctypes.byref(cfg))
