"""Host-side mirror of Brush's rasterizer interface on the gfx950 library.

Mirrors, with the same names, argument meaning and error behaviour:

* ``render`` — ``SplatOps::render`` (brush-render/src/lib.rs:69-88,
  render.rs:49-76) returning ``RenderOutput`` / ``RenderAux``
  (brush-render/src/render_aux.rs:17-81).
* ``rasterize_bwd`` / ``project_bwd`` — ``SplatBwdOps`` (brush-render-bwd/src/
  burn_glue.rs:79-172) returning ``RasterizeGrads`` / ``SplatGrads``
  (burn_glue.rs:56-68).
* ``render_splats`` — the non-differentiable entry point
  (brush-render/src/gaussian_splats.rs:417-437).
* ``render_splats_diff`` / ``render_splats_for_training`` — the
  differentiable entry points (brush-render-bwd/src/burn_glue.rs:476-546),
  here as a torch autograd function whose backward runs rasterize-backward and
  project-backward.

Tensors are torch tensors on a ROCm device; every call goes through
libbrush_hip.so and raises ``BrushHipError`` (a RuntimeError) on failure, in
the places where the reference panics.
"""
from __future__ import annotations

import ctypes
import enum
import math
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import BrushHipError, Uniforms, context, lib, ptr
from .camera import Camera, project_uniforms, tile_bounds


class SplatRenderMode(enum.Enum):
    """gaussian_splats.rs:17-22"""
    Default = 0
    Mip = 1


class RasterizationMode(enum.Enum):
    """gaussian_splats.rs:24-40"""
    Rgba = 0
    RgbaAndDepth = 1

    @property
    def render_depth(self) -> bool:
        return self is RasterizationMode.RgbaAndDepth


class RasterPass(enum.Enum):
    """gaussian_splats.rs:43-66"""
    Forward = 0
    Backward = 1
    BackwardSmoothCutoff = 2

    @property
    def bwd_info(self) -> bool:
        return self is not RasterPass.Forward

    @property
    def smooth_cutoff(self) -> bool:
        return self is RasterPass.BackwardSmoothCutoff


class Rasterizer(enum.Enum):
    """gaussian_splats.rs:68-101: Legacy 16x16 tiles, Candidate 16x8 tiles.
    The forward and the backward of one render must use the same one."""
    Legacy = 16
    Candidate = 8

    @property
    def tile_width(self) -> int:
        return 16

    @property
    def tile_height(self) -> int:
        return self.value

    @property
    def flag(self) -> int:
        return _lib.FLAG_TILE_16X8 if self is Rasterizer.Candidate else 0


class TextureMode(enum.Enum):
    """gaussian_splats.rs:103-108"""
    Packed = 0
    Float = 1


def sh_degree_from_coeffs(n: int) -> int:
    """brush-render/src/sh.rs: number of coefficients per channel -> degree."""
    table = {1: 0, 4: 1, 9: 2, 16: 3, 25: 4}
    if n not in table:
        raise ValueError(f"Invalid nr. of sh bases {n}")
    return table[n]


def _flags(render_mode: SplatRenderMode, raster_mode: RasterizationMode, raster_pass: RasterPass) -> int:
    f = 0
    if raster_pass.bwd_info:
        f |= _lib.FLAG_BWD_INFO
    if raster_pass.smooth_cutoff:
        f |= _lib.FLAG_SMOOTH_CUTOFF
    if raster_mode.render_depth and raster_pass.bwd_info:
        f |= _lib.FLAG_RENDER_DEPTH
    if render_mode is SplatRenderMode.Mip:
        f |= _lib.FLAG_MIP
    return f


def _check_f32(name, t, shape_tail, device):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be float32, got {t.dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must live on the GPU")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")
    if shape_tail is not None and tuple(t.shape[1:]) != tuple(shape_tail):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected [N, {', '.join(map(str, shape_tail))}]")


class ForwardState:
    """Owns one bh_fwd_state (the count-sized buffers of a forward pass)."""

    def __init__(self, ctx: _lib.Context, handle: ctypes.c_void_p):
        self.ctx = ctx
        self.handle = handle
        info = _lib.FwdInfo()
        ctx.check(lib().bh_fwd_state_info(handle, ctypes.byref(info)), "bh_fwd_state_info")
        self.info = info

    def tensor(self, field_name: str, shape, dtype) -> torch.Tensor:
        """Copy one of the state's device buffers into a new torch tensor."""
        out = torch.empty(shape, dtype=dtype, device=f"cuda:{self.ctx.device}")
        nbytes = out.numel() * out.element_size()
        src = getattr(self.info, field_name)
        if nbytes:
            self.ctx.use_current_stream()
            self.ctx.check(lib().bh_copy_device(self.ctx.handle, ptr(out), ctypes.c_void_p(src), nbytes),
                           "bh_copy_device")
        return out

    def backward_lanes(self) -> torch.Tensor | None:
        """A copy of the [N, 11] per-splat gradient lanes (row = global id)
        of this state's latest fused backward, when it ran with the
        context's keep_lanes debug mode; None otherwise."""
        p = ctypes.c_void_p()
        self.ctx.check(lib().bh_fwd_state_backward_lanes(self.handle, ctypes.byref(p)), "bh_fwd_state_backward_lanes")
        if not p.value:
            return None
        n = int(self.info.num_splats)
        out = torch.empty((n, _lib.COMPACT_GRAD_LANES), dtype=torch.float32, device=f"cuda:{self.ctx.device}")
        self.ctx.use_current_stream()
        self.ctx.check(lib().bh_copy_device(self.ctx.handle, ptr(out), p, out.numel() * 4), "bh_copy_device")
        return out

    def release(self):
        if self.handle:
            lib().bh_fwd_state_release(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


@dataclass
class RenderAux:
    """render_aux.rs:70-81"""
    num_visible: int
    num_intersections: int
    visible: torch.Tensor
    max_radius: torch.Tensor
    tile_offsets: torch.Tensor
    img_size: tuple

    def calc_tile_depth(self) -> torch.Tensor:
        """render_aux.rs:83-93: splats per tile."""
        t = self.tile_offsets.to(torch.int64)
        return (t[..., 1] - t[..., 0]).to(torch.int32)


@dataclass
class RenderOutput:
    """render_aux.rs:17-26.  The count-sized buffers are copied out of the
    forward state on first access, and the uniforms turned into a dict on
    first access."""
    out_img: torch.Tensor
    aux: RenderAux
    uniforms: _lib.Uniforms = field(repr=False)
    state: ForwardState = field(repr=False)

    @property
    def project_uniforms(self) -> dict:
        return self.uniforms.to_dict()

    @property
    def projected_splats(self) -> torch.Tensor:
        v = max(self.aux.num_visible, 1)
        return self.state.tensor("projected", (v, _lib.PROJECTED_LANES), torch.float32)

    @property
    def global_from_compact_gid(self) -> torch.Tensor:
        return self.state.tensor("global_from_compact_gid", (max(self.aux.num_visible, 1),), torch.int32)

    @property
    def compact_gid_from_isect(self) -> torch.Tensor:
        return self.state.tensor("compact_gid_from_isect", (max(self.aux.num_intersections, 1),), torch.int32)

    @property
    def tile_id_from_isect(self) -> torch.Tensor:
        return self.state.tensor("tile_id_from_isect", (max(self.aux.num_intersections, 1),), torch.int32)

    @property
    def intersect_counts(self) -> torch.Tensor:
        return self.state.tensor("intersect_counts", (self.state.info.num_splats,), torch.int32)

    @property
    def cum_tiles_hit(self) -> torch.Tensor:
        return self.state.tensor("cum_tiles_hit", (self.aux.num_visible,), torch.int32)

    @property
    def depths(self) -> torch.Tensor:
        return self.state.tensor("depths", (self.aux.num_visible,), torch.float32)

    @property
    def tile_offsets_pre(self) -> torch.Tensor:
        tbw, tbh = self.state.info.tile_bw, self.state.info.tile_bh
        return self.state.tensor("tile_offsets_pre", (tbh, tbw, 2), torch.int32)


_UNIFORMS_CACHE: dict = {}
_UNIFORMS_CACHE_MAX = 64


def _camera_uniforms(camera: Camera, img_w: int, img_h: int, n: int, degree: int, tile_h: int) -> Uniforms:
    """ProjectUniforms of a camera and frame (camera.rs:63-119, 200-254 in
    project_uniforms), kept for the last few cameras: a training or viewer
    loop renders the same camera many times, and the host-side camera maths
    (float64 fov/focal conversions, the world-to-camera inverse, the clamp
    limits) would otherwise run every call.  The key holds every field the
    uniforms depend on; the cached struct is read-only to its users."""
    try:
        key = (tuple(float(x) for x in camera.position), tuple(float(x) for x in camera.rotation),
               float(camera.fov_x), float(camera.fov_y), tuple(float(x) for x in camera.center_uv),
               repr(camera.camera_model), img_w, img_h, n, degree, tile_h)
    except TypeError:
        key = None
    u = _UNIFORMS_CACHE.get(key) if key is not None else None
    if u is None:
        ud = project_uniforms(camera, img_w, img_h, n, degree)
        ud["tile_bw"], ud["tile_bh"] = tile_bounds(img_w, img_h, tile_h)
        u = Uniforms.from_dict(ud)
        if key is not None:
            if len(_UNIFORMS_CACHE) >= _UNIFORMS_CACHE_MAX:
                _UNIFORMS_CACHE.pop(next(iter(_UNIFORMS_CACHE)))
            _UNIFORMS_CACHE[key] = u
    return u


def render(camera: Camera, img_size, transforms: torch.Tensor, sh_coeffs: torch.Tensor,
           raw_opacities: torch.Tensor, render_mode: SplatRenderMode = SplatRenderMode.Default,
           raster_mode: RasterizationMode = RasterizationMode.Rgba, background=(0.0, 0.0, 0.0),
           raster_pass: RasterPass = RasterPass.Forward, uniforms: dict | None = None,
           rasterizer: Rasterizer = Rasterizer.Legacy) -> RenderOutput:
    """SplatOps::render (render.rs:78-543); ``rasterizer`` picks 16x16 or 16x8
    tiles (the reference's render_with_rasterizer, lib.rs:93-108).

    ``uniforms`` may supply a precomputed ``project_uniforms`` dict instead of
    deriving it from ``camera``.
    """
    img_w, img_h = int(img_size[0]), int(img_size[1])
    if img_w <= 0 or img_h <= 0:
        raise ValueError("Can't render images with 0 size.")
    device = transforms.device
    _check_f32("transforms", transforms, (10,), None)
    _check_f32("raw_opacities", raw_opacities, (), device)
    if sh_coeffs.dim() != 3 or sh_coeffs.shape[2] != 3:
        raise ValueError(f"sh_coeffs has shape {tuple(sh_coeffs.shape)}, expected [N, C, 3]")
    _check_f32("sh_coeffs", sh_coeffs, tuple(sh_coeffs.shape[1:]), device)
    n = transforms.shape[0]
    if sh_coeffs.shape[0] != n or raw_opacities.shape[0] != n or raw_opacities.dim() != 1:
        raise ValueError("transforms, sh_coeffs and raw_opacities disagree on the number of splats")
    degree = sh_degree_from_coeffs(sh_coeffs.shape[1])
    transforms = transforms.contiguous()
    sh_coeffs = sh_coeffs.contiguous()
    raw_opacities = raw_opacities.contiguous()

    if uniforms is not None:
        ud = dict(uniforms)
        ud["img_w"], ud["img_h"] = img_w, img_h
        ud["tile_bw"], ud["tile_bh"] = tile_bounds(img_w, img_h, rasterizer.tile_height)
        u = Uniforms.from_dict(ud)
    else:
        u = _camera_uniforms(camera, img_w, img_h, n, degree, rasterizer.tile_height)
    flags = _flags(render_mode, raster_mode, raster_pass) | rasterizer.flag
    depth = (flags & _lib.FLAG_RENDER_DEPTH) != 0
    with torch.cuda.device(device):
        ctx = context(device.index if device.index is not None else torch.cuda.current_device())
        tbw, tbh = tile_bounds(img_w, img_h, rasterizer.tile_height)
        if raster_pass.bwd_info:
            out_img = torch.empty((img_h, img_w, 5 if depth else 4), dtype=torch.float32, device=device)
            visible = torch.empty((n,), dtype=torch.float32, device=device)
        else:
            out_img = torch.empty((img_h, img_w), dtype=torch.int32, device=device)
            visible = torch.zeros((1,), dtype=torch.float32, device=device)
        max_radius = torch.empty((n,), dtype=torch.float32, device=device)
        tile_offsets = torch.empty((tbh, tbw, 2), dtype=torch.int32, device=device)
        bg = (ctypes.c_float * 3)(*[float(x) for x in background])
        handle = ctypes.c_void_p()
        st = lib().bh_render_forward(
            ctx.handle, ctypes.byref(u), bg, ptr(transforms), ptr(sh_coeffs), ptr(raw_opacities), n, degree,
            flags, ptr(out_img), ptr(visible) if raster_pass.bwd_info else ctypes.c_void_p(0), ptr(max_radius),
            ptr(tile_offsets), ctypes.byref(handle))
        ctx.check(st, "render")
        state = ForwardState(ctx, handle)
    info = state.info
    aux = RenderAux(int(info.num_visible), int(info.num_intersections), visible, max_radius, tile_offsets,
                    (img_w, img_h))
    return RenderOutput(out_img, aux, info.uniforms, state)


@dataclass
class SplatGrads:
    """burn_glue.rs:62-68"""
    v_transforms: torch.Tensor
    v_coeffs: torch.Tensor
    v_raw_opac: torch.Tensor
    v_refine_weight: torch.Tensor


def _rasterize_bwd_ptrs(ctx, out_img, projected_p, cgids_p, tile_offsets, num_visible, background, img_size,
                        v_output, smooth_cutoff, render_depth, compute_refine_weight, rasterizer=Rasterizer.Legacy):
    img_w, img_h = int(img_size[0]), int(img_size[1])
    v_combined = torch.empty((max(num_visible, 1), _lib.COMPACT_GRAD_LANES), dtype=torch.float32,
                             device=out_img.device)
    flags = rasterizer.flag
    if smooth_cutoff:
        flags |= _lib.FLAG_SMOOTH_CUTOFF
    if render_depth:
        flags |= _lib.FLAG_RENDER_DEPTH
    if compute_refine_weight:
        flags |= _lib.FLAG_REFINE_WEIGHT
    bg = (ctypes.c_float * 3)(*[float(x) for x in background])
    st = lib().bh_rasterize_backward(ctx.handle, ptr(out_img), projected_p, cgids_p, ptr(tile_offsets),
                                     int(num_visible), bg, img_w, img_h, ptr(v_output), flags, ptr(v_combined))
    ctx.check(st, "rasterize_bwd")
    return v_combined


def rasterize_bwd(out_img, projected_splats, compact_gid_from_isect, tile_offsets, background, img_size, v_output,
                  smooth_cutoff: bool = False, render_depth: bool = False,
                  compute_refine_weight: bool = True, rasterizer: Rasterizer = Rasterizer.Legacy) -> torch.Tensor:
    """SplatBwdOps::rasterize_bwd(_with_refine_weight) -> v_combined [V, 11]
    (render_bwd.rs:90-238); ``rasterizer`` must be the forward's."""
    chans = 5 if render_depth else 4
    if out_img.dim() != 3 or out_img.shape[2] != chans or tuple(v_output.shape) != tuple(out_img.shape):
        raise ValueError("out_img and v_output must both be [H, W, 4] ([H, W, 5] with depth)")
    img_w, img_h = int(img_size[0]), int(img_size[1])
    tbw, tbh = tile_bounds(img_w, img_h, rasterizer.tile_height)
    if tuple(tile_offsets.shape) != (tbh, tbw, 2):
        raise ValueError(f"tile offsets must be [{tbh}, {tbw}, 2], got {tuple(tile_offsets.shape)}")
    num_visible = projected_splats.shape[0]
    with torch.cuda.device(out_img.device):
        ctx = context()
        return _rasterize_bwd_ptrs(ctx, out_img.contiguous(), ptr(projected_splats.contiguous()),
                                   ptr(compact_gid_from_isect.contiguous()), tile_offsets.contiguous(), num_visible,
                                   background, img_size, v_output.contiguous(), smooth_cutoff, render_depth,
                                   compute_refine_weight, rasterizer)


def _project_bwd_ptrs(ctx, transforms, sh_coeffs, raw_opac, gfc_p, uniforms: dict, render_mode, v_combined):
    n = transforms.shape[0]
    dev = transforms.device
    nc = sh_coeffs.shape[1]
    v_t = torch.empty((n, 10), dtype=torch.float32, device=dev)
    v_c = torch.empty((n, nc, 3), dtype=torch.float32, device=dev)
    v_o = torch.empty((n,), dtype=torch.float32, device=dev)
    v_r = torch.empty((n,), dtype=torch.float32, device=dev)
    ud = dict(uniforms)
    ud["total_splats"] = n
    ud["sh_degree"] = sh_degree_from_coeffs(nc)
    u = Uniforms.from_dict(ud)
    flags = _lib.FLAG_MIP if render_mode is SplatRenderMode.Mip else 0
    st = lib().bh_project_backward(ctx.handle, ctypes.byref(u), ptr(transforms), ptr(sh_coeffs), ptr(raw_opac),
                                   gfc_p, ptr(v_combined), flags, ptr(v_t), ptr(v_c), ptr(v_o), ptr(v_r))
    ctx.check(st, "project_bwd")
    return SplatGrads(v_t, v_c, v_o, v_r)


def project_bwd(transforms, sh_coeffs, raw_opac, global_from_compact_gid, project_uniforms: dict,
                render_mode: SplatRenderMode, v_combined) -> SplatGrads:
    """SplatBwdOps::project_bwd (render_bwd.rs:298-447) -> dense SplatGrads."""
    with torch.cuda.device(transforms.device):
        ctx = context()
        return _project_bwd_ptrs(ctx, transforms.contiguous(), sh_coeffs.contiguous(), raw_opac.contiguous(),
                                 ptr(global_from_compact_gid.contiguous()), project_uniforms, render_mode,
                                 v_combined.contiguous())


# ---- splat container and entry points ---------------------------------------------------

def fold_min_scale(transforms: torch.Tensor, raw_opac: torch.Tensor, f: torch.Tensor):
    """gaussian_splats.rs:139-164, the Mip-Splatting 3D filter: scales become
    sqrt(s^2 + f^2) and the opacity is scaled by sqrt(det(s^2)/det(s^2 + f^2))
    over the three axes, clamped to [1e-6, 1 - 1e-6] and turned back into a
    logit.  Differentiable in transforms and raw_opac; ``f`` [N] is a constant."""
    n = transforms.shape[0]
    f = f.detach().to(transforms.device, torch.float32)
    s2 = (transforms[:, 7:10] * 2.0).exp()
    s2f = s2 + (f * f).reshape(n, 1)
    new_log = s2f.log() * 0.5
    out = torch.cat([transforms[:, 0:7], new_log], dim=1)

    def det(t):
        return t[:, 0:1] * t[:, 1:2] * t[:, 2:3]

    coef = (det(s2) / det(s2f)).sqrt().reshape(n)
    opac = (torch.sigmoid(raw_opac) * coef).clamp(1e-6, 1.0 - 1e-6)
    return out, (opac / (1.0 - opac)).log()


@dataclass
class Splats:
    """gaussian_splats.rs:110-127: transforms [N,10] (means | quat wxyz |
    log-scales), sh_coeffs [N,C,3], raw_opacities [N] (logits), and an
    optional frozen per-splat world-space scale floor ``min_scale`` [N] that
    every render folds in (fold_min_scale) and export bakes."""
    transforms: torch.Tensor
    sh_coeffs: torch.Tensor
    raw_opacities: torch.Tensor
    render_mip: bool = False
    min_scale: torch.Tensor | None = None

    @staticmethod
    def from_tensor_data(means, rotation, log_scales, sh_coeffs, raw_opacity, mode=SplatRenderMode.Default):
        """gaussian_splats.rs:218-239"""
        if means.shape[1] != 3 or rotation.shape[1] != 4 or log_scales.shape[1] != 3:
            raise ValueError("means must be [N,3], rotation [N,4], log_scales [N,3]")
        transforms = torch.cat([means, rotation, log_scales], dim=1).contiguous()
        return Splats(transforms, sh_coeffs.contiguous(), raw_opacity.contiguous(), mode is SplatRenderMode.Mip)

    def num_splats(self) -> int:
        return int(self.transforms.shape[0])

    def sh_degree(self) -> int:
        return sh_degree_from_coeffs(self.sh_coeffs.shape[1])

    def means(self):
        return self.transforms[:, 0:3]

    def rotations(self):
        return self.transforms[:, 3:7]

    def log_scales(self):
        return self.transforms[:, 7:10]

    def with_min_scale(self, f: torch.Tensor) -> "Splats":
        """gaussian_splats.rs:241-247"""
        if f.shape != (self.num_splats(),):
            raise ValueError(f"min_scale must be [{self.num_splats()}], got {tuple(f.shape)}")
        return Splats(self.transforms, self.sh_coeffs, self.raw_opacities, self.render_mip, f)

    def folded(self):
        """(transforms, raw_opacities) with the min-scale floor folded in."""
        if self.min_scale is None:
            return self.transforms, self.raw_opacities
        return fold_min_scale(self.transforms, self.raw_opacities, self.min_scale)

    def scales(self):
        """gaussian_splats.rs:279-292: with the floor folded in."""
        return self.folded()[0][:, 7:10].exp()

    def opacities(self):
        """gaussian_splats.rs:261-277: with the floor's energy compensation."""
        return torch.sigmoid(self.folded()[1])

    def bake_min_scale(self) -> "Splats":
        """gaussian_splats.rs:294-307: fold the floor into the parameters and
        drop it; the result renders identically."""
        if self.min_scale is None:
            return self
        with torch.no_grad():
            t, o = self.folded()
        return Splats(t.contiguous(), self.sh_coeffs, o.contiguous(), self.render_mip, None)


def render_splats(splats: Splats, camera: Camera, img_size, background=(0.0, 0.0, 0.0),
                  splat_scale: float | None = None, texture_mode: TextureMode = TextureMode.Float):
    """Non-differentiable render (gaussian_splats.rs:417-437, 468-549):
    returns (image, RenderAux).  Float mode renders with the backward
    bookkeeping (f32 RGBA); Packed mode returns packed RGBA8 in an int32 [H, W]."""
    with torch.no_grad():
        transforms, raw_opacities = splats.folded()  # gaussian_splats.rs:484-491
        if splat_scale is not None:
            transforms = transforms.clone()
            transforms[:, 7:10] += math.log(splat_scale)
    raster_pass = RasterPass.Backward if texture_mode is TextureMode.Float else RasterPass.Forward
    mode = SplatRenderMode.Mip if splats.render_mip else SplatRenderMode.Default
    out = render(camera, img_size, transforms.detach(), splats.sh_coeffs.detach(),
                 raw_opacities.detach(), mode, RasterizationMode.Rgba, background, raster_pass)
    return out.out_img, out.aux


@dataclass
class SplatOutputDiff:
    """burn_glue.rs:386-412: the image is differentiable w.r.t. the splat
    parameters; the refine weight (|dL/dmean2d| statistic) is filled in by the
    backward pass into ``refine_weight`` (the reference registers it as the
    gradient of a dummy holder tensor)."""
    img: torch.Tensor
    num_visible: int
    visible: torch.Tensor
    max_radius: torch.Tensor
    aux: RenderAux
    refine_weight: torch.Tensor | None = None


class _DiffConfig:
    def __init__(self, camera, img_size, background, render_mode, raster_mode, raster_pass, compute_refine_weight,
                 rasterizer=None):
        self.rasterizer = rasterizer or Rasterizer.Legacy
        self.camera = camera
        self.img_size = img_size
        self.background = background
        self.render_mode = render_mode
        self.raster_mode = raster_mode
        self.raster_pass = raster_pass
        self.compute_refine_weight = compute_refine_weight
        # the forward's state and aux, not its RenderOutput: the output image
        # is the autograd node's own output, and a reference to it from here
        # would close a cycle (image -> grad_fn -> ctx -> cfg -> image) that
        # keeps every step's state and image alive until the cyclic garbage
        # collector runs
        self.state = None
        self.aux = None
        self.refine_weight = None


class _RenderSplatsFn(torch.autograd.Function):
    """RenderBackwards (burn_glue.rs:292-378) as a torch autograd node."""

    @staticmethod
    def forward(ctx, transforms, sh_coeffs, raw_opac, cfg: _DiffConfig):
        out = render(cfg.camera, cfg.img_size, transforms.detach(), sh_coeffs.detach(), raw_opac.detach(),
                     cfg.render_mode, cfg.raster_mode, cfg.background, cfg.raster_pass, rasterizer=cfg.rasterizer)
        cfg.state = out.state
        cfg.aux = out.aux
        ctx.cfg = cfg
        ctx.save_for_backward(transforms, sh_coeffs, raw_opac, out.out_img, out.aux.tile_offsets)
        return out.out_img

    @staticmethod
    def backward(ctx, v_img):
        """rasterize_bwd followed by project_bwd in one library call
        (bh_render_backward); the intermediate gradient lanes stay in library
        workspace, as v_combined stays inside RenderBackwards::backward."""
        cfg = ctx.cfg
        transforms, sh_coeffs, raw_opac, out_img, tile_offsets = ctx.saved_tensors
        n = transforms.shape[0]
        dev = transforms.device
        nc = sh_coeffs.shape[1]
        v_t = torch.empty((n, 10), dtype=torch.float32, device=dev)
        v_c = torch.empty((n, nc, 3), dtype=torch.float32, device=dev)
        v_o = torch.empty((n,), dtype=torch.float32, device=dev)
        v_r = torch.empty((n,), dtype=torch.float32, device=dev)
        flags = 0
        if cfg.raster_pass.smooth_cutoff:
            flags |= _lib.FLAG_SMOOTH_CUTOFF
        if cfg.raster_mode.render_depth:
            flags |= _lib.FLAG_RENDER_DEPTH
        if cfg.compute_refine_weight:
            flags |= _lib.FLAG_REFINE_WEIGHT
        bg = (ctypes.c_float * 3)(*[float(x) for x in cfg.background])
        with torch.cuda.device(dev):
            c = context()
            st = lib().bh_render_backward(c.handle, cfg.state.handle, ptr(out_img), ptr(tile_offsets), bg,
                                          ptr(transforms.detach().contiguous()),
                                          ptr(sh_coeffs.detach().contiguous()), ptr(raw_opac.detach().contiguous()),
                                          ptr(v_img.contiguous()), flags, ptr(v_t), ptr(v_c), ptr(v_o), ptr(v_r))
            c.check(st, "render_backward")
        cfg.refine_weight = v_r
        return v_t, v_c, v_o, None


def render_splats_diff(splats: Splats, camera: Camera, img_size, background=(0.0, 0.0, 0.0),
                       compute_refine_weight: bool = True, raster_pass: RasterPass = RasterPass.Backward,
                       raster_mode: RasterizationMode = RasterizationMode.Rgba,
                       rasterizer: Rasterizer = Rasterizer.Legacy) -> SplatOutputDiff:
    """Differentiable render (brush_render_bwd::render_splats and
    render_splats_with_pass, burn_glue.rs:476-483, 548-573)."""
    if not raster_pass.bwd_info:
        raise ValueError("render_splats_with_pass requires a Backward variant")
    mode = SplatRenderMode.Mip if splats.render_mip else SplatRenderMode.Default
    cfg = _DiffConfig(camera, img_size, background, mode, raster_mode, raster_pass, compute_refine_weight,
                      rasterizer)
    transforms, raw_opacities = splats.folded()  # burn_glue.rs:631-641, differentiable through the fold
    img = _RenderSplatsFn.apply(transforms, splats.sh_coeffs, raw_opacities, cfg)
    aux = cfg.aux
    res = SplatOutputDiff(img, aux.num_visible, aux.visible, aux.max_radius, aux)
    res._cfg = cfg

    def _refine():
        return cfg.refine_weight

    res.refine_weight_fn = _refine
    return res


def render_splats_for_training(splats: Splats, camera: Camera, img_size, background=(0.0, 0.0, 0.0),
                               compute_refine_weight: bool = True,
                               rasterization_mode: RasterizationMode = RasterizationMode.Rgba,
                               rasterizer: Rasterizer = Rasterizer.Legacy) -> SplatOutputDiff:
    """burn_glue.rs:518-546 (deferred SH gradients are an Apple-only path and
    are not offered)."""
    return render_splats_diff(splats, camera, img_size, background, compute_refine_weight, RasterPass.Backward,
                              rasterization_mode, rasterizer)
