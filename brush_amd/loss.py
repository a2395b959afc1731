"""Fused L1 + SSIM image loss on the gfx950 library (brush-loss's public surface).

Mirrors crates/brush-loss/src/lib.rs:
* ``ImageLossConfig`` — lib.rs:927-941 (``composite_bg`` None or an RGB
  triple, ``mask`` multiplies the map by the GT alpha);
* ``image_loss(pred, gt_packed, cfg)`` — lib.rs:1630-1681, differentiable:
  pred ``[H, W, 3|4]`` float32 on the GPU, gt_packed ``[H, W]`` int32/uint32
  holding packed RGBA8 (r in the low byte); returns the loss map
  ``[H, W, C]``; with 4 channels the alpha channel is ``|pred.a - gt.a|``;
* ``image_loss_eval`` — lib.rs:1683-1697, forward only.

``pred`` may be a channel slice of a wider image (``img[..., :3]`` of an
RGBA render): the library reads it through its pixel stride, without a copy.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import context, lib, ptr


@dataclass(frozen=True)
class ImageLossConfig:
    l1_weight: float
    ssim_weight: float
    composite_bg: tuple | None = None
    mask: bool = False

    def to_c(self) -> _lib.ImageLossConfig:
        c = _lib.ImageLossConfig()
        c.l1_weight = float(self.l1_weight)
        c.ssim_weight = float(self.ssim_weight)
        c.composite = 0 if self.composite_bg is None else 1
        for i in range(3):
            c.background[i] = 0.0 if self.composite_bg is None else float(self.composite_bg[i])
        c.mask = 1 if self.mask else 0
        return c


def pixel_view(pred: torch.Tensor):
    """(tensor, pixel stride) for reading ``pred`` [H, W, C] in place through
    its data pointer: channels unit-strided and pixels evenly strided (a
    channel slice of a contiguous image), else a contiguous copy."""
    if pred.dim() != 3 or pred.dtype != torch.float32 or pred.device.type != "cuda":
        raise ValueError("pred must be a float32 [H, W, C] tensor on the GPU")
    h, w, c = pred.shape
    if c not in (3, 4):
        raise ValueError(f"pred must have 3 or 4 channels, got {c}")
    s = pred.stride()
    if s[2] == 1 and s[1] >= c and s[0] == w * s[1]:
        return pred, int(s[1])
    return pred.contiguous(), c


def _data(t: torch.Tensor) -> ctypes.c_void_p:
    """Data pointer of a (possibly strided) view."""
    return ctypes.c_void_p(t.data_ptr())


def _check_gt(gt_packed: torch.Tensor, h: int, w: int):
    if gt_packed.dim() != 2 or tuple(gt_packed.shape) != (h, w):
        raise ValueError(f"gt_packed must be [{h}, {w}]")
    if gt_packed.dtype not in (torch.int32, torch.uint32):
        raise ValueError("gt_packed must hold packed RGBA8 as int32/uint32")
    return gt_packed.contiguous()


def image_loss_forward_raw(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig) -> torch.Tensor:
    base, stride = pixel_view(pred)
    h, w, c = pred.shape
    gt = _check_gt(gt_packed, h, w)
    out = torch.empty((h, w, c), dtype=torch.float32, device=pred.device)
    with torch.cuda.device(pred.device):
        ctx = context()
        cc = cfg.to_c()
        ctx.check(lib().bh_image_loss_forward(ctx.handle, _data(base), stride, c, ptr(gt), w, h, ctypes.byref(cc),
                                              ptr(out)), "image_loss_forward")
    return out


def image_loss_backward_raw(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig,
                            dl_dmap: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """dL/dpred in pred's pixel layout: ``out`` [H, W, stride] (allocated when
    None); channels past C are zero."""
    base, stride = pixel_view(pred)
    h, w, c = pred.shape
    gt = _check_gt(gt_packed, h, w)
    dmap = dl_dmap.contiguous()
    if tuple(dmap.shape) != (h, w, c):
        raise ValueError("dl_dmap must have pred's shape")
    if out is None:
        out = torch.empty((h, w, stride), dtype=torch.float32, device=pred.device)
    with torch.cuda.device(pred.device):
        ctx = context()
        cc = cfg.to_c()
        ctx.check(lib().bh_image_loss_backward(ctx.handle, _data(base), stride, c, ptr(gt), w, h, ctypes.byref(cc),
                                               ptr(dmap), ptr(out)), "image_loss_backward")
    return out


class _ImageLossFn(torch.autograd.Function):
    """ImageLossBackward (lib.rs:1584-1627) as a torch autograd node."""

    @staticmethod
    def forward(ctx, pred, gt_packed, cfg: ImageLossConfig):
        ctx.cfg = cfg
        ctx.save_for_backward(pred, gt_packed)
        return image_loss_forward_raw(pred, gt_packed, cfg)

    @staticmethod
    def backward(ctx, dl_dmap):
        pred, gt_packed = ctx.saved_tensors
        g = image_loss_backward_raw(pred, gt_packed, ctx.cfg, dl_dmap)
        c = pred.shape[2]
        return (g if g.shape[2] == c else g[..., :c]), None, None


def image_loss(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig) -> torch.Tensor:
    """Differentiable L1 + SSIM loss map (lib.rs:1630-1681)."""
    return _ImageLossFn.apply(pred, gt_packed, cfg)


def image_loss_eval(pred: torch.Tensor, gt_packed: torch.Tensor, cfg: ImageLossConfig) -> torch.Tensor:
    """Forward-only loss map (lib.rs:1683-1697)."""
    with torch.no_grad():
        return image_loss_forward_raw(pred.detach(), gt_packed, cfg)


def pack_rgba8(rgb: torch.Tensor, alpha: torch.Tensor | None = None) -> torch.Tensor:
    """Float RGB(A) in [0, 1] -> packed RGBA8 int32 [H, W] (r in the low byte),
    each channel round(clamp(x, 0, 1) * 255); alpha 255 when absent (the GT
    format of brush-dataset, scene.rs:118-135)."""
    q = torch.round(rgb.clamp(0.0, 1.0) * 255.0).to(torch.int64)
    a = torch.full_like(q[..., 0], 255) if alpha is None else torch.round(alpha.clamp(0.0, 1.0) * 255.0).to(torch.int64)
    packed = q[..., 0] | (q[..., 1] << 8) | (q[..., 2] << 16) | (a << 24)
    return (packed - ((packed >> 31) << 32)).to(torch.int32)
