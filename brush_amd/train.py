"""One training step of a splat scene on the gfx950 library: render, fused
L1 + SSIM loss, backward through the rasterizer, AdamScaled update.

Mirrors the pieces of crates/brush-train that follow the rasterizer:
* ``AdamScaled`` / ``AdamState`` — adam_scaled.rs:51-113, 216-383 (Adam with a
  per-column learning-rate scale and an optional per-row second moment);
* ``TrainConfig`` — the learning rates and loss weight of config.rs:67-210;
* ``SplatTrainer.step`` — the loss and optimizer part of train.rs:682-1051:
  ``render_splats_for_training``, ``image_loss`` with weights
  ``(1 - ssim_weight, -ssim_weight)``, ``loss_map.mean()``, backward, then one
  optimizer step on transforms (per-column rates: means, rotations, scales),
  SH coefficients (DC at ``lr_coeffs_dc``, higher bands divided by
  ``lr_coeffs_sh_scale``, second moment per splat) and raw opacities.

Scope: the step the benchmark configuration names.  The
reference's densification, pruning, opacity decay, mean noise, LR schedules,
appearance models and LPIPS are not part of it.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import context, lib, ptr
from .camera import Camera
from .loss import ImageLossConfig, image_loss_backward_raw, image_loss_forward_raw
from .render import RasterizationMode, Rasterizer, RasterPass, SplatRenderMode, Splats, fold_min_scale, render


@dataclass
class AdamState:
    """adam_scaled.rs:80-113: moments, step count, per-column scale, and
    whether the second moment is one value per row."""

    moment_1: torch.Tensor | None = None
    moment_2: torch.Tensor | None = None
    time: int = 0
    scaling: torch.Tensor | None = None
    reduce_moment_2: bool = False


class AdamScaled:
    """AdamScaledConfig + AdamScaled (adam_scaled.rs:57-69, 216-383)."""

    def __init__(self, beta_1: float = 0.9, beta_2: float = 0.999, epsilon: float = 1e-5):
        self.cfg = _lib.AdamConfig()
        self.cfg.beta_1, self.cfg.beta_2, self.cfg.epsilon = beta_1, beta_2, epsilon

    def step(self, lr: float, param: torch.Tensor, grad: torch.Tensor, state: AdamState) -> AdamState:
        """One in-place update of ``param`` (rows = first dim) with ``grad``."""
        if param.dtype != torch.float32 or grad.shape != param.shape or not param.is_contiguous():
            raise ValueError("param must be contiguous float32 with grad of the same shape")
        rows = param.shape[0]
        row_len = param[0].numel() if param.dim() > 1 and rows else 1
        if state.moment_1 is None:
            state.moment_1 = torch.empty_like(param)
            state.moment_2 = torch.empty((rows,) if state.reduce_moment_2 else param.shape, dtype=torch.float32,
                                         device=param.device)
        state.time += 1
        scale = None
        if state.scaling is not None:
            scale = state.scaling.reshape(-1)
            if scale.device != param.device or scale.dtype != torch.float32 or not scale.is_contiguous():
                scale = scale.to(device=param.device, dtype=torch.float32).contiguous()
            if scale.numel() != row_len:
                raise ValueError(f"scaling has {scale.numel()} entries for rows of {row_len}")
        g = grad.contiguous()
        with torch.cuda.device(param.device):
            ctx = context()
            ctx.check(lib().bh_adam_scaled_step(ctx.handle, ptr(param), ptr(g), ptr(state.moment_1),
                                                ptr(state.moment_2), ptr(scale) if scale is not None else None,
                                                rows, row_len, int(state.reduce_moment_2), float(lr),
                                                state.time, ctypes.byref(self.cfg)), "adam_scaled_step")
        return state


@dataclass
class TrainConfig:
    """Learning rates and loss weight (config.rs:67-210); lr_mean and
    lr_coeffs_dc default to BASELINE config 4's values, the rest to brush's."""

    lr_mean: float = 1.6e-4
    lr_rotation: float = 2e-3
    lr_scale: float = 7e-3
    lr_coeffs_dc: float = 2.5e-3
    lr_coeffs_sh_scale: float = 10.0
    lr_opac: float = 0.012
    ssim_weight: float = 0.2
    compute_refine_weight: bool = True


@dataclass
class SplatTrainer:
    config: TrainConfig = field(default_factory=TrainConfig)
    background: tuple = (0.0, 0.0, 0.0)
    rasterizer: Rasterizer = Rasterizer.Legacy

    def __post_init__(self):
        # train.rs:141-143: epsilon 1e-15
        self.optim = AdamScaled(epsilon=1e-15)
        self.state_transforms = AdamState()
        self.state_sh = AdamState(reduce_moment_2=True)
        self.state_opac = AdamState()
        self._chain = None
        self._lr_t = None

    def _uniform_chain(self, h: int, w: int, device) -> torch.Tensor:
        """dL/dmap of loss_map.mean(): 1 / (3 H W) everywhere (cached)."""
        if self._chain is None or tuple(self._chain.shape) != (h, w, 3) or self._chain.device != device:
            self._chain = torch.full((h, w, 3), 1.0 / (3 * h * w), dtype=torch.float32, device=device)
        return self._chain

    def step(self, splats: Splats, camera: Camera, gt_packed: torch.Tensor, record_grads: bool = False) -> dict:
        """One optimisation step; updates ``splats`` in place.  Returns the
        loss (a GPU scalar), num_visible and, with ``record_grads``, the
        gradients the optimizer consumed."""
        cfg = self.config
        h, w = gt_packed.shape
        t, s, o = splats.transforms, splats.sh_coeffs, splats.raw_opacities
        mode = SplatRenderMode.Mip if splats.render_mip else SplatRenderMode.Default
        rt, ro = t, o
        if splats.min_scale is not None:
            # the render sees the folded floor (burn_glue.rs:631-641); its
            # gradients are chained back through the fold after the backward
            with torch.enable_grad():
                t_leaf = t.detach().requires_grad_()
                o_leaf = o.detach().requires_grad_()
                rt, ro = fold_min_scale(t_leaf, o_leaf, splats.min_scale)
        out = render(camera, (w, h), rt.detach(), s.detach(), ro.detach(), mode, RasterizationMode.Rgba,
                     self.background, RasterPass.Backward, rasterizer=self.rasterizer)
        img = out.out_img  # [H, W, 4]
        loss_cfg = ImageLossConfig(1.0 - cfg.ssim_weight, -cfg.ssim_weight)
        rgb = img[..., :3]
        loss_map = image_loss_forward_raw(rgb, gt_packed, loss_cfg)
        loss = loss_map.mean()
        # d(loss_map.mean())/d(img): the loss VJP writes [H, W, 4] with a zero
        # alpha channel, which is the render's gradient
        v_img = image_loss_backward_raw(rgb, gt_packed, loss_cfg, self._uniform_chain(h, w, img.device))
        n = t.shape[0]
        v_t = torch.empty_like(t)
        v_c = torch.empty_like(s)
        v_o = torch.empty_like(o)
        v_r = torch.empty((n,), dtype=torch.float32, device=t.device)
        flags = _lib.FLAG_REFINE_WEIGHT if cfg.compute_refine_weight else 0
        bg = (ctypes.c_float * 3)(*[float(x) for x in self.background])
        with torch.cuda.device(t.device):
            ctx = context()
            rt_c, ro_c = rt.detach().contiguous(), ro.detach().contiguous()
            ctx.check(lib().bh_render_backward(ctx.handle, out.state.handle, ptr(img), ptr(out.aux.tile_offsets),
                                               bg, ptr(rt_c), ptr(s), ptr(ro_c), ptr(v_img), flags, ptr(v_t),
                                               ptr(v_c), ptr(v_o), ptr(v_r)), "render_backward")
        if splats.min_scale is not None:
            v_t, v_o = torch.autograd.grad([rt, ro], [t_leaf, o_leaf], [v_t, v_o])
        # optimizer (train.rs:966-1051); the per-column scales live on the device
        lr_t = (cfg.lr_mean,) * 3 + (cfg.lr_rotation,) * 4 + (cfg.lr_scale,) * 3
        if self._lr_t != lr_t:
            self.state_transforms.scaling = torch.tensor(lr_t, dtype=torch.float32, device=t.device)
            self._lr_t = lr_t
        if self.state_sh.scaling is None:
            sc = [1.0] + [1.0 / cfg.lr_coeffs_sh_scale] * (s.shape[1] - 1)
            self.state_sh.scaling = torch.tensor([v for v in sc for _ in range(3)], dtype=torch.float32,
                                                 device=t.device)
        with torch.no_grad():
            self.optim.step(1.0, t.data, v_t, self.state_transforms)
            self.optim.step(cfg.lr_coeffs_dc, s.data, v_c, self.state_sh)
            self.optim.step(cfg.lr_opac, o.data, v_o, self.state_opac)
        res = {"loss": loss, "num_visible": out.aux.num_visible, "refine_weight": v_r}
        if record_grads:
            res.update(v_transforms=v_t, v_coeffs=v_c, v_raw_opac=v_o, img=img)
        out.state.release()
        return res

