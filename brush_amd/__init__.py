"""brush_amd — Brush's differentiable Gaussian-splat tile rasterizer on MI355X.

The compute path is libbrush_hip.so (hand-written gfx950 HIP kernels behind the
C ABI in include/brush_hip.h); this package is the host-side mirror of the
reference's render interface.  Importing it does not touch the GPU.
"""
from .camera import Camera, focal_to_fov, fov_to_focal, project_uniforms, tile_bounds  # noqa: F401

__all__ = ["Camera", "focal_to_fov", "fov_to_focal", "project_uniforms", "tile_bounds"]
