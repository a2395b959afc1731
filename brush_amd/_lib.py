"""ctypes binding of libbrush_hip.so (include/brush_hip.h).

torch is imported first on purpose: torch ships its own HIP runtime under the
same soname (libamdhip64.so.7); loading it before libbrush_hip.so makes the
library bind to that runtime, so torch tensors and this library share one HIP
context.  There is no CPU fallback: without the built library every call
raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede loading libbrush_hip.so)

HERE = os.path.dirname(os.path.abspath(__file__))
# BH_LIB_PATH selects another build of the same sources (the sanitizer build
# of the host code, tests/test_sanitizers.py)
LIB_PATH = os.environ.get("BH_LIB_PATH") or os.path.join(HERE, "libbrush_hip.so")

OK = 0
STATUS_NAMES = {
    0: "BH_OK", 1: "BH_ERR_INVALID_ARG", 2: "BH_ERR_SHAPE", 3: "BH_ERR_OOM",
    4: "BH_ERR_DEVICE", 5: "BH_ERR_INTERNAL", 6: "BH_ERR_NOT_FINITE",
}

FLAG_BWD_INFO = 1
FLAG_SMOOTH_CUTOFF = 2
FLAG_RENDER_DEPTH = 4
FLAG_MIP = 8
FLAG_REFINE_WEIGHT = 16
FLAG_TILE_16X8 = 32

DEBUG_POISON = 1
DEBUG_VALIDATE = 2
DEBUG_EXACT_SIZES = 4
DEBUG_KEEP_LANES = 8

PROJECTED_LANES = 10
COMPACT_GRAD_LANES = 11
TILE_WIDTH = 16

# Every symbol include/brush_hip.h declares (checked by the CPU test suite).
EXPORTED = [
    "bh_ctx_create", "bh_ctx_destroy", "bh_ctx_set_stream", "bh_last_error", "bh_ctx_set_timing",
    "bh_ctx_set_timing_filter",
    "bh_ctx_read_timings", "bh_ctx_reset_timings", "bh_ctx_workspace_bytes", "bh_ctx_release_workspace",
    "bh_ctx_set_debug",
    "bh_radix_argsort", "bh_radix_argsort_noalloc",
    "bh_prefix_sum", "bh_get_tile_offsets", "bh_render_forward", "bh_fwd_state_info", "bh_fwd_state_backward_lanes",
    "bh_fwd_state_release", "bh_rasterize_backward", "bh_render_backward", "bh_project_backward",
    "bh_image_loss_forward", "bh_image_loss_backward", "bh_adam_scaled_step", "bh_copy_to_host",
    "bh_copy_to_device", "bh_copy_device", "bh_device_alloc", "bh_device_free", "bh_synchronize",
    "bh_ply_decode_rows", "bh_ply_decode_compressed", "bh_ply_encode_rows",
]


class BrushHipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class Uniforms(ctypes.Structure):
    """bh_project_uniforms."""

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

    @staticmethod
    def from_dict(d: dict) -> "Uniforms":
        u = Uniforms()
        for i, v in enumerate(d["viewmat"]):
            u.viewmat[i] = float(v)
        for k in ("half_max_render_fov", "fx", "fy", "cx", "cy", "lim_pos_x", "lim_pos_y", "lim_neg_x", "lim_neg_y"):
            setattr(u, k, float(d[k]))
        for i in range(3):
            u.camera_pos[i] = float(d["camera_pos"][i])
        for k in ("img_w", "img_h", "tile_bw", "tile_bh", "sh_degree", "total_splats", "num_visible"):
            setattr(u, k, int(d.get(k, 0)))
        u.camera_model = int(d.get("camera_model", 0))
        for i, v in enumerate(d.get("camera_params", ())):
            u.camera_params[i] = float(v)
        return u

    def to_dict(self) -> dict:
        return dict(
            viewmat=[float(x) for x in self.viewmat],
            half_max_render_fov=self.half_max_render_fov,
            fx=self.fx, fy=self.fy, cx=self.cx, cy=self.cy,
            lim_pos_x=self.lim_pos_x, lim_pos_y=self.lim_pos_y,
            lim_neg_x=self.lim_neg_x, lim_neg_y=self.lim_neg_y,
            camera_pos=[float(x) for x in self.camera_pos],
            img_w=self.img_w, img_h=self.img_h, tile_bw=self.tile_bw, tile_bh=self.tile_bh,
            sh_degree=self.sh_degree, total_splats=self.total_splats, num_visible=self.num_visible,
            camera_model=self.camera_model, camera_params=[float(x) for x in self.camera_params],
        )


class FwdInfo(ctypes.Structure):
    """bh_fwd_info."""

    _fields_ = [
        ("num_splats", ctypes.c_uint32),
        ("num_visible", ctypes.c_uint32),
        ("num_intersections", ctypes.c_uint32),
        ("num_tiles", ctypes.c_uint32),
        ("tile_bw", ctypes.c_uint32), ("tile_bh", ctypes.c_uint32),
        ("img_w", ctypes.c_uint32), ("img_h", ctypes.c_uint32),
        ("sh_degree", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("uniforms", Uniforms),
        ("projected", ctypes.c_void_p),
        ("global_from_compact_gid", ctypes.c_void_p),
        ("depths", ctypes.c_void_p),
        ("intersect_counts", ctypes.c_void_p),
        ("cum_tiles_hit", ctypes.c_void_p),
        ("tile_id_from_isect", ctypes.c_void_p),
        ("compact_gid_from_isect", ctypes.c_void_p),
        ("tile_offsets_pre", ctypes.c_void_p),
    ]


class ImageLossConfig(ctypes.Structure):
    """bh_image_loss_config (include/brush_hip.h)."""

    _fields_ = [("l1_weight", ctypes.c_float), ("ssim_weight", ctypes.c_float), ("composite", ctypes.c_uint32),
                ("background", ctypes.c_float * 3), ("mask", ctypes.c_uint32)]


class AdamConfig(ctypes.Structure):
    """bh_adam_config (include/brush_hip.h)."""

    _fields_ = [("beta_1", ctypes.c_float), ("beta_2", ctypes.c_float), ("epsilon", ctypes.c_float)]


PLY_CONST, PLY_I8, PLY_U8, PLY_I16, PLY_U16, PLY_I32, PLY_U32, PLY_F32, PLY_F64 = range(9)
PLY_OP_PLAIN, PLY_OP_COLOR = 0, 1
PLY_BIG_ENDIAN = 1


class PlyColumn(ctypes.Structure):
    """bh_ply_column (include/brush_hip.h)."""

    _fields_ = [("offset", ctypes.c_uint32), ("type", ctypes.c_uint16), ("op", ctypes.c_uint16),
                ("konst", ctypes.c_float)]


class PlyCompressedLayout(ctypes.Structure):
    """bh_ply_compressed_layout (include/brush_hip.h)."""

    _fields_ = [("vertex_row_bytes", ctypes.c_uint32), ("position_offset", ctypes.c_uint32),
                ("scale_offset", ctypes.c_uint32), ("rotation_offset", ctypes.c_uint32),
                ("color_offset", ctypes.c_uint32), ("sh_row_bytes", ctypes.c_uint32),
                ("sh_rest_count", ctypes.c_uint32), ("sh_offsets", ctypes.c_uint16 * 72)]


class KernelTiming(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 48), ("launches", ctypes.c_uint32), ("total_ms", ctypes.c_double)]


_lib = None


def lib() -> ctypes.CDLL:
    """Loads libbrush_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} not found: build it with `python -m brush_amd.build` "
                           "(there is no CPU fallback for the rasterizer)")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    U32 = ctypes.c_uint32
    U64 = ctypes.c_uint64
    I = ctypes.c_int
    S = ctypes.c_int  # bh_status
    PP = ctypes.POINTER(ctypes.c_void_p)
    UP = ctypes.POINTER(Uniforms)
    sig = {
        "bh_ctx_create": (S, [I, PP]),
        "bh_ctx_destroy": (None, [P]),
        "bh_ctx_set_stream": (S, [P, P]),
        "bh_last_error": (ctypes.c_char_p, [P]),
        "bh_ctx_set_timing": (S, [P, I]),
        "bh_ctx_set_timing_filter": (S, [P, ctypes.c_char_p]),
        "bh_ctx_read_timings": (S, [P, ctypes.POINTER(KernelTiming), I, ctypes.POINTER(I)]),
        "bh_ctx_reset_timings": (S, [P]),
        "bh_ctx_workspace_bytes": (U64, [P]),
        "bh_ctx_set_debug": (S, [P, U32]),
        "bh_ctx_release_workspace": (S, [P]),
        "bh_radix_argsort": (S, [P, P, P, U32, U32, P, P]),
        "bh_radix_argsort_noalloc": (S, [P, P, P, U32, U32, P, P]),
        "bh_prefix_sum": (S, [P, P, P, U32]),
        "bh_get_tile_offsets": (S, [P, P, U32, U32, P]),
        "bh_render_forward": (S, [P, UP, P, P, P, P, U32, U32, U32, P, P, P, P, PP]),
        "bh_fwd_state_info": (S, [P, ctypes.POINTER(FwdInfo)]),
        "bh_fwd_state_backward_lanes": (S, [P, PP]),
        "bh_fwd_state_release": (None, [P]),
        "bh_rasterize_backward": (S, [P, P, P, P, P, U32, P, U32, U32, P, U32, P]),
        "bh_render_backward": (S, [P, P, P, P, P, P, P, P, P, U32, P, P, P, P]),
        "bh_image_loss_forward": (S, [P, P, U32, U32, P, U32, U32, ctypes.POINTER(ImageLossConfig), P]),
        "bh_image_loss_backward": (S, [P, P, U32, U32, P, U32, U32, ctypes.POINTER(ImageLossConfig), P, P]),
        "bh_adam_scaled_step": (S, [P, P, P, P, P, P, U32, U32, U32, ctypes.c_float, U32,
                                    ctypes.POINTER(AdamConfig)]),
        "bh_project_backward": (S, [P, UP, P, P, P, P, P, U32, P, P, P, P]),
        "bh_ply_decode_rows": (S, [P, P, U64, U32, U64, U32, U32, ctypes.POINTER(PlyColumn), U32, P, P, P]),
        "bh_ply_decode_compressed": (S, [P, P, U64, P, U64, P, U64, U64, U32, U32,
                                         ctypes.POINTER(PlyCompressedLayout), P, P, P]),
        "bh_ply_encode_rows": (S, [P, P, P, P, U64, U32, P]),
        "bh_copy_to_host": (S, [P, P, P, U64]),
        "bh_copy_to_device": (S, [P, P, P, U64]),
        "bh_copy_device": (S, [P, P, P, U64]),
        "bh_device_alloc": (S, [P, PP, U64]),
        "bh_device_free": (S, [P, P]),
        "bh_synchronize": (S, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class Context:
    """One bh_ctx on one device; work is queued on torch's current stream."""

    def __init__(self, device: int = 0):
        L = lib()
        h = ctypes.c_void_p()
        st = L.bh_ctx_create(int(device), ctypes.byref(h))
        if st != OK:
            raise BrushHipError(st, f"bh_ctx_create(device={device}) failed")
        self.handle = h
        self.device = device
        self._stream = None

    def check(self, status: int, what: str = ""):
        if status != OK:
            msg = lib().bh_last_error(self.handle).decode(errors="replace")
            raise BrushHipError(status, f"{what}: {msg}" if what else msg)

    def use_current_stream(self):
        s = torch.cuda.current_stream(self.device).cuda_stream
        if s != self._stream:
            self.check(lib().bh_ctx_set_stream(self.handle, ctypes.c_void_p(s)), "bh_ctx_set_stream")
            self._stream = s

    def set_timing(self, enable: bool, only: str | None = None):
        """Bracket kernel launches with HIP events; ``only`` restricts this to
        the kernel of that name."""
        self.check(lib().bh_ctx_set_timing_filter(self.handle, (only or "").encode()), "bh_ctx_set_timing_filter")
        self.check(lib().bh_ctx_set_timing(self.handle, int(enable)), "bh_ctx_set_timing")

    def enable_timing(self, enable: bool):
        """Switches the event brackets on or off, keeping the kernel filter."""
        self.check(lib().bh_ctx_set_timing(self.handle, int(enable)), "bh_ctx_set_timing")

    def reset_timings(self):
        self.check(lib().bh_ctx_reset_timings(self.handle), "bh_ctx_reset_timings")

    def read_timings(self) -> dict:
        arr = (KernelTiming * 64)()
        n = ctypes.c_int(0)
        self.check(lib().bh_ctx_read_timings(self.handle, arr, 64, ctypes.byref(n)), "bh_ctx_read_timings")
        return {arr[i].name.decode(): (int(arr[i].launches), float(arr[i].total_ms)) for i in range(n.value)}

    def set_debug(self, poison: bool = False, validate: bool = False, exact_sizes: bool = False,
                  keep_lanes: bool = False):
        """BH_DEBUG_POISON: workspace blocks start as 0xFF bytes;
        BH_DEBUG_VALIDATE: NaN / Inf splat parameters (forward) and gradients
        (fused backward) raise BH_ERR_NOT_FINITE;
        BH_DEBUG_EXACT_SIZES: every forward waits for its counts before it
        queues the launches that depend on them (no plan from the previous
        forward);
        BH_DEBUG_KEEP_LANES: the fused backward keeps its per-splat gradient
        lanes in the forward state (ForwardState.backward_lanes)."""
        flags = ((DEBUG_POISON if poison else 0) | (DEBUG_VALIDATE if validate else 0)
                 | (DEBUG_EXACT_SIZES if exact_sizes else 0) | (DEBUG_KEEP_LANES if keep_lanes else 0))
        self.check(lib().bh_ctx_set_debug(self.handle, flags), "bh_ctx_set_debug")

    def workspace_bytes(self) -> int:
        return int(lib().bh_ctx_workspace_bytes(self.handle))

    def release_workspace(self) -> None:
        """Frees the cached workspace blocks no forward state holds."""
        self.check(lib().bh_ctx_release_workspace(self.handle), "bh_ctx_release_workspace")

    def __del__(self):
        try:
            if getattr(self, "handle", None):
                lib().bh_ctx_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


_contexts: dict[int, Context] = {}


def context(device: int | None = None) -> Context:
    """The process-wide context of ``device`` (default: torch's current device),
    bound to torch's current stream."""
    if device is None:
        device = torch.cuda.current_device()
    ctx = _contexts.get(device)
    if ctx is None:
        ctx = Context(device)
        _contexts[device] = ctx
    ctx.use_current_stream()
    return ctx


def ptr(t) -> ctypes.c_void_p:
    """Device pointer of a contiguous torch tensor (or None)."""
    if t is None:
        return ctypes.c_void_p(0)
    assert t.is_contiguous(), "tensor must be contiguous"
    return ctypes.c_void_p(t.data_ptr())
