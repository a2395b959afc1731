"""The C-ABI library: it loads without a GPU, exports every entry point that
include/brush_hip.h declares, and rejects bad arguments with status codes
instead of aborting (apps/brush-c/src/lib.rs:109-166 converts panics into exit
codes; this library never panics)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "brush_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(bh_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from brush_amd import _lib

    assert sorted(_lib.EXPORTED) == _declared()


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)
    from brush_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libbrush_hip.so not built")
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [name for name in _declared() if not hasattr(raw, name)]
    assert not missing, f"not exported: {missing}"


def test_null_arguments_return_status_codes():
    import torch  # noqa: F401
    from brush_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libbrush_hip.so not built")
    L = _lib.lib()
    null = ctypes.c_void_p(0)
    assert L.bh_ctx_create(0, None) == 1  # BH_ERR_INVALID_ARG
    assert L.bh_ctx_set_stream(null, null) == 1
    assert L.bh_radix_argsort(null, null, null, 0, 32, null, null) == 1
    assert L.bh_prefix_sum(null, null, null, 0) == 1
    assert L.bh_render_forward(null, None, null, null, null, null, 0, 0, 0, null, null, null, null, None) == 1
    assert L.bh_rasterize_backward(null, null, null, null, null, 0, null, 1, 1, null, 0, null) == 1
    assert L.bh_project_backward(null, None, null, null, null, null, null, 0, null, null, null, null) == 1
    assert L.bh_fwd_state_info(null, None) == 1
    assert L.bh_ply_decode_rows(null, null, 0, 4, 1, 1, 0, None, 1, null, null, null) == 1
    assert L.bh_ply_decode_compressed(null, null, 0, null, 0, null, 0, 1, 1, 0, None, null, null, null) == 1
    assert L.bh_ply_encode_rows(null, null, null, null, 1, 1, null) == 1
    assert L.bh_last_error(null) == b"null context"
    L.bh_fwd_state_release(null)
    L.bh_ctx_destroy(null)


def test_context_creation_reports_missing_device():
    import torch
    from brush_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libbrush_hip.so not built")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    st = _lib.lib().bh_ctx_create(0, ctypes.byref(h))
    assert st == 4 and not h.value  # BH_ERR_DEVICE
