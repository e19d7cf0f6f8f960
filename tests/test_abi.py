"""The C-ABI library loads, exports every entry point include/fhip.h declares, and the Python binding's
signature table covers exactly those entry points.  No compute calls (no GPU needed)."""
import ctypes
import os
import re

from infer_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "fhip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(fhip_[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    names = declared()
    assert {"fhip_fp8_linear", "fhip_i8_linear", "fhip_i8_conv2d", "fhip_quantize_linear",
            "fhip_bf16_gemv_argmax", "fhip_weight_prepare", "fhip_capture_begin"} <= names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in sorted(declared()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    assert set(_lib.SIGNATURES) == declared()


def test_error_paths_without_device():
    lib = _lib.lib()
    assert lib.fhip_version() == 1
    assert lib.fhip_last_error(None) == b"null context"
    assert lib.fhip_context_destroy(None) == _lib.ERR_INVALID
    assert lib.fhip_synchronize(None) == _lib.ERR_INVALID
    assert lib.fhip_weight_release(None) == _lib.ERR_INVALID
    assert lib.fhip_fp8_linear(None, 12, None, 1.0, 1, None, 1.0, None, 1.0, 0, 1.0, 1.0, 12, None, 1.0) \
        == _lib.ERR_INVALID
    h = ctypes.c_void_p()
    # no usable device in this container: creation fails cleanly instead of crashing
    import torch
    if not torch.cuda.is_available():
        assert lib.fhip_context_create(0, ctypes.byref(h)) != 0
