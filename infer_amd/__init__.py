"""MI355X (gfx950) backend for Feather's quantized linear hot path.

The kernels live in libfhip.so (C ABI: include/fhip.h); `infer_amd.runtime.Context` drives them
from Python.  The Feather-side C++ adapter (KernelBase subclasses registered for DeviceType::HIP and a
HipBackendContext) is in integration/.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
