"""ctypes binding of libfhip.so (the C ABI declared in include/fhip.h).

The library is loaded from this package directory.  There is no fallback: if it is missing the
import of a kernel fails loudly with the build command to run.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfhip.so")

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_BUDGET, ERR_STATE = 0, -1, -2, -3, -4, -5
INT8, FP16, FP32, INT32, INT64, BF16, FP8E4M3, FP8E5M2 = 1, 3, 4, 5, 6, 11, 12, 13
BIAS_NONE, BIAS_VECTOR, BIAS_MATRIX = 0, 1, 2
LAYOUT_KN, LAYOUT_NK = 0, 1
I8_MATMUL, I8_FC, I8_GEMM = 0, 1, 2
NCHW, NHWC = 0, 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float
_INT = ctypes.c_int
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_PP = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); kept in step with include/fhip.h
SIGNATURES = {
    "fhip_version": (_INT, []),
    "fhip_context_create": (_INT, [_INT, _PP]),
    "fhip_context_destroy": (_INT, [_P]),
    "fhip_context_set_stream": (_INT, [_P, _P]),
    "fhip_context_stream": (_P, [_P]),
    "fhip_set_workspace_limit": (_INT, [_P, _SZ]),
    "fhip_set_weight_cache_limit": (_INT, [_P, _SZ]),
    "fhip_weight_cache_bytes": (_INT, [_P, ctypes.POINTER(_SZ)]),
    "fhip_synchronize": (_INT, [_P]),
    "fhip_last_error": (ctypes.c_char_p, [_P]),
    "fhip_last_backend": (ctypes.c_char_p, [_P]),
    "fhip_memory_alloc": (_INT, [_P, _SZ, _PP]),
    "fhip_memory_free": (_INT, [_P, _P]),
    "fhip_memory_upload": (_INT, [_P, _P, _P, _SZ]),
    "fhip_memory_download": (_INT, [_P, _P, _P, _SZ]),
    "fhip_memory_copy": (_INT, [_P, _P, _P, _SZ]),
    "fhip_weight_prepare": (_INT, [_P, _P, _INT, _I64, _I64, _INT, _P, _I64, _P, _I64, _U64, _PP]),
    "fhip_weight_prepare_host": (_INT, [_P, _P, _INT, _I64, _I64, _INT, _P, _I64, _P, _I64, _U64, _PP]),
    "fhip_conv_weight_prepare": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _I32, _P, _I64, _P, _I64, _U64, _PP]),
    "fhip_weight_release": (_INT, [_P]),
    "fhip_weight_matches": (_INT, [_P, _P, _U64]),
    "fhip_cast": (_INT, [_P, _INT, _P, _F, _I64, _INT, _P, _F]),
    "fhip_fp8_linear": (_INT, [_P, _INT, _P, _F, _I64, _P, _F, _P, _F, _INT, _F, _F, _INT, _P, _F]),
    "fhip_i8_linear": (_INT, [_P, _INT, _P, _F, _I32, _I64, _P, _P, _INT, _I32, _F, _F, _P, _F, _I32]),
    "fhip_i8_linear_ex": (_INT, [_P, _INT, _P, _F, _I32, _I64, _P, _P, _INT, _I32, _F, _F, _INT, _P, _F, _I32, _F,
                                 _I32]),
    "fhip_i8_conv2d": (_INT, [_P, _P, _I64, _I64, _I64, _I64, _INT, _F, _I32, _P, _P, _I32, _I32, _I32, _I32, _I32,
                              _I32, _I32, _P, _I64, _I64, _F, _I32]),
    "fhip_quantize_linear": (_INT, [_P, _INT, _P, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "fhip_dequantize_linear": (_INT, [_P, _P, _I64, _I64, _I64, _P, _P, _I64, _INT, _P]),
    "fhip_bf16_gemv_argmax": (_INT, [_P, _P, _I64, _I64, _P, _I64, _P, _P]),
    "fhip_bf16_gemv_argmax_noalloc": (_INT, [_P, _P, _I64, _I64, _P, _I64, _P, _P]),
    "fhip_fp8_gemv_argmax": (_INT, [_P, _INT, _P, _F, _I64, _I64, _P, _F, _I64, _F, _P]),
    "fhip_capture_begin": (_INT, [_P]),
    "fhip_capture_end": (_INT, [_P, _PP]),
    "fhip_graph_launch": (_INT, [_P, _P]),
    "fhip_graph_destroy": (_INT, [_P]),
}

_lib = None


class FhipError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"fhip error {code}: {message}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m infer_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib
