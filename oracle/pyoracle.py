"""ctypes bindings for the parity oracle (liboracle.so) and the reference build (_ref/libfeather_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker.  The shipped package (infer_amd) never imports this module.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libfeather_ref.so")

INT8, FP16, FP32, INT32, INT64, BF16, FP8E4M3, FP8E5M2 = 1, 3, 4, 5, 6, 11, 12, 13
BIAS_NONE, BIAS_VECTOR, BIAS_MATRIX = 0, 1, 2
I8_MATMUL, I8_FC, I8_GEMM = 0, 1, 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float
_INT = ctypes.c_int


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _sig(lib, name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


_lib = None
_ref = None


def lib():
    """Load liboracle.so (built by `make -C oracle`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle`")
        L = ctypes.CDLL(ORACLE_SO)
        _sig(L, "fo_fp8_encode", ctypes.c_uint8, _INT, _F)
        _sig(L, "fo_fp8_decode", _F, _INT, ctypes.c_uint8)
        _sig(L, "fo_bf16_encode", ctypes.c_uint16, _F)
        _sig(L, "fo_fp16_encode", ctypes.c_uint16, _F)
        _sig(L, "fo_fp16_decode", _F, ctypes.c_uint16)
        _sig(L, "fo_fp16_encode_cast", ctypes.c_uint16, _F)
        _sig(L, "fo_fp16_encode_bits_range", None, _INT, ctypes.c_uint32, _I64, _P)
        _sig(L, "fo_bf16_plain_encode_bits_range", None, ctypes.c_uint32, _I64, _P)
        _sig(L, "fo_fp8_encode_array", None, _INT, _P, _P, _I64)
        _sig(L, "fo_bf16_encode_array", None, _P, _P, _I64)
        _sig(L, "fo_fp8_encode_bits_range", None, _INT, ctypes.c_uint32, _I64, _P)
        _sig(L, "fo_bf16_encode_bits_range", None, ctypes.c_uint32, _I64, _P)
        _sig(L, "fo_cast_to_fp8", _INT, _INT, _P, _I64, _INT, _F, _P)
        _sig(L, "fo_cast_from_fp8", _INT, _INT, _P, _F, _I64, _INT, _P)
        _sig(L, "fo_fp8_matmul", _INT, _INT, _P, _F, _P, _F, _I64, _I64, _I64, _P, _F)
        _sig(L, "fo_fp8_gemm", _INT, _INT, _P, _F, _P, _F, _INT, _P, _F, _INT, _F, _F, _I64, _I64, _I64, _P, _F)
        _sig(L, "fo_fp8_fc", _INT, _INT, _P, _F, _P, _F, _P, _F, _INT, _I64, _I64, _I64, _P, _F)
        _sig(L, "fo_fp8_gemm_f32", _INT, _INT, _P, _F, _P, _F, _INT, _I64, _I64, _I64, _P)
        _sig(L, "fo_i8_linear", _INT, _INT, _P, _F, _I32, _P, _INT, _P, _I64, _P, _I64, _P, _INT, _F, _F,
             _I64, _I64, _I64, _P, _F, _I32, _P)
        _sig(L, "fo_i8_conv2d", _INT, _P, _I64, _I64, _I64, _I64, _INT, _F, _I32, _P, _I64, _I64, _I64,
             _P, _I64, _P, _I64, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _I64, _I64, _F, _I32)
        _sig(L, "fo_quantize_linear", _INT, _INT, _P, _P, _INT, _P, _I64, _P, _I64, _I64, _P)
        _sig(L, "fo_dequantize_linear", _INT, _P, _P, _INT, _P, _I64, _P, _I64, _I64, _INT, _P)
        _sig(L, "fo_bf16_gemm_argmax", _I64, _P, _P, _I64, _I64, _P)
        _sig(L, "fo_fp8_gemm_argmax", _I64, _INT, _P, _F, _P, _F, _I64, _I64, _F)
        _sig(L, "fo_set_threads", _INT, _INT)
        _lib = L
    return _lib


def ref_available():
    return os.path.exists(REF_SO)


def ref():
    """Load the reference build (oracle/_ref/libfeather_ref.so, `make -C oracle ref`)."""
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_SO} missing: run `make -C oracle ref` where the Feather tree exists")
        R = ctypes.CDLL(REF_SO)
        _sig(R, "ref_max_threads", _INT)
        _sig(R, "ref_fp8_encode_bits_range", None, _INT, ctypes.c_uint32, _I64, _P)
        _sig(R, "ref_fp8_decode", _F, _INT, ctypes.c_uint8)
        _sig(R, "ref_bf16_encode_bits_range", None, ctypes.c_uint32, _I64, _P)
        _sig(R, "ref_fp16_encode_bits_range", None, _INT, ctypes.c_uint32, _I64, _P)
        _sig(R, "ref_bf16_plain_encode_bits_range", None, ctypes.c_uint32, _I64, _P)
        _sig(R, "ref_fp16_decode", _F, _INT, ctypes.c_uint16)
        _sig(R, "ref_quantize_int8_values", None, _P, _I64, _F, _I32, _P)
        _sig(R, "ref_requantize", _INT, _P, _I64, _I64, _F, _P, _I64, _F, _I32, _P)
        _sig(R, "ref_fp8_linear", _INT, _INT, _P, _F, _P, _F, _INT, _P, _F, _INT, _F, _F, _I64, _I64, _I64, _P, _F)
        _sig(R, "ref_fp8_packed_create", _P, _INT, _P, _INT, _I64, _I64)
        _sig(R, "ref_fp8_packed_compute", _INT, _P, _P, _F, _F, _I64, _P, _F)
        _sig(R, "ref_fp8_packed_argmax", _INT, _P, _P, _F, _F, _F, ctypes.POINTER(ctypes.c_int64))
        _sig(R, "ref_fp8_packed_destroy", None, _P)
        _sig(R, "ref_bf16_argmax_create", _P, _P, _I64, _I64)
        _sig(R, "ref_bf16_argmax_compute", _INT, _P, _P, ctypes.POINTER(ctypes.c_int64))
        _sig(R, "ref_bf16_argmax_destroy", None, _P)
        _sig(R, "ref_i8_gemm_create", _P, _P, _F, _I32, _I64, _I64, _P, _P, _I64, _I64, _P, _F, _F, _F, _I32)
        _sig(R, "ref_i8_gemm_compute", _INT, _P)
        _sig(R, "ref_i8_gemm_output", None, _P, _P)
        _sig(R, "ref_i8_gemm_destroy", None, _P)
        _sig(R, "ref_i8_conv2d_create", _P, _P, _I64, _I64, _I64, _I64, _INT, _F, _I32, _P, _I64, _I64, _I64, _I32,
             _P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I64, _I64, _F, _I32)
        _sig(R, "ref_i8_conv2d_compute", _INT, _P)
        _sig(R, "ref_i8_conv2d_output", None, _P, _P)
        _sig(R, "ref_i8_conv2d_destroy", None, _P)
        _sig(R, "ref_has_avx_vnni", _INT)
        _sig(R, "ref_set_threads", None, _INT)
        _ref = R
    return _ref


# ---- numpy-level helpers ------------------------------------------------------------------

def fp8_encode(dtype, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().fo_fp8_encode_array(dtype, _ptr(x), _ptr(out), x.size)
    return out


def fp8_decode_table(dtype):
    return np.array([lib().fo_fp8_decode(dtype, c) for c in range(256)], dtype=np.float32)


def fp8_decode(dtype, codes):
    return fp8_decode_table(dtype)[np.asarray(codes, dtype=np.uint8)]


def bf16_encode(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().fo_bf16_encode_array(_ptr(x), _ptr(out), x.size)
    return out


def fp16_encode(x):
    x = np.asarray(x, np.float32)
    f = lib().fo_fp16_encode
    return np.array([f(float(v)) for v in x.reshape(-1)], dtype=np.uint16).reshape(x.shape)


def bf16_decode(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def cast_to_fp8(src_dtype, src, fp8_dtype, out_scale):
    src = np.ascontiguousarray(src)
    out = np.empty(src.shape, np.uint8)
    rc = lib().fo_cast_to_fp8(src_dtype, _ptr(src), src.size, fp8_dtype, out_scale, _ptr(out))
    assert rc == 0
    return out


def cast_from_fp8(fp8_dtype, codes, in_scale, dst_dtype):
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.empty(codes.shape, np.float32 if dst_dtype == FP32 else np.uint16)
    rc = lib().fo_cast_from_fp8(fp8_dtype, _ptr(codes), in_scale, codes.size, dst_dtype, _ptr(out))
    assert rc == 0
    return out


def fp8_gemm(dtype, a, sa, b, sb, trans_b, s_out, bias=None, s_bias=1.0, bias_kind=BIAS_NONE,
             alpha=1.0, beta=1.0):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    m, k = a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    out = np.empty((m, n), np.uint8)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.uint8)
    rc = lib().fo_fp8_gemm(dtype, _ptr(a), sa, _ptr(b), sb, int(trans_b), _ptr(bias), s_bias, bias_kind,
                           alpha, beta, m, k, n, _ptr(out), s_out)
    assert rc == 0
    return out


def fp8_matmul(dtype, a, sa, b, sb, s_out):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.uint8)
    rc = lib().fo_fp8_matmul(dtype, _ptr(a), sa, _ptr(b), sb, m, k, n, _ptr(out), s_out)
    assert rc == 0
    return out


def fp8_sums(dtype, a, sa, b, sb, trans_b):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    m, k = a.shape
    n = b.shape[0] if trans_b else b.shape[1]
    out = np.empty((m, n), np.float32)
    rc = lib().fo_fp8_gemm_f32(dtype, _ptr(a), sa, _ptr(b), sb, int(trans_b), m, k, n, _ptr(out))
    assert rc == 0
    return out


def i8_linear(kind, a, s_a, zp_a, w, trans_b, w_scales, w_zps, bias, bias_kind, alpha, beta, s_out, zp_out,
              want_acc=False):
    """Returns (status, out int8 [M,N], acc int32 [M,N] or None)."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = a.shape
    n = w.shape[0] if trans_b else w.shape[1]
    ws = np.ascontiguousarray(np.atleast_1d(w_scales), dtype=np.float32)
    wz = None if w_zps is None else np.ascontiguousarray(np.atleast_1d(w_zps), dtype=np.int32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.int32)
    out = np.zeros((m, n), np.int8)
    acc = np.zeros((m, n), np.int32) if want_acc else None
    rc = lib().fo_i8_linear(kind, _ptr(a), s_a, zp_a, _ptr(w), int(trans_b), _ptr(ws), ws.size, _ptr(wz),
                            0 if wz is None else wz.size, _ptr(bias), bias_kind, alpha, beta, m, k, n,
                            _ptr(out), s_out, zp_out, _ptr(acc))
    return rc, out, acc


def i8_conv2d(x, s_in, zp_in, w, w_scales, bias, stride, pad, s_out, zp_out, dilation=(1, 1), group=1,
              layout=0, w_zps=None):
    """x NCHW (layout 0) or NHWC (layout 1) int8; w [OC, IC/g, KH, KW]. Returns (status, out)."""
    x = np.ascontiguousarray(x, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    if layout == 0:
        n, c, h, wd = x.shape
    else:
        n, h, wd, c = x.shape
    oc, _, kh, kw = w.shape
    sh, sw = (stride, stride) if np.isscalar(stride) else stride
    ph, pw = (pad, pad) if np.isscalar(pad) else pad
    dh, dw = dilation
    oh = (h + 2 * ph - dh * (kh - 1) - 1) // sh + 1
    ow = (wd + 2 * pw - dw * (kw - 1) - 1) // sw + 1
    ws = np.ascontiguousarray(np.atleast_1d(w_scales), dtype=np.float32)
    wz = None if w_zps is None else np.ascontiguousarray(np.atleast_1d(w_zps), dtype=np.int32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.int32)
    out = np.zeros((n, oc, oh, ow) if layout == 0 else (n, oh, ow, oc), np.int8)
    rc = lib().fo_i8_conv2d(_ptr(x), n, c, h, wd, layout, s_in, zp_in, _ptr(w), oc, kh, kw, _ptr(ws), ws.size,
                            _ptr(wz), 0 if wz is None else wz.size, _ptr(bias), sh, sw, ph, pw, dh, dw, group,
                            _ptr(out), oh, ow, s_out, zp_out)
    return rc, out


def quantize_linear(src_dtype, x, scales, zps, axis=-1):
    x = np.ascontiguousarray(x)
    dims = np.array(x.shape, dtype=np.int64)
    sc = np.ascontiguousarray(np.atleast_1d(scales), dtype=np.float32)
    zp = np.ascontiguousarray(np.atleast_1d(zps), dtype=np.int32)
    out = np.zeros(x.shape, np.int8)
    rc = lib().fo_quantize_linear(src_dtype, _ptr(x), _ptr(dims), len(x.shape), _ptr(sc), sc.size, _ptr(zp),
                                  zp.size, axis, _ptr(out))
    return rc, out


def dequantize_linear(q, scales, zps, dst_dtype=FP32, axis=-1):
    q = np.ascontiguousarray(q, dtype=np.int8)
    dims = np.array(q.shape, dtype=np.int64)
    sc = np.ascontiguousarray(np.atleast_1d(scales), dtype=np.float32)
    zp = np.ascontiguousarray(np.atleast_1d(zps), dtype=np.int32)
    out = np.zeros(q.shape, np.float32 if dst_dtype == FP32 else np.uint16)
    rc = lib().fo_dequantize_linear(_ptr(q), _ptr(dims), len(q.shape), _ptr(sc), sc.size, _ptr(zp), zp.size,
                                    axis, dst_dtype, _ptr(out))
    return rc, out


def bf16_gemm_argmax(a_bits, b_bits, want_logits=False):
    a_bits = np.ascontiguousarray(a_bits, dtype=np.uint16).reshape(-1)
    b_bits = np.ascontiguousarray(b_bits, dtype=np.uint16)
    v, k = b_bits.shape
    logits = np.empty(v, np.float32) if want_logits else None
    tok = lib().fo_bf16_gemm_argmax(_ptr(a_bits), _ptr(b_bits), k, v, _ptr(logits))
    return (tok, logits) if want_logits else tok


def fp8_gemm_argmax(dtype, a, sa, b, sb, s_out):
    a = np.ascontiguousarray(a, dtype=np.uint8).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    v, k = b.shape
    return lib().fo_fp8_gemm_argmax(dtype, _ptr(a), sa, _ptr(b), sb, k, v, s_out)
