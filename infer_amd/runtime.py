"""Python host side of the MI355X backend: a context object over the C ABI (include/fhip.h).

This mirrors Feather's BackendContext (include/core/backend.h:43-96) for Python callers: one
context per session with its own stream, device memory owned by torch tensors.  Every kernel call
is ordered after the work already queued on torch's current stream, and torch's current stream
waits for the kernel (event-based bridging, skipped when the current stream is the context's own,
as in `with torch.cuda.stream(ctx.stream)`).  PyTorch is used only for device memory and streams.
"""
import ctypes

import numpy as np
import torch

from . import _lib as L
from ._lib import FhipError

_c = ctypes


def _p(t):
    """Device pointer of a torch tensor (None -> NULL)."""
    return None if t is None else _c.c_void_p(t.data_ptr())


def _host_array(values, dtype):
    arr = np.ascontiguousarray(np.atleast_1d(np.asarray(values, dtype=dtype)))
    return arr, arr.ctypes.data_as(_c.c_void_p)


class Weight:
    """A prepared (re-laid-out) immutable weight held by a Context."""

    def __init__(self, ctx, handle, source, dtype, k, n):
        self.ctx, self.handle, self.source = ctx, handle, source
        self.dtype, self.k, self.n = dtype, k, n

    def release(self):
        if self.handle:
            L.lib().fhip_weight_release(self.handle)
            self.handle = None

    def matches(self, source, version):
        return bool(L.lib().fhip_weight_matches(self.handle, _p(source), version))


class Context:
    def __init__(self, device=0, stream=None):
        self.lib = L.lib()
        self.device = device
        h = _c.c_void_p()
        rc = self.lib.fhip_context_create(device, _c.byref(h))
        if rc != 0:
            raise FhipError(rc, "fhip_context_create failed")
        self.handle = h
        s = stream if stream is not None else torch.cuda.Stream(device)
        self._check(self.lib.fhip_context_set_stream(self.handle, _c.c_void_p(s.cuda_stream)))
        self.stream = s

    def _run(self, fn, *args, check=True):
        cur = torch.cuda.current_stream(self.device)
        bridged = cur.cuda_stream != self.stream.cuda_stream
        if bridged:
            self.stream.wait_stream(cur)
        rc = fn(self.handle, *args)
        if bridged:
            cur.wait_stream(self.stream)
        return self._check(rc) if check else rc

    # -- status -------------------------------------------------------------------------------
    def last_error(self):
        return self.lib.fhip_last_error(self.handle).decode()

    def last_backend(self):
        return self.lib.fhip_last_backend(self.handle).decode()

    def _check(self, rc):
        if rc != 0:
            raise FhipError(rc, self.last_error())
        return rc

    def close(self):
        if self.handle:
            self.lib.fhip_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        self._check(self.lib.fhip_synchronize(self.handle))

    def set_workspace_limit(self, nbytes):
        self._check(self.lib.fhip_set_workspace_limit(self.handle, nbytes))

    def set_weight_cache_limit(self, nbytes):
        self._check(self.lib.fhip_set_weight_cache_limit(self.handle, nbytes))

    def weight_cache_bytes(self):
        v = _c.c_size_t()
        self._check(self.lib.fhip_weight_cache_bytes(self.handle, _c.byref(v)))
        return v.value

    # -- weights --------------------------------------------------------------------------------
    def prepare_weight(self, w, dtype, k, n, layout, scales=None, zero_points=None, version=0, check=True):
        """w: device tensor holding [K,N] (layout KN) or [N,K] (layout NK) bytes."""
        sc, sp = (None, None) if scales is None else _host_array(scales, np.float32)
        zp, zpp = (None, None) if zero_points is None else _host_array(zero_points, np.int32)
        h = _c.c_void_p()
        rc = self._run(self.lib.fhip_weight_prepare, _p(w), dtype, k, n, layout, sp, 0 if sc is None else sc.size,
                       zpp, 0 if zp is None else zp.size, version, _c.byref(h), check=False)
        if rc != 0:
            if check:
                self._check(rc)
            return rc
        return Weight(self, h, w, dtype, k, n)

    def prepare_weight_host(self, w, dtype, k, n, layout, scales=None, zero_points=None, version=0, check=True):
        """w: host numpy array holding [K,N] (layout KN) or [N,K] (layout NK) bytes (e.g. a model file's
        mmapped weight); it must stay alive while the prepared weight is cached under its address."""
        w = np.ascontiguousarray(w)
        sc, sp = (None, None) if scales is None else _host_array(scales, np.float32)
        zp, zpp = (None, None) if zero_points is None else _host_array(zero_points, np.int32)
        h = _c.c_void_p()
        rc = self._run(self.lib.fhip_weight_prepare_host, w.ctypes.data_as(_c.c_void_p), dtype, k, n, layout, sp,
                       0 if sc is None else sc.size, zpp, 0 if zp is None else zp.size, version, _c.byref(h),
                       check=False)
        if rc != 0:
            if check:
                self._check(rc)
            return rc
        return Weight(self, h, w, dtype, k, n)

    def prepare_conv_weight(self, w, scales, zero_points=None, group=1, version=0, check=True):
        oc, icg, kh, kw = w.shape
        sc, sp = _host_array(scales, np.float32)
        zp, zpp = (None, None) if zero_points is None else _host_array(zero_points, np.int32)
        h = _c.c_void_p()
        rc = self._run(self.lib.fhip_conv_weight_prepare, _p(w), oc, icg, kh, kw, group, sp, sc.size, zpp,
                       0 if zp is None else zp.size, version, _c.byref(h), check=False)
        if rc != 0:
            if check:
                self._check(rc)
            return rc
        wt = Weight(self, h, w, L.INT8, icg * kh * kw, oc)
        wt.geometry = (oc, icg, kh, kw, group)
        return wt

    # -- kernels (return the status code; check=True raises on error) -------------------------
    def cast(self, src, src_dtype, src_scale, dst, dst_dtype, dst_scale, check=True):
        return self._run(self.lib.fhip_cast, src_dtype, _p(src), src_scale, src.numel(), dst_dtype, _p(dst), dst_scale, check=check)

    def fp8_linear(self, a, a_dtype, a_scale, m, w, w_scale, out, out_dtype, out_scale, bias=None, bias_scale=1.0,
                   bias_kind=L.BIAS_NONE, alpha=1.0, beta=1.0, check=True):
        return self._run(self.lib.fhip_fp8_linear, a_dtype, _p(a), a_scale, m, w.handle, w_scale, _p(bias), bias_scale,
                                      bias_kind, alpha, beta, out_dtype, _p(out), out_scale, check=check)

    def i8_linear(self, kind, a, s_a, zp_a, m, w, out, s_out, zp_out, bias=None, bias_kind=L.BIAS_NONE,
                  bias_abs_max=0, alpha=1.0, beta=1.0, check=True):
        return self._run(self.lib.fhip_i8_linear, kind, _p(a), s_a, zp_a, m, w.handle, _p(bias), bias_kind,
                                     bias_abs_max, alpha, beta, _p(out), s_out, zp_out, check=check)

    def i8_linear_ex(self, kind, a, s_a, zp_a, m, w, out, out_dtype, s_out, zp_out, dq_scale=1.0, dq_zp=0, bias=None,
                     bias_kind=L.BIAS_NONE, bias_abs_max=0, alpha=1.0, beta=1.0, check=True):
        """INT8 linear with the following DequantizeLinear fused (out_dtype FP32/FP16/BF16)."""
        return self._run(self.lib.fhip_i8_linear_ex, kind, _p(a), s_a, zp_a, m, w.handle, _p(bias), bias_kind,
                         bias_abs_max, alpha, beta, out_dtype, _p(out), s_out, zp_out, dq_scale, dq_zp, check=check)

    def i8_conv2d(self, x, layout, s_in, zp_in, w, out, s_out, zp_out, stride=(1, 1), pad=(0, 0), dilation=(1, 1),
                  bias=None, bias_abs_max=0, check=True):
        if layout == L.NCHW:
            n, c, h, wd = x.shape
            oh, ow = out.shape[2], out.shape[3]
        else:
            n, h, wd, c = x.shape
            oh, ow = out.shape[1], out.shape[2]
        return self._run(self.lib.fhip_i8_conv2d, _p(x), n, c, h, wd, layout, s_in, zp_in, w.handle, _p(bias),
                                     bias_abs_max, stride[0], stride[1], pad[0], pad[1], dilation[0], dilation[1],
                                     _p(out), oh, ow, s_out, zp_out, check=check)

    def quantize_linear(self, x, src_dtype, scales, zero_points, out, channels=1, inner=1, check=True):
        sc, sp = _host_array(scales, np.float32)
        zp, zpp = _host_array(zero_points, np.int32)
        return self._run(self.lib.fhip_quantize_linear, src_dtype, _p(x), x.numel(), channels, inner, sp, zpp, zp.size,
                                           _p(out), check=check)

    def dequantize_linear(self, q, scales, zero_points, out, dst_dtype, channels=1, inner=1, check=True):
        sc, sp = _host_array(scales, np.float32)
        zp, zpp = _host_array(zero_points, np.int32)
        return self._run(self.lib.fhip_dequantize_linear, _p(q), q.numel(), channels, inner, sp, zpp, zp.size,
                                             dst_dtype, _p(out), check=check)

    def bf16_gemv_argmax(self, a, w, tokens, logits=None, check=True):
        m, k = a.shape
        v = w.shape[0]
        return self._run(self.lib.fhip_bf16_gemv_argmax, _p(a), m, k, _p(w), v, _p(tokens), _p(logits), check=check)

    def fp8_gemv_argmax(self, dtype, a, a_scale, w, w_scale, out_scale, tokens, check=True):
        m, k = a.shape
        v = w.shape[0]
        return self._run(self.lib.fhip_fp8_gemv_argmax, dtype, _p(a), a_scale, m, k, _p(w), w_scale, v, out_scale,
                                           _p(tokens), check=check)

    # -- capture ---------------------------------------------------------------------------------
    def capture_begin(self):
        self._check(self.lib.fhip_capture_begin(self.handle))

    def capture_end(self):
        g = _c.c_void_p()
        self._check(self.lib.fhip_capture_end(self.handle, _c.byref(g)))
        return g

    def graph_launch(self, g):
        self._check(self.lib.fhip_graph_launch(self.handle, g))

    def graph_destroy(self, g):
        self.lib.fhip_graph_destroy(g)
