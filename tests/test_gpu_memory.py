"""Tensor memory entry points (fhip_memory_*), which the HIP BackendContext uses to keep device replicas
of a session's tensors (the CUDA runtime's AcquireTensorDevice / SyncTensorToHost, src/kernel/cuda/
runtime.h:106-145): bytes survive upload -> device copy -> download unchanged, a kernel reads an uploaded
replica, and allocation or host transfers are refused while a capture is open.
"""
import ctypes

import numpy as np
import pytest
import torch

from infer_amd import _lib as L
from oracle import pyoracle as po
from tests.common import rng

pytestmark = pytest.mark.gpu


def _alloc(ctx, n):
    p = ctypes.c_void_p()
    assert ctx.lib.fhip_memory_alloc(ctx.handle, n, ctypes.byref(p)) == L.OK, ctx.lib.fhip_last_error(ctx.handle)
    return p


@pytest.mark.parametrize("nbytes", [1, 4097, 3 << 20])
def test_memory_upload_copy_download_roundtrip(ctx, nbytes):
    lib, h = ctx.lib, ctx.handle
    src = rng(nbytes).integers(0, 256, nbytes, dtype=np.uint8)
    a, b = _alloc(ctx, nbytes), _alloc(ctx, nbytes)
    try:
        assert lib.fhip_memory_upload(h, a, src.ctypes.data, nbytes) == L.OK
        assert lib.fhip_memory_copy(h, b, a, nbytes) == L.OK
        back = np.zeros(nbytes, dtype=np.uint8)
        assert lib.fhip_memory_download(h, back.ctypes.data, b, nbytes) == L.OK
        assert np.array_equal(back, src)
    finally:
        assert lib.fhip_memory_free(h, a) == L.OK
        assert lib.fhip_memory_free(h, b) == L.OK


def test_memory_replica_feeds_a_kernel(ctx):
    """A Cast reads an uploaded replica and writes a replica that is downloaded: same bytes as the oracle."""
    lib, h = ctx.lib, ctx.handle
    x = (rng(5).standard_normal(1000) * 3).astype(np.float32)
    dst = _alloc(ctx, x.nbytes)
    out = _alloc(ctx, x.size)
    try:
        assert lib.fhip_memory_upload(h, dst, x.ctypes.data, x.nbytes) == L.OK
        assert lib.fhip_cast(h, L.FP32, dst, 1.0, x.size, L.FP8E4M3, out, 0.25) == L.OK
        got = np.zeros(x.size, dtype=np.uint8)
        assert lib.fhip_memory_download(h, got.ctypes.data, out, x.size) == L.OK
        assert np.array_equal(got, po.cast_to_fp8(po.FP32, x, po.FP8E4M3, 0.25))
    finally:
        lib.fhip_memory_free(h, dst)
        lib.fhip_memory_free(h, out)


def test_memory_calls_refused_during_capture(ctx):
    lib, h = ctx.lib, ctx.handle
    a, a2 = _alloc(ctx, 256), _alloc(ctx, 256)
    host = np.zeros(256, dtype=np.uint8)
    b = ctypes.c_void_p()
    with torch.cuda.stream(ctx.stream):
        ctx.capture_begin()
        try:
            assert lib.fhip_memory_alloc(h, 256, ctypes.byref(b)) == L.ERR_STATE
            assert lib.fhip_memory_upload(h, a, host.ctypes.data, 256) == L.ERR_STATE
            assert lib.fhip_memory_download(h, host.ctypes.data, a, 256) == L.ERR_STATE
            assert lib.fhip_memory_free(h, a) == L.ERR_STATE
            assert lib.fhip_memory_copy(h, a2, a, 256) == L.OK  # stream-ordered: captured
        finally:
            g = ctx.capture_end()
            ctx.graph_destroy(g)
    assert lib.fhip_memory_free(h, a) == L.OK
    assert lib.fhip_memory_free(h, a2) == L.OK
    assert lib.fhip_memory_alloc(h, 0, ctypes.byref(b)) == L.OK and not b.value
    assert lib.fhip_memory_free(h, None) == L.OK
