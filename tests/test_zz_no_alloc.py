"""The allocation-free LM-head argmax (fhip_bf16_gemv_argmax_noalloc) against the allocating entry point
(fhip_bf16_gemv_argmax), both called through the C ABI: tokens and fp32 logits must be identical, on two
calls in a row (the second one smaller, so it runs on what the first left in the static scratch array),
and on every replay of a graph captured around it.  The allocating entry point is itself held to the
oracle by the argmax parity tests.
"""
import ctypes

import numpy as np
import pytest
import torch

from infer_amd import _lib as L
from oracle import pyoracle as po
from tests.common import SEEDS, rng

pytestmark = pytest.mark.gpu


def _head(seed, m, k, v):
    r = rng(seed)
    a = po.bf16_encode(r.standard_normal((m, k), dtype=np.float32))
    w = po.bf16_encode(r.standard_normal((v, k), dtype=np.float32) * np.float32(0.02))
    return (torch.from_numpy(a.view(np.int16)).cuda(), torch.from_numpy(w.view(np.int16)).cuda())


def _call(ctx, fn, a, w, tokens, logits):
    m, k = a.shape
    v = w.shape[0]
    rc = fn(ctx.handle, a.data_ptr(), m, k, w.data_ptr(), v, tokens.data_ptr(),
            logits.data_ptr() if logits is not None else None)
    assert rc == L.OK, (rc, ctx.lib.fhip_last_error(ctx.handle))


def _both(ctx, a, w):
    m, v = a.shape[0], w.shape[0]
    out = {}
    for name in ("fhip_bf16_gemv_argmax", "fhip_bf16_gemv_argmax_noalloc"):
        tok = torch.full((m,), -7, dtype=torch.int64, device="cuda")
        lg = torch.full((m, v), float("nan"), dtype=torch.float32, device="cuda")
        with torch.cuda.stream(ctx.stream):
            _call(ctx, getattr(ctx.lib, name), a, w, tok, lg)
            ctx.synchronize()
        out[name] = (tok.cpu().numpy(), lg.cpu().numpy())
    return out["fhip_bf16_gemv_argmax"], out["fhip_bf16_gemv_argmax_noalloc"]


def test_noalloc_argmax_matches_allocating_entry_point_twice(ctx):
    # first call: the C5 head at M=8 (MFMA kernel); second call smaller: M=1 (GEMV kernel), V=32003
    for (m, v), seed in (((8, 151936), SEEDS[5] + 21), ((1, 32003), SEEDS[5] + 22)):
        print(f"noalloc argmax m={m} v={v} seed={seed:#x}", flush=True)
        a, w = _head(seed, m, 1024, v)
        (t_ref, l_ref), (t_got, l_got) = _both(ctx, a, w)
        assert np.array_equal(t_got, t_ref), (t_got, t_ref)
        assert np.array_equal(l_got.view(np.uint32), l_ref.view(np.uint32))
        assert ctx.lib.fhip_last_backend(ctx.handle) == b"bf16_gemv_argmax_noalloc"


def test_noalloc_argmax_empty_and_invalid(ctx):
    lib = ctx.lib
    assert lib.fhip_bf16_gemv_argmax_noalloc(ctx.handle, None, 0, 1024, None, 10, None, None) == L.OK
    assert lib.fhip_bf16_gemv_argmax_noalloc(ctx.handle, None, 1, 1024, None, 10, None, None) == L.ERR_INVALID
    a, w = _head(3, 17, 64, 100)
    tok = torch.empty(17, dtype=torch.int64, device="cuda")
    assert lib.fhip_bf16_gemv_argmax_noalloc(ctx.handle, a.data_ptr(), 17, 64, w.data_ptr(), 100, tok.data_ptr(),
                                             None) == L.ERR_UNSUPPORTED


def test_noalloc_argmax_captured_replays(ctx):
    m, k, v = 1, 1024, 151936
    a, w = _head(SEEDS[5] + 23, m, k, v)
    tok = torch.empty(m, dtype=torch.int64, device="cuda")
    fn = ctx.lib.fhip_bf16_gemv_argmax_noalloc
    with torch.cuda.stream(ctx.stream):
        _call(ctx, fn, a, w, tok, None)
        ctx.synchronize()
        ctx.capture_begin()
        _call(ctx, fn, a, w, tok, None)
        g = ctx.capture_end()
    try:
        for i in range(4):
            r = rng(700 + i)
            a.copy_(torch.from_numpy(po.bf16_encode(r.standard_normal((m, k), dtype=np.float32)).view(np.int16)))
            torch.cuda.synchronize()
            ref = torch.empty(m, dtype=torch.int64, device="cuda")
            with torch.cuda.stream(ctx.stream):
                _call(ctx, ctx.lib.fhip_bf16_gemv_argmax, a, w, ref, None)   # eager, allocating
                ctx.synchronize()
                tok.fill_(-1)
                ctx.synchronize()
                ctx.graph_launch(g)
                ctx.synchronize()
            assert tok.cpu().tolist() == ref.cpu().tolist(), (i, tok.cpu().tolist(), ref.cpu().tolist())
    finally:
        ctx.graph_destroy(g)
