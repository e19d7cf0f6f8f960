"""Execution capture (fhip_capture_* -> a HIP graph, BackendContext::Capture in the reference,
include/core/backend.h:43-96): a decode step captured once and replayed gives, on every replay, exactly
what the same calls give eagerly -- with the inputs rewritten and the device synchronised between
replays.  The step covers the fused FP8 decode linear, the BF16 LM-head argmax (its completion ticket
re-arms itself inside the graph), QuantizeLinear and the INT8 Gemm with its DequantizeLinear fused.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import fp8_tensor, rng

pytestmark = pytest.mark.gpu


def test_captured_decode_step_replays_match_eager(ctx):
    r = rng(90)
    k, n, v = 1024, 3584, 50021
    dtype = po.FP8E4M3
    w_nk, sw = fp8_tensor((r.standard_normal((n, k)) * 0.02).astype(np.float32), dtype)
    wf = ctx.prepare_weight(torch.from_numpy(w_nk).cuda(), dtype, k, n, 1, version=90)
    head = torch.from_numpy(po.bf16_encode((r.standard_normal((v, k)) * 0.02).astype(np.float32)).view(np.int16)).cuda()
    wq = torch.from_numpy(r.integers(-127, 128, (256, k)).astype(np.int8)).cuda()
    w8 = ctx.prepare_weight(wq, po.INT8, k, 256, 1, scales=r.uniform(1e-3, 1e-2, 256).astype(np.float32), version=91)

    x = torch.empty((1, k), dtype=torch.int16, device="cuda")      # bf16 activation row
    y = torch.empty((1, n), dtype=torch.int16, device="cuda")      # bf16 out of the FP8 linear
    tok = torch.empty(1, dtype=torch.int64, device="cuda")
    xf = torch.empty((4, k), dtype=torch.float32, device="cuda")   # fp32 rows for the INT8 chain
    xq = torch.empty((4, k), dtype=torch.int8, device="cuda")
    yf = torch.empty((4, 256), dtype=torch.float32, device="cuda")

    def step():
        ctx.fp8_linear(x, po.BF16, 0.0078125, 1, wf, sw, y, po.BF16, 0.0625)
        ctx.bf16_gemv_argmax(y[:, :k], head, tok)
        ctx.quantize_linear(xf, po.FP32, [0.03], [0], xq)
        ctx.i8_linear_ex(po.I8_FC, xq, 0.03, 0, 4, w8, yf, po.FP32, 0.5, 0, dq_scale=0.5,
                         dq_zp=0)

    def fill(seed):
        g = rng(seed)
        x.copy_(torch.from_numpy(po.bf16_encode(g.standard_normal((1, k)).astype(np.float32)).view(np.int16)))
        xf.copy_(torch.from_numpy(g.standard_normal((4, k)).astype(np.float32)))

    def snapshot():
        torch.cuda.synchronize()
        return y.cpu().numpy().copy(), int(tok.item()), xq.cpu().numpy().copy(), yf.cpu().numpy().copy()

    with torch.cuda.stream(ctx.stream):
        fill(0)
        step()  # eager warm-up grows the workspace before capture
        ctx.synchronize()
        ctx.capture_begin()
        step()
        # preparing a weight while capturing is refused (state error), and capture stays usable
        h = ctypes.c_void_p()
        assert ctx.lib.fhip_weight_prepare(ctx.handle, wq.data_ptr(), po.INT8, k, 256, 1,
                                           np.ones(1, np.float32).ctypes.data_as(ctypes.c_void_p), 1, None, 0, 5,
                                           ctypes.byref(h)) == -5
        g = ctx.capture_end()
        try:
            for seed in (1, 2, 3):
                fill(seed)
                step()
                eager = snapshot()
                fill(seed)
                ctx.graph_launch(g)
                replay = snapshot()
                assert np.array_equal(eager[0], replay[0]), seed
                assert eager[1] == replay[1], seed
                assert np.array_equal(eager[2], replay[2]), seed
                assert np.array_equal(eager[3], replay[3]), seed
                # the replay also equals a second replay of the same inputs (nothing left armed)
                ctx.graph_launch(g)
                again = snapshot()
                assert again[1] == replay[1] and np.array_equal(again[0], replay[0])
        finally:
            ctx.graph_destroy(g)
    wf.release()
    w8.release()


def test_graph_survives_workspace_growth():
    """A graph captured while the workspace was small keeps replaying correctly after an eager call grows
    the workspace: the buffer the graph was captured with stays allocated while the graph exists (the
    bf16-activation GEMM stages its FP8 codes in the workspace)."""
    from infer_amd.runtime import Context
    c = Context(0)
    r = rng(91)
    k, n = 1024, 512
    dtype = po.FP8E4M3
    w_nk, sw = fp8_tensor((r.standard_normal((n, k)) * 0.02).astype(np.float32), dtype)
    wt = c.prepare_weight(torch.from_numpy(w_nk).cuda(), dtype, k, n, 1, version=92)
    m_small, m_big = 64, 8192

    def bf16_rows(seed, m):
        g = rng(seed)
        return torch.from_numpy(po.bf16_encode(g.standard_normal((m, k)).astype(np.float32)).view(np.int16)).cuda()

    x = bf16_rows(1, m_small)
    y = torch.empty((m_small, n), dtype=torch.int16, device="cuda")
    xb, yb = bf16_rows(2, m_big), torch.empty((m_big, n), dtype=torch.int16, device="cuda")
    with torch.cuda.stream(c.stream):
        c.fp8_linear(x, po.BF16, 0.0078125, m_small, wt, sw, y, po.BF16, 0.0625)
        c.synchronize()
        eager = y.cpu().numpy().copy()
        c.capture_begin()
        c.fp8_linear(x, po.BF16, 0.0078125, m_small, wt, sw, y, po.BF16, 0.0625)
        g = c.capture_end()
        try:
            # grows the workspace from m_small * k to m_big * k bytes while the graph is alive
            c.fp8_linear(xb, po.BF16, 0.0078125, m_big, wt, sw, yb, po.BF16, 0.0625)
            big_first = None
            for _ in range(3):
                y.zero_()
                c.graph_launch(g)
                c.fp8_linear(xb, po.BF16, 0.0078125, m_big, wt, sw, yb, po.BF16, 0.0625)
                c.synchronize()
                assert np.array_equal(y.cpu().numpy(), eager)
                big = yb.cpu().numpy()
                if big_first is None:
                    big_first = big.copy()
                assert np.array_equal(big, big_first)
        finally:
            c.graph_destroy(g)
    # the retired buffer is freed with the last graph; the context keeps working
    with torch.cuda.stream(c.stream):
        c.fp8_linear(x, po.BF16, 0.0078125, m_small, wt, sw, y, po.BF16, 0.0625)
        c.synchronize()
    assert np.array_equal(y.cpu().numpy(), eager)
    wt.release()
    c.close()
