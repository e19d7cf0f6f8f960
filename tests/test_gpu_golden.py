"""The HIP path against the golden fixtures in tests/golden -- outputs of the reference's own code
(tests/golden/make_golden.py) -- through the C ABI.

Bar: Cast, QuantizeLinear and INT8 requantization bit-exact; FP8 linear within the FP8-output tolerance of
tests/common.py; argmax tokens exact.
"""
import os

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import fp8_linear_check

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
E4, E5 = po.FP8E4M3, po.FP8E5M2


def golden(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def codec_bits():
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    return (hi[:, None] | np.array([0x0000, 0x8000], np.uint32)[None, :]).reshape(-1)


@pytest.mark.parametrize("name,dtype", [("e4m3", E4), ("e5m2", E5)])
def test_cast_codec_matches_golden(ctx, name, dtype):
    g = golden("codec")
    x = dev(codec_bits().view(np.float32))
    codes = torch.empty(x.numel(), dtype=torch.uint8, device="cuda")
    ctx.cast(x, po.FP32, 1.0, codes, dtype, 1.0)
    assert np.array_equal(codes.cpu().numpy(), g[f"{name}_encode"])
    dec = torch.empty(256, dtype=torch.float32, device="cuda")
    ctx.cast(dev(np.arange(256, dtype=np.uint8)), dtype, 1.0, dec, po.FP32, 1.0)
    assert np.array_equal(dec.cpu().numpy().view(np.uint32), g[f"{name}_decode"].view(np.uint32))


def test_cast_bf16_matches_golden(ctx):
    g = golden("codec")
    x = dev(codec_bits().view(np.float32))
    out = torch.empty(x.numel(), dtype=torch.int16, device="cuda")
    ctx.cast(x, po.FP32, 1.0, out, po.BF16, 1.0)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), g["bf16_encode"])


def test_cast_fp16_matches_golden(ctx):
    """Cast to FP16 follows FloatToHalf (half away from zero), not DequantizeLinear's RNE encoder."""
    g = golden("codec")
    x = dev(codec_bits().view(np.float32))
    out = torch.empty(x.numel(), dtype=torch.int16, device="cuda")
    ctx.cast(x, po.FP32, 1.0, out, po.FP16, 1.0)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), g["fp16_cast_encode"])


def test_quantize_linear_matches_golden(ctx):
    g = golden("quant")
    x = dev(g["q_x"])
    out = torch.empty(x.numel(), dtype=torch.int8, device="cuda")
    for i in range(3):
        ctx.quantize_linear(x, po.FP32, [float(g[f"q_s{i}"])], [int(g[f"q_zp{i}"])], out)
        assert np.array_equal(out.cpu().numpy(), g[f"q_out{i}"]), i


def test_i8_matmul_requant_matches_golden(ctx):
    g = golden("quant")
    a, w = g["rq_a"], g["rq_w"]
    m, k = a.shape
    n = w.shape[1]
    for i in range(2):
        wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 0, scales=g[f"rq_ws{i}"], version=20 + i)
        out = torch.empty((m, n), dtype=torch.int8, device="cuda")
        ctx.i8_linear(po.I8_MATMUL, dev(a), float(g["rq_s_a"]), 0, m, wt, out, float(g[f"rq_s_out{i}"]),
                      int(g[f"rq_zp{i}"]))
        assert np.array_equal(out.cpu().numpy(), g[f"rq_out{i}"]), i
        wt.release()


@pytest.mark.parametrize("name,dtype", [("e4m3", E4), ("e5m2", E5)])
def test_fp8_linear_matches_golden(ctx, name, dtype):
    g = golden("linear")
    a, w_nk = g[f"{name}_a"], g[f"{name}_w_nk"]
    sa, sw, s_out = (float(v) for v in g[f"{name}_scales"])
    m, k = a.shape
    n = w_nk.shape[0]
    wt = ctx.prepare_weight(dev(w_nk), dtype, k, n, 1, version=30)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out)
    fp8_linear_check(dtype, out.cpu().numpy(), g[f"{name}_direct_t1"], a, sa, w_nk, sw, s_out, "HIP vs reference", backend=ctx.last_backend())
    rows = []
    for i in range(m):  # the decode path, one row per call, against the reference's prepared M = 1 kernel
        o1 = torch.empty((1, n), dtype=torch.uint8, device="cuda")
        ctx.fp8_linear(dev(a[i:i + 1]), dtype, sa, 1, wt, sw, o1, dtype, s_out)
        rows.append(o1.cpu().numpy()[0])
    fp8_linear_check(dtype, np.stack(rows), g[f"{name}_packed"], a, sa, w_nk, sw, s_out, "HIP m=1 vs reference", backend=ctx.last_backend())
    wt.release()


def test_argmax_matches_golden(ctx):
    g = golden("argmax")
    a, w = g["bf16_a"], g["bf16_w"]
    rows = a.shape[0]
    toks = torch.empty(rows, dtype=torch.int64, device="cuda")
    ctx.bf16_gemv_argmax(dev(a), dev(w), toks)  # all rows in one call (the m >= 2 kernel)
    assert toks.cpu().numpy().tolist() == g["bf16_tokens"].tolist()
    one = torch.empty(1, dtype=torch.int64, device="cuda")
    for i in range(rows):  # and one row per call (the m = 1 kernel)
        ctx.bf16_gemv_argmax(dev(a[i:i + 1]), dev(w), one)
        assert one.item() == g["bf16_tokens"][i], i
    for name, dtype in (("e4m3", E4), ("e5m2", E5)):
        sa, sw, s_out = (float(v) for v in g[f"{name}_scales"])
        ac, wc = g[f"{name}_a"], g[f"{name}_w"]
        ctx.fp8_gemv_argmax(dtype, dev(ac), sa, dev(wc), sw, s_out, toks)
        assert toks.cpu().numpy().tolist() == g[f"{name}_tokens"].tolist(), name
        for i in range(rows):
            ctx.fp8_gemv_argmax(dtype, dev(ac[i:i + 1]), sa, dev(wc), sw, s_out, one)
            assert one.item() == g[f"{name}_tokens"][i], (name, i)


def test_i8_gemm_and_conv_match_golden(ctx):
    """HIP INT8 Gemm and Conv2D against the reference's x86 INT8 kernels' outputs, bit for bit."""
    g = golden("int8")
    s_a, zp_a, alpha, beta, s_out, zp_out = (float(v) for v in g["g_params"])
    a, w = g["g_a"], g["g_w_nk"]
    m, k = a.shape
    n = w.shape[0]
    wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=g["g_ws"], version=50)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    bias = g["g_bias"]
    ctx.i8_linear(po.I8_GEMM, dev(a), s_a, int(zp_a), m, wt, out, s_out, int(zp_out), bias=dev(bias),
                  bias_kind=po.BIAS_VECTOR, bias_abs_max=int(np.abs(bias).max()), alpha=alpha, beta=beta)
    assert np.array_equal(out.cpu().numpy(), g["g_out"])
    wt.release()
    for name in ("c0", "c1"):
        layout, group, sh, sw, ph, pw, dh, dw, zp = (int(v) for v in g[f"{name}_geom"])
        cw = ctx.prepare_conv_weight(dev(g[f"{name}_w"]), g[f"{name}_ws"], group=group, version=51)
        ref = g[f"{name}_out"]
        y = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
        cb = g[f"{name}_bias"]
        ctx.i8_conv2d(dev(g[f"{name}_x"]), layout, 0.05, zp, cw, y, 0.4, 3, stride=(sh, sw), pad=(ph, pw),
                      dilation=(dh, dw), bias=dev(cb), bias_abs_max=int(np.abs(cb).max()))
        assert np.array_equal(y.cpu().numpy(), ref), name
        cw.release()
