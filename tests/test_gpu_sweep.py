"""Seeded random sweeps over the entry points' shape space, against the oracle, to the same bars as the focused
tests: INT8 Conv2D bit-exact over groups (window, gathered and one-channel-per-group kernels), both layouts,
strides, padding, dilation and zero points; INT8 MatMul/FC/Gemm bit-exact over M (both the K-split and the
tile kernels), K, N, zero points, bias kinds, alpha/beta and fused DequantizeLinear outputs; FP8 linear within
one code or the fp32 summation-order bound;
BF16 argmax tokens exact up to the order-induced BF16 boundary flip rule."""
import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import fp8_linear_check, fp8_pow2_scale, fp8_tensor, rng
from tests.test_gpu_argmax import check_tokens, head_inputs

pytestmark = pytest.mark.gpu


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def conv_case(seed):
    r = rng(seed)
    c = int(r.choice([1, 3, 8, 24, 64, 128]))
    group = int(r.choice([g for g in (1, 2, 4, c) if c % g == 0]))
    oc = group * int(r.integers(1, 5)) * (1 if group > 4 else int(r.choice([1, 8, 16])))
    kh, kw = int(r.choice([1, 2, 3, 5])), int(r.choice([1, 2, 3, 5]))
    stride = (int(r.integers(1, 3)), int(r.integers(1, 3)))
    dil = (int(r.integers(1, 3)), int(r.integers(1, 3)))
    pad = (int(r.integers(0, 3)), int(r.integers(0, 3)))
    h = int(r.integers(kh * dil[0], 40))
    wd = int(r.choice([int(r.integers(kw * dil[1], 40)), 32, 48, 64]))
    n = int(r.integers(1, 3))
    layout = int(r.integers(0, 2))
    return dict(c=c, group=group, oc=oc, kh=kh, kw=kw, stride=stride, dil=dil, pad=pad, h=h, wd=wd, n=n,
                layout=layout, zp_in=int(r.integers(-20, 21)), zp_out=int(r.integers(-10, 11)))


@pytest.mark.parametrize("seed", range(40))
def test_sweep_i8_conv(ctx, seed):
    p = conv_case(1000 + seed)
    r = rng(2000 + seed)
    oh = (p["h"] + 2 * p["pad"][0] - p["dil"][0] * (p["kh"] - 1) - 1) // p["stride"][0] + 1
    ow = (p["wd"] + 2 * p["pad"][1] - p["dil"][1] * (p["kw"] - 1) - 1) // p["stride"][1] + 1
    if oh <= 0 or ow <= 0:
        pytest.skip("empty output")
    x = r.integers(-128, 128, (p["n"], p["c"], p["h"], p["wd"])).astype(np.int8)
    w = r.integers(-127, 128, (p["oc"], p["c"] // p["group"], p["kh"], p["kw"])).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, p["oc"]).astype(np.float32)
    bias = r.integers(-5000, 5000, p["oc"]).astype(np.int32)
    xl = x if p["layout"] == 0 else np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    rc, ref = po.i8_conv2d(xl, 0.03, p["zp_in"], w, s_w, bias, p["stride"], p["pad"], 0.05, p["zp_out"],
                           dilation=p["dil"], group=p["group"], layout=p["layout"])
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, group=p["group"], version=20 + seed)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(xl), p["layout"], 0.03, p["zp_in"], wt, out, 0.05, p["zp_out"], stride=p["stride"],
                  pad=p["pad"], dilation=p["dil"], bias=dev(bias), bias_abs_max=5000)
    got = out.cpu().numpy()
    print(p, ctx.last_backend())
    assert np.array_equal(got, ref), f"{p} ({ctx.last_backend()}): {np.count_nonzero(got != ref)} mismatches"
    wt.release()


@pytest.mark.parametrize("seed", range(30))
def test_sweep_i8_linear(ctx, seed):
    r = rng(6000 + seed)
    kind = int(r.choice([po.I8_GEMM, po.I8_FC, po.I8_MATMUL]))
    m = int(r.choice([1, 7, 16, 33, 100, 200, 385, 512, 700, 1100]))
    k = int(r.choice([16, 48, 64, 128, 320, 1024, 2048]))
    n = int(r.integers(1, 900))
    zp_a, zp_y = int(r.integers(-30, 31)), int(r.integers(-20, 21))
    bias_kind = po.BIAS_NONE if kind == po.I8_MATMUL else int(r.choice([po.BIAS_NONE, po.BIAS_VECTOR, po.BIAS_MATRIX]))
    if kind == po.I8_FC and bias_kind == po.BIAS_MATRIX:
        bias_kind = po.BIAS_VECTOR
    alpha, beta = (1.0, 1.0) if kind != po.I8_GEMM or r.random() < 0.6 else (float(r.choice([0.5, 0.75, 2.0])),
                                                                             float(r.choice([-1.5, 0.0, 1.0])))
    pow2 = r.random() < 0.3
    out_dtype = int(r.choice([po.INT8, po.INT8, po.FP32, po.FP16, po.BF16]))
    xq = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    s_w = np.full(n, 2.0 ** -8, np.float32) if pow2 else r.uniform(1e-3, 1e-2, n).astype(np.float32)
    s_x, s_y = (0.0625, 2.0) if pow2 else (0.02, float(r.uniform(0.05, 0.5)))
    bias = None
    if bias_kind == po.BIAS_VECTOR:
        bias = r.integers(-20000, 20000, n).astype(np.int32)
    elif bias_kind == po.BIAS_MATRIX:
        bias = r.integers(-3000, 3000, (m, n)).astype(np.int32)
    trans_b = kind == po.I8_GEMM
    w_src = w if trans_b else np.ascontiguousarray(w.T)
    rc, ref, _ = po.i8_linear(kind, xq, s_x, zp_a, w_src, trans_b, s_w, None, bias, bias_kind, alpha, beta, s_y, zp_y)
    assert rc == 0
    s_dq, zp_dq = 0.0125, 3
    if out_dtype != po.INT8:
        rc, ref = po.dequantize_linear(ref, [s_dq], [zp_dq], out_dtype)
        assert rc == 0
    wt = ctx.prepare_weight(dev(w_src), po.INT8, k, n, 1 if trans_b else 0, scales=s_w, version=700 + seed)
    tdt = {po.INT8: torch.int8, po.FP32: torch.float32}.get(out_dtype, torch.int16)
    out = torch.empty((m, n), dtype=tdt, device="cuda")
    kw = {}
    if bias is not None:
        kw = dict(bias=dev(bias), bias_kind=bias_kind, bias_abs_max=int(np.abs(bias).max()))
    ctx.i8_linear_ex(kind, dev(xq), s_x, zp_a, m, wt, out, out_dtype, s_y, zp_y, dq_scale=s_dq, dq_zp=zp_dq,
                     alpha=alpha, beta=beta, **kw)
    got = out.cpu().numpy()
    case = f"kind={kind} m={m} k={k} n={n} bias={bias_kind} ab=({alpha},{beta}) out={out_dtype} ({ctx.last_backend()})"
    print(case)
    assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), case
    wt.release()


@pytest.mark.parametrize("seed", range(30))
def test_sweep_fp8_linear(ctx, seed):
    r = rng(3000 + seed)
    dtype = int(r.choice([po.FP8E4M3, po.FP8E5M2]))
    m = int(r.choice([1, 2, 3, 5, 8, 13, 16, 17, 33, 64, 100, 256]))
    k = 16 * int(r.integers(1, 129))
    n = int(r.integers(1, 600))
    layout = int(r.integers(0, 2))
    x = r.standard_normal((m, k)).astype(np.float32)
    wf = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    a, sa = fp8_tensor(x, dtype)
    w_nk, sw = fp8_tensor(wf, dtype)
    sums = po.fp8_sums(dtype, a, sa, w_nk, sw, True)
    s_out = fp8_pow2_scale(float(np.max(np.abs(sums))), dtype)
    w_src = w_nk if layout == 1 else np.ascontiguousarray(w_nk.T)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, layout, version=100 + seed)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out)
    ref = po.fp8_gemm(dtype, a, sa, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, out.cpu().numpy(), ref, a, sa, w_nk, sw, s_out,
                     f"sweep m={m} k={k} n={n} layout={layout} ({ctx.last_backend()})", backend=ctx.last_backend())
    wt.release()


def test_sweep_bf16_argmax(ctx):
    flips = 0
    for seed in range(30):
        r = rng(4000 + seed)
        m = int(r.choice([1, 2, 3, 8, 16]))
        k = 8 * int(r.integers(1, 514))
        v = int(r.integers(1, 3001))
        a, w = head_inputs(5000 + seed, m, k, v)
        tokens = torch.empty(m, dtype=torch.int64, device="cuda")
        ctx.bf16_gemv_argmax(dev(a), dev(w), tokens)
        flips += check_tokens(a, w, tokens.cpu().numpy())
    assert flips <= 2
