"""Seeded random sweeps over the entry points' shape space, against the oracle, to the same bars as the focused
tests: INT8 Conv2D bit-exact over groups (window, gathered and one-channel-per-group kernels), both layouts,
strides, padding, dilation and zero points; FP8 linear within one code or the fp32 summation-order bound;
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
                     f"sweep m={m} k={k} n={n} layout={layout} ({ctx.last_backend()})")
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
