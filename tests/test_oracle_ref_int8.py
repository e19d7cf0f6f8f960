"""The oracle's INT8 Gemm and Conv2D against Feather's own x86 INT8 kernels (src/kernel/x86/int8.cc, built
from the Feather tree into oracle/_ref by `make -C oracle ref`; skipped where that build is absent).

The oracle restates the Common kernels (common/gemm.cc:136-198, conv2d.cc:482-581).  The x86 Gemm uses the
same double-precision requantization and must agree exactly.  The x86 conv requantizes with a float fast
path (FastQuantizeAccumulator8, int8.cc:410-446): it agrees with Common everywhere except on exact
round-half boundaries: exact ties (which power-of-two scales make possible) and values within float32
rounding of one.  There the two reference paths differ by one code; the test checks that every such
difference sits within a few float32 ulps of a tie of Common's real value, so the HIP kernels (which follow
Common) differ from the x86 path only there.
"""
import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.skipif(not po.ref_available(), reason="oracle/_ref not built (needs the Feather tree)")


def _x86_gemm(a, s_a, zp_a, w_nk, ws, bias, alpha, beta, s_out, zp_out):
    R = po.ref()
    m, k = a.shape
    n = w_nk.shape[0]
    h = R.ref_i8_gemm_create(po._ptr(a), s_a, zp_a, m, k, po._ptr(w_nk), po._ptr(ws), ws.size, n,
                             po._ptr(bias) if bias is not None else None, alpha, beta, s_out, zp_out)
    try:
        rc = R.ref_i8_gemm_compute(h)
        out = np.empty((m, n), np.int8)
        R.ref_i8_gemm_output(h, po._ptr(out))
    finally:
        R.ref_i8_gemm_destroy(h)
    return rc, out


@pytest.mark.parametrize("m,k,n,zp_a,alpha,beta", [(128, 1024, 1024, 0, 1.0, 1.0), (37, 300, 129, -7, 1.0, 1.0),
                                                   (64, 512, 256, 3, 0.75, -1.5)])
def test_oracle_gemm_equals_x86_int8_gemm(m, k, n, zp_a, alpha, beta):
    r = np.random.default_rng(m * 7 + n)
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    ws = r.uniform(1e-3, 1e-2, n).astype(np.float32)
    bias = r.integers(-20000, 20000, n).astype(np.int32)
    rc_x, out_x = _x86_gemm(a, 0.03, zp_a, w, ws, bias, alpha, beta, 0.05, 0)
    rc_o, out_o, _ = po.i8_linear(po.I8_GEMM, a, 0.03, zp_a, w, True, ws, None, bias, po.BIAS_VECTOR, alpha, beta,
                                  0.05, 0)
    assert rc_x == 0 and rc_o == 0
    assert np.array_equal(out_o, out_x)


def _conv_acc(x, w, bias, oc, oy, ox, stride=2, pad=1):
    _, c, h, wd = x.shape
    kh, kw = w.shape[2:]
    acc = int(bias[oc])
    for i in range(kh):
        for j in range(kw):
            y, xx = oy * stride - pad + i, ox * stride - pad + j
            if 0 <= y < h and 0 <= xx < wd:
                acc += int(np.dot(x[0, :, y, xx].astype(np.int64), w[oc, :, i, j].astype(np.int64)))
    return acc


@pytest.mark.parametrize("s_in,s_out", [(0.05, 0.5), (0.0625, 0.5)])
def test_oracle_conv_vs_x86_int8_conv(s_in, s_out):
    r = np.random.default_rng(44)
    x = r.integers(-128, 128, (1, 64, 160, 160)).astype(np.int8)
    w = r.integers(-127, 128, (128, 64, 3, 3)).astype(np.int8)
    # power-of-two weight scales with a power-of-two s_in make exact ties possible
    ws = (2.0 ** r.integers(-9, -6, 128)).astype(np.float32) if s_in == 0.0625 else \
        r.uniform(1e-3, 1e-2, 128).astype(np.float32)
    bias = r.integers(-5000, 5000, 128).astype(np.int32)
    R = po.ref()
    h = R.ref_i8_conv2d_create(po._ptr(x), 1, 64, 160, 160, 0, s_in, 0, po._ptr(w), 128, 3, 3, 1, po._ptr(ws),
                               po._ptr(bias), 2, 2, 1, 1, 1, 1, 80, 80, s_out, 0)
    try:
        assert R.ref_i8_conv2d_compute(h) == 0
        out_x = np.empty((1, 128, 80, 80), np.int8)
        R.ref_i8_conv2d_output(h, po._ptr(out_x))
    finally:
        R.ref_i8_conv2d_destroy(h)
    rc, out_o = po.i8_conv2d(x, s_in, 0, w, ws, bias, 2, 1, s_out, 0)
    assert rc == 0
    diff = np.argwhere(out_o != out_x)
    print(f"s_in={s_in}: x86 conv path {'VNNI' if R.ref_has_avx_vnni() else 'AVX2'}, "
          f"{len(diff)} of {out_o.size} outputs differ from Common")
    assert len(diff) <= 64
    for _, oc, oy, ox in diff:
        assert abs(int(out_o[0, oc, oy, ox]) - int(out_x[0, oc, oy, ox])) == 1
        real = _conv_acc(x, w, bias, oc, oy, ox) * (np.float64(s_in) * np.float64(ws[oc])) / np.float64(s_out)
        # within float32 rounding (a few ulps of |real|) of a round-half boundary
        dist = abs((real - np.floor(real)) - 0.5)
        print(f"  ({oc},{oy},{ox}): Common real {real!r}, {dist:.3g} from the tie")
        assert dist <= 4 * 2.0 ** -24 * max(1.0, abs(real)), f"difference at ({oc},{oy},{ox}) is not at a tie"


def _x86_conv(x, layout, s_in, zp_in, w, group, ws, bias, stride, pad, dil, s_out, zp_out):
    R = po.ref()
    if layout == 0:
        n, c, h, wd = x.shape
    else:
        n, h, wd, c = x.shape
    oc, _, kh, kw = w.shape
    oh = (h + 2 * pad[0] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    ow = (wd + 2 * pad[1] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    hd = R.ref_i8_conv2d_create(po._ptr(x), n, c, h, wd, layout, s_in, zp_in, po._ptr(w), oc, kh, kw, group,
                                po._ptr(ws), po._ptr(bias) if bias is not None else None, stride[0], stride[1], pad[0],
                                pad[1], dil[0], dil[1], oh, ow, s_out, zp_out)
    try:
        rc = R.ref_i8_conv2d_compute(hd)
        out = np.empty((n, oc, oh, ow) if layout == 0 else (n, oh, ow, oc), np.int8)
        R.ref_i8_conv2d_output(hd, po._ptr(out))
    finally:
        R.ref_i8_conv2d_destroy(hd)
    return rc, out


def _brute_conv_point(x, zp_in, w, group, bias, stride, pad, dil, ws, s_in, s_out, zp_out, b, o, y, xx):
    """One NCHW output of the Common conv (conv2d.cc:482-581) by plain integer loops and the double
    requantization: the arbiter where the two reference paths disagree."""
    _, c, h, wd = x.shape
    oc, icg, kh, kw = w.shape
    g = o // (oc // group)
    acc = int(bias[o])
    for ci in range(icg):
        for ky in range(kh):
            for kx in range(kw):
                iy, ix = y * stride[0] - pad[0] + ky * dil[0], xx * stride[1] - pad[1] + kx * dil[1]
                if 0 <= iy < h and 0 <= ix < wd:
                    acc += (int(x[b, g * icg + ci, iy, ix]) - zp_in) * int(w[o, ci, ky, kx])
    t = acc * (np.float64(np.float32(s_in)) * np.float64(ws[o])) / np.float64(np.float32(s_out)) + zp_out
    return int(np.clip(np.sign(t) * np.floor(abs(t) + 0.5), -128, 127))


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("c,oc,group,k,stride,pad,dil,zp_in", [
    (64, 96, 1, 3, (1, 1), (1, 1), (1, 1), 0),     # stride 1
    (32, 48, 2, 3, (2, 1), (1, 2), (1, 1), -9),    # groups, asymmetric stride/pad, zero point
    (32, 48, 2, 3, (2, 1), (1, 2), (2, 2), -9),    # ... and dilation
    (64, 64, 1, 1, (1, 1), (0, 0), (1, 1), 5),     # pointwise
    (16, 24, 1, 5, (2, 2), (2, 2), (1, 1), 0),     # 5x5
])
def test_oracle_conv_geometries_vs_x86(layout, c, oc, group, k, stride, pad, dil, zp_in):
    """The oracle's Conv2D against the reference's x86 INT8 conv on the geometries its code paths split on
    (oc8 maddubs / pair / pointwise / VNNI tiles, int8.cc:684-2346): equal wherever the x86 float
    requantization does not sit within float rounding of a round-half boundary.

    Reference finding: for NCHW activations with a horizontal dilation other than 1, the x86 kernel's
    generic path (int8.cc:776-794) walks consecutive input columns for consecutive kernel columns, i.e. it
    ignores dilation_w, so it disagrees with the reference's own Common kernel.  There the oracle (and the
    HIP kernels) follow Common, which this test checks against plain integer loops on sampled outputs."""
    r = np.random.default_rng(c * 131 + oc + k + group + dil[1])
    n, h, wd = 2, 19, 23
    x = r.integers(-128, 128, (n, c, h, wd)).astype(np.int8)
    xl = x if layout == 0 else np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    w = r.integers(-127, 128, (oc, c // group, k, k)).astype(np.int8)
    ws = r.uniform(1e-3, 1e-2, oc).astype(np.float32)
    bias = r.integers(-4000, 4000, oc).astype(np.int32)
    rc_x, out_x = _x86_conv(xl, layout, 0.05, zp_in, w, group, ws, bias, stride, pad, dil, 0.4, 3)
    rc_o, out_o = po.i8_conv2d(xl, 0.05, zp_in, w, ws, bias, stride, pad, 0.4, 3, dilation=dil, group=group,
                               layout=layout)
    assert rc_x == 0 and rc_o == 0
    if layout == 0 and dil[1] != 1:
        oo = out_o
        pts = [(bb, o, yy, xq) for bb in range(n) for o in (0, oc // 2 + 1, oc - 1)
               for yy in (0, oo.shape[2] // 2, oo.shape[2] - 1) for xq in (0, oo.shape[3] // 2, oo.shape[3] - 1)]
        for pt in pts:
            assert oo[pt] == _brute_conv_point(x, zp_in, w, group, bias, stride, pad, dil, ws, 0.05, 0.4, 3, *pt), pt
        assert np.mean(out_o != out_x) > 0.5  # the x86 path's dilation_w slip, documented above
        return
    diff = np.argwhere(out_o != out_x)
    assert len(diff) <= max(2, out_o.size // 50000), f"{len(diff)} of {out_o.size} differ"
    assert np.all(np.abs(out_o.astype(np.int32) - out_x.astype(np.int32)) <= 1)
