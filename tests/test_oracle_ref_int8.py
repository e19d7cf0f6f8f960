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
    h = R.ref_i8_conv2d_create(po._ptr(x), 1, 64, 160, 160, s_in, 0, po._ptr(w), 128, 3, 3, po._ptr(ws),
                               po._ptr(bias), 2, 1, 80, 80, s_out, 0)
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
