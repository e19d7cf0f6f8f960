"""Pins of the oracle's linear, INT8, quantization and argmax functions.

Known answers are transcribed from the reference's own tests (file:line in each test); brute force
(numpy int64 / float64) pins the accumulators; the reference's own code (oracle/_ref: x86 FP8 linear,
QuantizeInt8Value, QuantizeAccumulator, x86 BF16 argmax) pins what the closed forms leave open.
"""
import ctypes

import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import fp8_code_distance, fp8_linear_check, fp8_pow2_scale, fp8_tensor, rng

E4, E5 = po.FP8E4M3, po.FP8E5M2
needs_ref = pytest.mark.skipif(not po.ref_available(), reason="reference build (oracle/_ref) not present")


# ---- FP8 linear --------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [E4, E5])
def test_fp8_matmul_gemm_fc_small_closed_form(dtype):
    """test/fp8_test.cc:768-822: [[1,2],[3,4]] (scale 0.25) x [[5,6],[7,8]] (scale 0.5) = {19,22,43,50}."""
    a = po.fp8_encode(dtype, np.array([[1, 2], [3, 4]], np.float32) / np.float32(0.25))
    b = po.fp8_encode(dtype, np.array([[5, 6], [7, 8]], np.float32) / np.float32(0.5))
    expected = np.array([[19, 22], [43, 50]], np.float64)
    for out in (po.fp8_matmul(dtype, a, 0.25, b, 0.5, 0.25),
                po.fp8_gemm(dtype, a, 0.25, b, 0.5, False, 0.25),
                po.fp8_gemm(dtype, a, 0.25, np.ascontiguousarray(b.T), 0.5, True, 0.25)):
        got = po.fp8_decode(dtype, out).astype(np.float64) * 0.25
        if dtype == E4:  # the reference test's tolerance (it runs e4m3 only); e5m2 steps are 32/4 = 8 here
            assert np.all(np.abs(got - expected) <= 2.0)
        # and exactly the FP8 encoding of the exact products (no rounding happens before the encode)
        assert np.array_equal(out, po.fp8_encode(dtype, (expected / 0.25).astype(np.float32)))


def test_fp8_gemm_bias_alpha_beta_closed_form():
    """gemm.cc:87-98: out = Enc((alpha*sum + beta*Dec(bias)*s_bias) / s_out)."""
    d = E4
    a = po.fp8_encode(d, np.array([[1, 2]], np.float32))
    b = po.fp8_encode(d, np.array([[1, 0], [0, 1], [1, 1]], np.float32))  # [N,K]
    bias = po.fp8_encode(d, np.array([4, 8, 16], np.float32) / np.float32(2.0))
    out = po.fp8_gemm(d, a, 1.0, b, 1.0, True, 0.5, bias=bias, s_bias=2.0, bias_kind=po.BIAS_VECTOR,
                      alpha=2.0, beta=0.5)
    expected = np.array([[2 * 1 + 2, 2 * 2 + 4, 2 * 3 + 8]], np.float32) / np.float32(0.5)
    assert np.array_equal(out, po.fp8_encode(d, expected))
    # FC: bias added without alpha/beta (fc.cc:62-68)
    fc = np.empty((1, 3), np.uint8)
    bt = np.ascontiguousarray(b.T)
    assert po.lib().fo_fp8_fc(d, po._ptr(a), 1.0, po._ptr(bt), 1.0, po._ptr(bias), 2.0, po.BIAS_VECTOR, 1, 2, 3,
                              po._ptr(fc), 0.5) == 0
    assert np.array_equal(fc, po.fp8_encode(d, np.array([[1 + 4, 2 + 8, 3 + 16]], np.float32) / np.float32(0.5)))


@pytest.mark.parametrize("dtype", [E4, E5])
def test_fp8_sums_vs_float64_brute_force(dtype):
    """The oracle's fp32 K-ordered sum stays within the recursive-summation bound of the exact sum."""
    r = rng(3)
    m, k, n = 5, 700, 33
    a, sa = fp8_tensor(r.standard_normal((m, k)).astype(np.float32), dtype)
    b, sb = fp8_tensor((r.standard_normal((n, k)) * 0.02).astype(np.float32), dtype)
    sums = po.fp8_sums(dtype, a, sa, b, sb, True).astype(np.float64)
    ad = po.fp8_decode(dtype, a).astype(np.float64) * sa
    bd = po.fp8_decode(dtype, b).astype(np.float64) * sb
    exact = ad @ bd.T
    bound = (k - 1) * 2.0 ** -24 * (np.abs(ad) @ np.abs(bd).T) + 1e-30
    assert np.all(np.abs(sums - exact) <= bound)
    # a transposed operand or a dropped term would be far outside the bound
    assert np.max(np.abs(sums - ad @ np.roll(bd, 1, axis=1).T) - bound) > 0


@needs_ref
@pytest.mark.parametrize("dtype", [E4, E5])
@pytest.mark.parametrize("trans_b", [False, True])
def test_fp8_linear_vs_reference_x86(dtype, trans_b):
    """The reference's own x86 FP8 linear (linear_fp8.cc) agrees with the oracle within the FP8-output
    tolerance (it pre-scales the LHS and applies rhs_scale after the sum, so sums differ by rounding)."""
    R = po.ref()
    r = rng(4)
    m, k, n = 7, 1024, 200
    a, sa = fp8_tensor(r.standard_normal((m, k)).astype(np.float32), dtype)
    w_nk, sw = fp8_tensor((r.standard_normal((n, k)) * 0.02).astype(np.float32), dtype)
    s_out = fp8_pow2_scale(float(np.abs(po.fp8_sums(dtype, a, sa, w_nk, sw, True)).max()), dtype)
    ref_w = w_nk if trans_b else np.ascontiguousarray(w_nk.T)
    out = np.empty((m, n), np.uint8)
    assert R.ref_fp8_linear(dtype, po._ptr(a), sa, po._ptr(ref_w), sw, int(trans_b), None, 1.0, 0, 1.0, 1.0,
                            m, k, n, po._ptr(out), s_out) == 0
    fp8_linear_check(dtype, out, po.fp8_gemm(dtype, a, sa, w_nk, sw, True, s_out), a, sa, w_nk, sw, s_out,
                     "x86 reference vs oracle")
    # prepared (packed) decode path of the reference, M=1 only (linear_fp8.cc:564)
    h = R.ref_fp8_packed_create(dtype, po._ptr(ref_w), int(trans_b), k, n)
    out2 = np.empty((m, n), np.uint8)
    for i in range(m):
        row = np.ascontiguousarray(a[i:i + 1])
        dst = np.empty((1, n), np.uint8)
        assert R.ref_fp8_packed_compute(h, po._ptr(row), sa, sw, 1, po._ptr(dst), s_out) == 0
        out2[i] = dst[0]
    R.ref_fp8_packed_destroy(h)
    assert fp8_code_distance(out2, out).max() <= 1


# ---- QuantizeLinear / DequantizeLinear / requantization --------------------------------------

def test_quantize_known_answers():
    """test/quantization_math_test.cc:32-73."""
    x = np.array([-100.0, -1.0, -0.25, 0.25, 1.0, 100.0], np.float32)
    rc, q = po.quantize_linear(po.FP32, x, [0.5], [-3])
    assert rc == 0 and q.tolist() == [-128, -5, -4, -3, -1, 127]
    rc, back = po.dequantize_linear(q, [0.5], [-3])
    assert back[1] == -1.0 and back[4] == 1.0
    x2 = np.array([[1, 2, 4], [-1, -2, -4]], np.float32)
    rc, q2 = po.quantize_linear(po.FP32, x2, [0.5, 1.0, 2.0], [0, 1, -2], axis=1)
    assert rc == 0 and q2.reshape(-1).tolist() == [2, 3, 0, -2, -1, -4]
    rc, b2 = po.dequantize_linear(q2, [0.5, 1.0, 2.0], [0, 1, -2], axis=1)
    assert b2.reshape(-1)[:4].tolist() == [1.0, 2.0, 4.0, -1.0]
    # invalid metadata (quantization_math_test.cc:90-111): NaN scale, per-channel size mismatch
    assert po.quantize_linear(po.FP32, x, [float("nan")], [0])[0] == -1
    assert po.quantize_linear(po.FP32, x2, [1.0, 2.0], [0], axis=1)[0] == -1
    assert po.quantize_linear(po.FP32, x, [1.0], [200])[0] == -1


@needs_ref
def test_quantize_matches_reference_quantize_int8_value():
    """Every element against the reference's QuantizeInt8Value (include/quant/quantization.h:94-99),
    including ties, NaN, infinities and saturation."""
    R = po.ref()
    r = rng(5)
    s = np.float32(0.0625)
    x = np.concatenate([r.standard_normal(100000).astype(np.float32) * 4,
                        (np.arange(-300, 300, dtype=np.float32) + 0.5) * s,
                        np.array([np.nan, np.inf, -np.inf, 1e30, -1e30, 0.0, -0.0], np.float32)])
    for zp in (0, 7, -128, 127):
        ref = np.empty(x.size, np.int8)
        R.ref_quantize_int8_values(po._ptr(x), x.size, s, zp, po._ptr(ref))
        rc, got = po.quantize_linear(po.FP32, x, [s], [zp])
        assert rc == 0 and np.array_equal(got, ref)


def test_requantize_known_answers():
    """RequantizeInt32 (quantization_math_test.cc:75-88): acc scale 0.25 -> out scale 0.5, zp 2."""
    # through the MatMul flavour: one-element products with weight scale 0.25 and input scale 1
    acc = np.array([-4, 0, 4, 1000], np.int64)
    out = []
    for v in acc:
        a = np.array([[1]], np.int8) if abs(v) <= 127 else np.array([[125]], np.int8)
        w = np.array([[v if abs(v) <= 127 else 8]], np.int8)
        rc, o, _ = po.i8_linear(po.I8_MATMUL, a, 1.0, 0, w, False, [0.25], None, None, 0, 1, 1, 0.5, 2)
        assert rc == 0
        out.append(int(o[0, 0]))
    assert out == [0, 2, 4, 127]


def test_int8_kernel_known_answers():
    """test/common_int8_kernel_test.cc:103-211."""
    # FC: zero points, per-channel weights, int32 bias -> {8, 14}
    a = np.array([[5, 1]], np.int8)
    w = np.array([[2, 3], [6, -1]], np.int8)          # [K=2, N=2], per-channel along axis 1
    rc, o, _ = po.i8_linear(po.I8_FC, a, 0.5, 3, w, False, [0.25, 0.5], [-2, 1], np.array([4, -4], np.int32),
                            po.BIAS_VECTOR, 1, 1, 0.25, 10)
    assert rc == 0 and o.reshape(-1).tolist() == [8, 14]
    # MatMul saturates: 127*127 at output scale 0.01 -> 127
    rc, o, _ = po.i8_linear(po.I8_MATMUL, np.array([[127]], np.int8), 1.0, 0, np.array([[127]], np.int8), False,
                            [1.0], None, None, 0, 1, 1, 0.01, 0)
    assert rc == 0 and o[0, 0] == 127
    # Gemm with int32 vector bias -> {2,4,4,6}
    rc, o, _ = po.i8_linear(po.I8_GEMM, np.array([[1, 2], [3, 4]], np.int8), 1.0, 0,
                            np.array([[1, 0], [0, 1]], np.int8), False, [1.0], None, np.array([1, 2], np.int32),
                            po.BIAS_VECTOR, 1.0, 1.0, 1.0, 0)
    assert rc == 0 and o.reshape(-1).tolist() == [2, 4, 4, 6]
    # Conv2D 1x1 with input zp 3, weight zp 2, bias 4 -> 6
    rc, o = po.i8_conv2d(np.array([[[[5]]]], np.int8), 0.5, 3, np.array([[[[6]]]], np.int8), [0.25],
                         np.array([4], np.int32), 1, 0, 0.25, 0, w_zps=[2])
    assert rc == 0 and o.reshape(-1).tolist() == [6]


def test_int8_overflow_returns_failure():
    """The running int64 sum must stay within int32 (gemm.cc:177-181; int8_kernel_utils.h:99-114)."""
    k = 140000
    a = np.full((1, k), -128, np.int8)
    w = np.full((1, k), -128, np.int8)
    rc, _, _ = po.i8_linear(po.I8_GEMM, a, 1.0, 0, w, True, [1.0], None, None, 0, 1.0, 1.0, 1.0, 0)
    assert rc == -1


@pytest.mark.parametrize("kind", [po.I8_MATMUL, po.I8_FC, po.I8_GEMM])
def test_int8_accumulator_vs_numpy(kind):
    r = rng(6)
    m, k, n = 9, 333, 17
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    trans = kind == po.I8_GEMM
    ws = w if trans else np.ascontiguousarray(w.T)
    zp_a = -5
    wz = r.integers(-3, 4, n).astype(np.int32)
    rc, _, acc = po.i8_linear(kind, a, 0.1, zp_a, ws, trans, np.full(n, 0.01, np.float32), wz, None, 0, 1.0, 1.0,
                              1.0, 0, True)
    assert rc == 0
    exact = (a.astype(np.int64) - zp_a) @ (w.astype(np.int64) - wz[:, None]).T
    assert np.array_equal(acc, exact)


@needs_ref
def test_int8_requant_matches_reference_quantize_accumulator():
    """The fp64 requantization epilogue against the reference's own QuantizeAccumulator, with power-of-two
    scales so exact .5 ties occur (they round away from zero)."""
    R = po.ref()
    r = rng(7)
    m, k, n = 16, 64, 48
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (k, n)).astype(np.int8)
    for s_w, s_out in ((np.full(n, 2.0 ** -6, np.float32), 2.0), (r.uniform(1e-3, 1e-2, n).astype(np.float32), 0.37)):
        rc, out, acc = po.i8_linear(po.I8_MATMUL, a, 0.0625, 0, w, False, s_w, None, None, 0, 1, 1, s_out, 3, True)
        ref = np.empty((m, n), np.int8)
        assert R.ref_requantize(po._ptr(acc), m, n, 0.0625, po._ptr(s_w), n, s_out, 3, po._ptr(ref)) == 0
        assert np.array_equal(out, ref)


def test_conv_vs_numpy_brute_force():
    r = rng(8)
    n, c, h, wd, oc, g = 2, 6, 9, 7, 4, 2
    x = r.integers(-128, 128, (n, c, h, wd)).astype(np.int8)
    w = r.integers(-127, 128, (oc, c // g, 3, 3)).astype(np.int8)
    bias = r.integers(-100, 100, oc).astype(np.int32)
    zp = 3
    rc, out = po.i8_conv2d(x, 1.0, zp, w, [1.0], bias, 2, 1, 1.0, 0, group=g)
    assert rc == 0
    xp = np.pad(x.astype(np.int64) - zp, ((0, 0), (0, 0), (1, 1), (1, 1)))
    oh, ow = out.shape[2], out.shape[3]
    acc = np.zeros((n, oc, oh, ow), np.int64)
    for o in range(oc):
        gi = o // (oc // g)
        for ci in range(c // g):
            for ky in range(3):
                for kx in range(3):
                    acc[:, o] += w[o, ci, ky, kx] * xp[:, gi * (c // g) + ci, ky:ky + 2 * oh:2, kx:kx + 2 * ow:2]
        acc[:, o] += bias[o]
    assert np.array_equal(out, np.clip(acc, -128, 127).astype(np.int8))


# ---- argmax -------------------------------------------------------------------------------------

def test_bf16_argmax_known_answers():
    """test/qwen_gemm_argmax_test.cc:83-102 and :231-251."""
    a = po.bf16_encode(np.array([1.0, 2.0], np.float32))
    b = po.bf16_encode(np.array([[1.0, 0.0], [0.0, 1.0], [0.5, 0.5]], np.float32))
    assert po.bf16_gemm_argmax(a, b) == 1
    a1 = po.bf16_encode(np.array([1.0], np.float32))
    b1 = po.bf16_encode(np.array([[np.nan], [-0.0], [0.0]], np.float32))
    assert po.bf16_gemm_argmax(a1, b1) == 1
    assert po.bf16_gemm_argmax(a1, po.bf16_encode(np.full((4, 1), np.nan, np.float32))) == 0


def test_fp8_argmax_known_answer():
    """test/qwen_gemm_argmax_test.cc:104-131 (both formats)."""
    for d in (E4, E5):
        a = po.fp8_encode(d, np.array([1.0, 2.0], np.float32) / np.float32(0.25))
        b = po.fp8_encode(d, np.array([[1.0, 0.0], [0.0, 1.0], [0.5, 0.5]], np.float32) / np.float32(0.5))
        assert po.fp8_gemm_argmax(d, a, 0.25, b, 0.5, 1.0) == 1


@needs_ref
def test_bf16_argmax_vs_reference_x86():
    R = po.ref()
    for seed in range(6):
        r = rng(100 + seed)
        k, v = 256, 3000
        a = po.bf16_encode(r.standard_normal(k).astype(np.float32))
        w = po.bf16_encode((r.standard_normal((v, k)) * 0.02).astype(np.float32))
        if seed == 3:
            w[10] = w[2999]  # an exact tie: the lower index must win
            w[2999, 0] = 0x7FC0  # and a NaN row
        h = R.ref_bf16_argmax_create(po._ptr(w), k, v)
        tok = ctypes.c_int64()
        assert R.ref_bf16_argmax_compute(h, po._ptr(a), ctypes.byref(tok)) == 0
        R.ref_bf16_argmax_destroy(h)
        assert po.bf16_gemm_argmax(a, w) == tok.value


def _round_half_away(x):
    """std::round on float64, exactly: ties go away from zero."""
    t = np.trunc(x)
    return np.where(np.abs(x - t) >= 0.5, t + np.sign(x), t)


@pytest.mark.parametrize("alpha,beta", [(0.75, -1.5), (1.0, 0.0), (-2.0, 0.375), (3.0, 1.0)])
def test_int8_gemm_alpha_beta_matrix_bias_closed_form(alpha, beta):
    """The Gemm INT8 branch with alpha/beta != 1 and a matrix bias, against a numpy float64 statement of
    src/kernel/common/gemm.cc:171-195: acc = double(alpha)*dot + double(beta)*bias, real = acc * (double(s_a) *
    double(s_w[c])), q = clamp(round_half_away(real / double(s_out) + zp_out)).  Power-of-two scales make exact
    .5 ties; per-channel weight scales and zero points on both operands."""
    r = rng(77)
    m, k, n = 13, 96, 21
    a = r.integers(-6, 7, (m, k)).astype(np.int8)
    w = r.integers(-4, 5, (n, k)).astype(np.int8)
    a[0] = 127                     # row 0 against channels 0 / 1 saturates both ways
    w[0], w[1] = 100, -100
    wz = r.integers(-2, 3, n).astype(np.int32)
    wz[:2] = 0
    ws = (2.0 ** r.integers(-3, 0, n)).astype(np.float32)
    bias = r.integers(-300, 300, (m, n)).astype(np.int32)
    s_a, zp_a, s_out, zp_out = 0.5, -1, 0.25, 3
    rc, got, acc = po.i8_linear(po.I8_GEMM, a, s_a, zp_a, w, True, ws, wz, bias, po.BIAS_MATRIX, alpha, beta, s_out,
                                zp_out, True)
    assert rc == 0
    dot = (a.astype(np.int64) - zp_a) @ (w.astype(np.int64) - wz[:, None]).T
    assert np.array_equal(acc, dot)
    real = (np.float64(np.float32(alpha)) * dot.astype(np.float64) + np.float64(np.float32(beta)) * bias) * \
        (np.float64(np.float32(s_a)) * ws.astype(np.float64)[None, :])
    q = np.clip(_round_half_away(real / np.float64(np.float32(s_out)) + zp_out), -128, 127).astype(np.int8)
    assert np.array_equal(got, q)
    # the case is not degenerate: ties and both clamps occur
    t = real / s_out + zp_out
    assert np.any(np.abs(t - np.trunc(t)) == 0.5)
    assert np.any(q == 127) and np.any(q == -128)
