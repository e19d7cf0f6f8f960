"""GPU parity of the INT8 path (QuantizeLinear, MatMul/FC/Gemm INT8, Conv2D INT8, DequantizeLinear).

Oracle: oracle/feather_oracle.c restating src/kernel/common/{gemm,fc,matmul,conv2d}.cc and
quantize_linear_utils.h.  Bar: bit-exact int8/fp32 outputs.
"""
import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import SEEDS, rng

pytestmark = pytest.mark.gpu


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def c1_inputs(seed=SEEDS[1], m=128, k=1024, n=1024):
    """Config 1: X ~ N(0,1) per-tensor int8 (s = max|X|/127), W int8 U[-127,127] per-channel scales
    U(1e-3, 1e-2), bias ~ N(0, 0.1) quantized as round(b / (s_x * s_w)) (static_quantizer.cc:256-287)."""
    r = rng(seed)
    x = r.standard_normal((m, k)).astype(np.float32)
    s_x = np.float32(np.max(np.abs(x)) / 127.0)
    w = r.integers(-127, 128, size=(n, k), dtype=np.int64).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    b = (r.standard_normal(n) * 0.1).astype(np.float32)
    bias = np.round(b.astype(np.float64) / (np.float64(s_x) * s_w.astype(np.float64))).astype(np.int32)
    return x, s_x, w, s_w, bias


def test_quantize_linear_fp32_per_tensor(ctx):
    x, s_x, *_ = c1_inputs()
    x = x.copy()
    x[0, :8] = [np.nan, np.inf, -np.inf, 0.5 * s_x, -0.5 * s_x, 1.5 * s_x, 1e30, -1e30]
    for zp in (0, 3, -128):
        out = torch.empty(x.shape, dtype=torch.int8, device="cuda")
        ctx.quantize_linear(dev(x), po.FP32, [s_x], [zp], out)
        rc, ref = po.quantize_linear(po.FP32, x, [s_x], [zp])
        assert rc == 0
        assert np.array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("src_dtype", [po.BF16, po.FP16])
def test_quantize_linear_half_per_tensor_every_code(ctx, src_dtype):
    """Per-tensor QuantizeLinear (the reciprocal-multiply kernel) over all 65536 BF16 / FP16 codes: NaN, Inf,
    subnormals, and, at power-of-two scales, exact x.5 ties that must go to the division and round away."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for scale, zp in ((0.25, 0), (2.0 ** -7, 3), (0.0123, -5), (3.0, 127)):
        out = torch.empty(codes.shape, dtype=torch.int8, device="cuda")
        ctx.quantize_linear(dev(codes), src_dtype, [scale], [zp], out)
        rc, ref = po.quantize_linear(src_dtype, codes, [scale], [zp])
        assert rc == 0
        got = out.cpu().numpy()
        assert np.array_equal(got, ref), f"scale {scale} zp {zp}: {np.count_nonzero(got != ref)} mismatches"


@pytest.mark.parametrize("src_dtype", [po.BF16, po.FP16])
def test_quantize_linear_half_per_channel(ctx, src_dtype):
    r = rng(5)
    x = r.standard_normal((4, 200, 3)).astype(np.float32)
    bits = po.bf16_encode(x) if src_dtype == po.BF16 else po.fp16_encode(x)
    scales = r.uniform(0.01, 0.05, 200).astype(np.float32)
    zps = r.integers(-5, 6, 200).astype(np.int32)
    out = torch.empty(x.shape, dtype=torch.int8, device="cuda")
    ctx.quantize_linear(dev(bits), src_dtype, scales, zps, out, channels=200, inner=3)
    rc, ref = po.quantize_linear(src_dtype, bits, scales, zps, axis=1)
    assert rc == 0
    assert np.array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("dst", [po.FP32, po.BF16, po.FP16])
def test_dequantize_linear(ctx, dst):
    q = np.arange(-128, 128, dtype=np.int8).reshape(16, 16)
    q = np.tile(q, (3, 1))
    for scales, zps, ch, inner, axis in (([0.0123], [7], 1, 1, -1), (list(np.linspace(0.01, 0.2, 16)), [1] * 16, 16, 1, 1)):
        out = torch.empty(q.shape, dtype=torch.float32 if dst == po.FP32 else torch.int16, device="cuda")
        ctx.dequantize_linear(dev(q), scales, zps, out, dst, channels=ch, inner=inner)
        rc, ref = po.dequantize_linear(q, scales, zps, dst, axis=axis)
        assert rc == 0
        got = out.cpu().numpy()
        if dst != po.FP32:
            got = got.view(np.uint16)
        assert np.array_equal(got.view(np.uint32) if dst == po.FP32 else got,
                              ref.view(np.uint32) if dst == po.FP32 else ref)


@pytest.mark.parametrize("kind", [po.I8_GEMM, po.I8_FC, po.I8_MATMUL])
def test_i8_linear_config1_bitexact(ctx, kind):
    x, s_x, w_nk, s_w, bias = c1_inputs()
    m, k = x.shape
    n = w_nk.shape[0]
    _, xq = po.quantize_linear(po.FP32, x, [s_x], [0])
    trans_b = kind == po.I8_GEMM
    w_src = w_nk if trans_b else np.ascontiguousarray(w_nk.T)
    bias_kind = po.BIAS_NONE if kind == po.I8_MATMUL else po.BIAS_VECTOR
    # output scale from the fp32 reference (calibration rule max|y| / 127, tools/int8_calibrate.cc:146-147)
    _, _, acc = po.i8_linear(kind, xq, s_x, 0, w_src, trans_b, s_w, None, bias, bias_kind, 1.0, 1.0, 1.0, 0, True)
    y = (acc.astype(np.float64) + (bias if bias_kind else 0)) * s_x * s_w.astype(np.float64)
    s_y = np.float32(np.max(np.abs(y)) / 127.0)
    rc, ref, _ = po.i8_linear(kind, xq, s_x, 0, w_src, trans_b, s_w, None, bias, bias_kind, 1.0, 1.0, s_y, 0)
    assert rc == 0
    wt = ctx.prepare_weight(dev(w_src), po.INT8, k, n, 1 if trans_b else 0, scales=s_w, version=kind)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    ctx.i8_linear(kind, dev(xq), s_x, 0, m, wt, out, s_y, 0, bias=dev(bias), bias_kind=bias_kind,
                  bias_abs_max=int(np.abs(bias).max()))
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    wt.release()


@pytest.mark.parametrize("out_dtype", [po.FP32, po.FP16, po.BF16])
def test_i8_gemm_fused_dequantize_matches_chain(ctx, out_dtype):
    """Config 1's Gemm -> DequantizeLinear pair in one launch equals the two nodes run one after the other,
    bit for bit, including a DequantizeLinear whose parameters differ from the Gemm output's."""
    x, s_x, w_nk, s_w, bias = c1_inputs()
    m, k = x.shape
    n = w_nk.shape[0]
    _, xq = po.quantize_linear(po.FP32, x, [s_x], [0])
    wt = ctx.prepare_weight(dev(w_nk), po.INT8, k, n, 1, scales=s_w, version=40)
    for s_y, zp_y, s_dq, zp_dq in ((0.05, 0, 0.05, 0), (0.0371, -6, 0.0125, 3)):
        rc, yq, _ = po.i8_linear(po.I8_GEMM, xq, s_x, 0, w_nk, True, s_w, None, bias, po.BIAS_VECTOR, 1.0, 1.0, s_y,
                                 zp_y)
        assert rc == 0
        rc, ref = po.dequantize_linear(yq, [s_dq], [zp_dq], out_dtype)
        assert rc == 0
        tdt = torch.float32 if out_dtype == po.FP32 else torch.int16
        out = torch.empty((m, n), dtype=tdt, device="cuda")
        ctx.i8_linear_ex(po.I8_GEMM, dev(xq), s_x, 0, m, wt, out, out_dtype, s_y, zp_y, dq_scale=s_dq, dq_zp=zp_dq,
                         bias=dev(bias), bias_kind=po.BIAS_VECTOR, bias_abs_max=int(np.abs(bias).max()))
        got = out.cpu().numpy()
        if out_dtype != po.FP32:
            got = got.view(np.uint16)
        assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), (s_y, zp_y)
    wt.release()


def test_i8_gemm_zero_points_alpha_beta_ragged(ctx):
    r = rng(21)
    m, k, n = 37, 80, 45
    xq = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    s_w = np.float32(0.004)
    bias = r.integers(-3000, 3000, (m, n)).astype(np.int32)
    # power-of-two scales so exact .5 ties occur in the requantization
    s_x, s_y = 0.0625, 2.0
    for zp_a, zp_y, alpha, beta in ((5, -3, 1.0, 1.0), (-20, 10, 0.75, -1.5)):
        rc, ref, _ = po.i8_linear(po.I8_GEMM, xq, s_x, zp_a, w, True, [s_w], None, bias, po.BIAS_MATRIX, alpha, beta,
                                  s_y, zp_y)
        assert rc == 0
        wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=[s_w], version=9)
        out = torch.empty((m, n), dtype=torch.int8, device="cuda")
        ctx.i8_linear(po.I8_GEMM, dev(xq), s_x, zp_a, m, wt, out, s_y, zp_y, bias=dev(bias),
                      bias_kind=po.BIAS_MATRIX, bias_abs_max=3000, alpha=alpha, beta=beta)
        assert np.array_equal(out.cpu().numpy(), ref)
        wt.release()


def test_i8_gemm_large_tile_path_long_k(ctx):
    """Enough 32x32 tiles for the larger GEMM tile, and K = 1040: 17 steps of 64 with a 16-deep tail, so
    the waves' K split runs a second unrolled round and a partial final step."""
    r = rng(22)
    m, k, n = 520, 1040, 1000
    xq = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, n).astype(np.float32)
    bias = r.integers(-20000, 20000, n).astype(np.int32)
    s_x, s_y, zp_a, zp_y = 0.01, 0.5, 3, -2
    rc, ref, _ = po.i8_linear(po.I8_GEMM, xq, s_x, zp_a, w, True, s_w, None, bias, po.BIAS_VECTOR, 1.0, 1.0, s_y,
                              zp_y)
    assert rc == 0
    wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=s_w, version=10)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    ctx.i8_linear(po.I8_GEMM, dev(xq), s_x, zp_a, m, wt, out, s_y, zp_y, bias=dev(bias), bias_kind=po.BIAS_VECTOR,
                  bias_abs_max=20000)
    assert ctx.last_backend() == "i8_mfma_gemm_32x32_ksplit4"
    assert np.array_equal(out.cpu().numpy(), ref)
    wt.release()


def c4_inputs(seed=SEEDS[4], pow2=True):
    r = rng(seed)
    x = r.integers(-128, 128, (1, 64, 160, 160)).astype(np.int8)
    w = r.integers(-127, 128, (128, 64, 3, 3)).astype(np.int8)
    if pow2:
        s_in = 0.0078125
        s_w = (2.0 ** -r.integers(6, 9, 128)).astype(np.float32)
    else:
        s_in = np.float32(r.uniform(0.01, 0.02))
        s_w = r.uniform(1e-3, 1e-2, 128).astype(np.float32)
    bias = r.integers(-20000, 20000, 128).astype(np.int32)
    return x, np.float32(s_in), w, s_w, bias


@pytest.mark.parametrize("pow2", [True, False])
def test_i8_conv_config4_bitexact(ctx, pow2):
    x, s_in, w, s_w, bias = c4_inputs(pow2=pow2)
    s_out = np.float32(0.25 if pow2 else 0.3)
    rc, ref = po.i8_conv2d(x, s_in, 0, w, s_w, bias, 2, 1, s_out, 0)
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, version=4)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(x), 0, s_in, 0, wt, out, s_out, 0, stride=(2, 2), pad=(1, 1), bias=dev(bias),
                  bias_abs_max=20000)
    assert ctx.last_backend() == "i8_mfma_conv_window"
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    wt.release()


def test_i8_conv_window_128_channel_blocks(ctx):
    """A grid large enough (here 1024 blocks) for the window kernel's 128-output-channel blocks, with OC
    = 160 ending in a partial block; smaller grids (C4 among them) take 64-channel blocks."""
    r = rng(53)
    n, c, h, wd, oc = 4, 64, 64, 64, 160
    x = r.integers(-128, 128, (n, c, h, wd)).astype(np.int8)
    w = r.integers(-127, 128, (oc, c, 3, 3)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, oc).astype(np.float32)
    bias = r.integers(-3000, 3000, oc).astype(np.int32)
    rc, ref = po.i8_conv2d(x, 0.03, 3, w, s_w, bias, 1, 1, 0.4, -2)
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, version=8)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(x), 0, 0.03, 3, wt, out, 0.4, -2, stride=(1, 1), pad=(1, 1), bias=dev(bias), bias_abs_max=3000)
    assert ctx.last_backend() == "i8_mfma_conv_window"
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    wt.release()


@pytest.mark.parametrize("sign", [1, -1])
def test_i8_conv_requant_near_ties(ctx, sign):
    """The conv epilogue's requantization on values just off an x.5 point: with s_in * s_w / s_out =
    0.5 + 2^-21 every odd sum x lands x * 2^-21 (<= 1.2e-4) above or below a tie; the reference rounds each
    away from the tie, and so must the reciprocal-multiply fast path with its division fallback
    (requant_i8).  Small operands keep most sums inside the int8 range."""
    r = rng(77)
    n, c, h, wd, oc = 1, 64, 9, 32, 16
    x = r.integers(-2, 3, (n, c, h, wd)).astype(np.int8)
    w = (sign * r.integers(-2, 3, (oc, c, 3, 3))).astype(np.int8)
    s_w = np.full(oc, np.float32(0.5 + 2.0 ** -21), np.float32)
    rc, ref = po.i8_conv2d(x, 1.0, 0, w, s_w, None, 1, 1, 1.0, 0)
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, version=7)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(x), 0, 1.0, 0, wt, out, 1.0, 0, stride=(1, 1), pad=(1, 1))
    assert ctx.last_backend() == "i8_mfma_conv_window"
    got = out.cpu().numpy()
    odd = np.count_nonzero((np.abs(ref) < 127) & (np.abs(ref) > 0))
    assert odd > 1000
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    wt.release()


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("c,oc,group,kh,kw,stride,pad,dil", [
    (24, 24, 24, 3, 3, (1, 1), (1, 1), (1, 1)),   # depthwise
    (12, 24, 12, 3, 3, (2, 2), (1, 1), (1, 1)),   # channel multiplier 2, stride 2
    (16, 16, 16, 5, 3, (1, 2), (2, 0), (2, 1)),   # asymmetric kernel, stride, pad and dilation
    (1, 16, 1, 3, 3, (1, 1), (0, 1), (1, 1)),     # one input channel, group 1
])
def test_i8_conv_one_channel_per_group(ctx, layout, c, oc, group, kh, kw, stride, pad, dil):
    """Convolutions whose groups hold one input channel (depthwise, channel multipliers, single-channel
    inputs) run on the direct kernel; bit-exact against the oracle with a non-zero input zero point and bias."""
    r = rng(61 + c + oc + kh)
    n, h, wd = 2, 19, 23
    x = r.integers(-128, 128, (n, c, h, wd)).astype(np.int8)
    w = r.integers(-127, 128, (oc, c // group, kh, kw)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, oc).astype(np.float32)
    bias = r.integers(-3000, 3000, oc).astype(np.int32)
    xl = x if layout == 0 else np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    rc, ref = po.i8_conv2d(xl, 0.04, -9, w, s_w, bias, stride, pad, 0.03, 5, dilation=dil, group=group,
                           layout=layout)
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, group=group, version=9)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(xl), layout, 0.04, -9, wt, out, 0.03, 5, stride=stride, pad=pad, dilation=dil,
                  bias=dev(bias), bias_abs_max=3000)
    assert ctx.last_backend() == "i8_conv_depthwise"
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    wt.release()


def test_i8_conv_general_path_large_image(ctx):
    """The gathered conv kernel grid-strides its pixel tiles: a 2100 x 2100 output (68906 tiles of 64 pixels,
    past the grid's 65535 y extent) on a grouped 1x1 conv with two input channels per group."""
    r = rng(71)
    n, c, h, wd, oc, g = 1, 4, 2100, 2100, 2, 2
    x = r.integers(-128, 128, (n, c, h, wd)).astype(np.int8)
    w = r.integers(-127, 128, (oc, c // g, 1, 1)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, oc).astype(np.float32)
    rc, ref = po.i8_conv2d(x, 0.05, 2, w, s_w, None, 1, 0, 0.01, -3, group=g)
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, group=g, version=10)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(x), 0, 0.05, 2, wt, out, 0.01, -3)
    assert ctx.last_backend() == "i8_mfma_conv_64x64"
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    wt.release()


@pytest.mark.parametrize("layout", [0, 1])
def test_i8_conv_groups_dilation_zero_point(ctx, layout):
    r = rng(31)
    n, c, h, wd, oc, g = 2, 8, 13, 11, 12, 2
    x = r.integers(-128, 128, (n, c, h, wd)).astype(np.int8)
    w = r.integers(-127, 128, (oc, c // g, 3, 2)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, oc).astype(np.float32)
    bias = r.integers(-500, 500, oc).astype(np.int32)
    xl = x if layout == 0 else np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    rc, ref = po.i8_conv2d(xl, 0.05, -7, w, s_w, bias, (2, 1), (1, 2), 0.02, 4, dilation=(2, 1), group=g,
                           layout=layout)
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, group=g, version=5)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(xl), layout, 0.05, -7, wt, out, 0.02, 4, stride=(2, 1), pad=(1, 2), dilation=(2, 1),
                  bias=dev(bias), bias_abs_max=500)
    assert np.array_equal(out.cpu().numpy(), ref)
    wt.release()


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("wd,pad", [(23, (1, 0)), (76, (1, 1)), (96, (1, 1)), (160, (0, 3))])
def test_i8_conv_window_path_general_geometry(ctx, layout, wd, pad):
    """The LDS-window conv kernel (group 1, IC % 64 == 0) on a ragged shape: OC not a multiple of 64,
    asymmetric stride/pad/dilation, non-zero input zero point, output width not a multiple of 32.
    Width 23 stages NCHW rows byte by byte; width 76 (rows 4-byte aligned, odd left pad, two blocks per
    output row) takes the aligned-dword staging with a 3-byte shift; widths 96 and 160 (rows a multiple of
    16 bytes) take the 16-byte chunk staging, with left pads 1 and 3 (window starts before the row, chunk
    offsets 15 and 13) and chunks past the right edge."""
    r = rng(41)
    n, c, h, oc = 2, 128, 17, 80
    x = r.integers(-128, 128, (n, c, h, wd)).astype(np.int8)
    w = r.integers(-127, 128, (oc, c, 3, 3)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, oc).astype(np.float32)
    bias = r.integers(-3000, 3000, oc).astype(np.int32)
    xl = x if layout == 0 else np.ascontiguousarray(x.transpose(0, 2, 3, 1))
    rc, ref = po.i8_conv2d(xl, 0.03, -5, w, s_w, bias, (1, 2), pad, 0.05, 2, dilation=(2, 1), layout=layout)
    assert rc == 0
    wt = ctx.prepare_conv_weight(dev(w), s_w, version=6)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(xl), layout, 0.03, -5, wt, out, 0.05, 2, stride=(1, 2), pad=pad, dilation=(2, 1),
                  bias=dev(bias), bias_abs_max=3000)
    assert ctx.last_backend() == "i8_mfma_conv_window"
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches"
    wt.release()


def test_i8_linear_overflow_bound_declines_where_common_fails(ctx):
    """The int32 partial-sum rule (gemm.cc:177-181; int8_kernel_utils.h:99-114).  The host bound is
    K * (128 + |zp_a|) * max|w - zp_w| + |bias|: with (a - zp_a) = -255 and w = 127 on every step,
    K = 66304 keeps every partial sum inside int32 -- the HIP path runs and is bit-exact -- while
    K = 66432 overflows at the last steps: the Common kernel returns -1 and the HIP path declines with
    FHIP_ERR_UNSUPPORTED (-2) so that Feather's Common kernel runs and fails exactly as the reference does."""
    n, m = 32, 2
    for k, expect in ((66304, 0), (66432, -2)):
        a = np.full((m, k), -128, np.int8)
        a[1, ::3] = 5                              # a second, ordinary row
        w = np.full((n, k), 127, np.int8)
        w[1:, ::2] = -3
        rc_ref, ref, _ = po.i8_linear(po.I8_GEMM, a, 0.5, 127, w, True, np.full(n, 1e-8, np.float32), None, None, 0,
                                      1.0, 1.0, 1.0, 0)
        assert rc_ref == (0 if expect == 0 else -1)
        wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=np.full(n, 1e-8, np.float32), version=40 + k)
        out = torch.empty((m, n), dtype=torch.int8, device="cuda")
        rc = ctx.i8_linear(po.I8_GEMM, dev(a), 0.5, 127, m, wt, out, 1.0, 0, check=False)
        assert rc == expect, (k, rc, ctx.last_error())
        if expect == 0:
            assert np.array_equal(out.cpu().numpy(), ref)
        wt.release()


def test_i8_fc_bias_overflow_declines(ctx):
    """FC adds the int32 bias into the accumulator (fc.cc:105-159), so |bias| counts toward the bound: a bias
    of magnitude near 2^31 declines (-2) although the dot products alone are small."""
    r = rng(41)
    m, k, n = 4, 256, 64
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=np.full(n, 0.01, np.float32), version=45)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    for babs, expect in ((1 << 20, 0), ((1 << 31) - 1000, -2)):
        bias = np.full(n, babs, np.int32)
        bias[::2] *= -1
        rc = ctx.i8_linear(po.I8_FC, dev(a), 0.02, 0, m, wt, out, 1.0, 0, bias=dev(bias), bias_kind=po.BIAS_VECTOR,
                           bias_abs_max=babs, check=False)
        assert rc == expect, (babs, rc, ctx.last_error())
        if expect == 0:
            rc_ref, ref, _ = po.i8_linear(po.I8_FC, a, 0.02, 0, w, True, np.full(n, 0.01, np.float32), None, bias,
                                          po.BIAS_VECTOR, 1.0, 1.0, 1.0, 0)
            assert rc_ref == 0 and np.array_equal(out.cpu().numpy(), ref)
    wt.release()


def test_weight_zero_point_declines(ctx):
    """A weight zero point != 0 (the static quantizer writes symmetric weights, static_quantizer.cc:211-255)
    is declined (-2) by the linear and the conv, and the Common kernel handles it (the oracle runs it)."""
    r = rng(42)
    m, k, n = 3, 64, 16
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    zps = np.zeros(n, np.int32)
    zps[5] = 2
    wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=np.full(n, 0.01, np.float32), zero_points=zps,
                            version=46)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    assert ctx.i8_linear(po.I8_GEMM, dev(a), 0.02, 0, m, wt, out, 1.0, 0, check=False) == -2
    rc_ref, _, _ = po.i8_linear(po.I8_GEMM, a, 0.02, 0, w, True, np.full(n, 0.01, np.float32), zps, None, 0, 1.0,
                                1.0, 1.0, 0)
    assert rc_ref == 0
    wt.release()
    wc = r.integers(-127, 128, (8, 4, 3, 3)).astype(np.int8)
    cw = ctx.prepare_conv_weight(dev(wc), np.full(8, 0.01, np.float32), zero_points=np.arange(8, dtype=np.int32),
                                 version=47)
    x = r.integers(-128, 128, (1, 4, 9, 9)).astype(np.int8)
    y = torch.empty((1, 8, 9, 9), dtype=torch.int8, device="cuda")
    assert ctx.i8_conv2d(dev(x), 0, 0.5, 0, cw, y, 1.0, 0, pad=(1, 1), check=False) == -2
    cw.release()


@pytest.mark.parametrize("kh", [1, 3])
def test_i8_conv_value_just_above_minus_half(ctx, kh):
    """Conv2D INT8 (64 input channels: the staged-window kernel) with every output's v * K = -0.5 + 1.2e-8,
    where the float-pair requantization must not round p - floor(p); the reference's code is 18."""
    c, oc, h, w_ = 64, 64, 8, 32
    x = np.zeros((1, c, h, w_), np.int8)
    x[0, 0], x[0, 1] = -127, -1
    wt = np.zeros((oc, c, kh, kh), np.int8)
    wt[:, 0, kh // 2, kh // 2], wt[:, 1, kh // 2, kh // 2] = 27, 108
    s_w = np.full(oc, float.fromhex("0x1.fc2cp-8"), np.float32)
    s_x, s_y = float.fromhex("0x1.2cdd28p-7"), float.fromhex("0x1.01dc72p-1")
    pad = (kh // 2, kh // 2)
    bias = np.zeros(oc, np.int32)
    rc, ref = po.i8_conv2d(x, s_x, 0, wt, s_w, bias, (1, 1), pad, s_y, 18)
    assert rc == 0 and ref[0, 0, h // 2, w_ // 2] == 18
    wp = ctx.prepare_conv_weight(dev(wt), s_w, group=1, version=950 + kh)
    out = torch.empty(ref.shape, dtype=torch.int8, device="cuda")
    ctx.i8_conv2d(dev(x), 0, s_x, 0, wp, out, s_y, 18, stride=(1, 1), pad=pad, bias=dev(bias), bias_abs_max=0)
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{ctx.last_backend()}: {np.count_nonzero(got != ref)} mismatches"
    wp.release()
