"""GPU parity of the INT8 linear's large-M path (the MFMA tile GEMM in its INT8 mode): bit-exact against the
oracle for Gemm / FC / MatMul, both weight layouts, zero points, vector and matrix bias, alpha/beta, ragged M
and N, both stage depths (K a multiple of 128, or of 64 only), both tile sizes, exact requantization ties
(power-of-two scales) and the fused DequantizeLinear outputs."""
import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import rng

pytestmark = pytest.mark.gpu


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


CASES = [
    # m, k, n, kind, bias_kind, zp_a, zp_y, alpha, beta, pow2 scales, backend
    (512, 1024, 1024, po.I8_GEMM, po.BIAS_VECTOR, 0, 0, 1.0, 1.0, False, "i8_mfma_gemm_128x128_bk128_w8"),
    (420, 192, 700, po.I8_GEMM, po.BIAS_MATRIX, -20, 10, 0.75, -1.5, True, "i8_mfma_gemm_128x128_w8"),
    (3000, 256, 4000, po.I8_GEMM, po.BIAS_VECTOR, 7, -4, 1.0, 1.0, False, "i8_mfma_gemm_256x256_bk128_w8"),
    (3100, 320, 3900, po.I8_FC, po.BIAS_VECTOR, -3, 2, 1.0, 1.0, True, "i8_mfma_gemm_256x256_w8"),
    (385, 128, 33, po.I8_MATMUL, po.BIAS_NONE, 12, 0, 1.0, 1.0, False, "i8_mfma_gemm_128x128_bk128_w8"),
    (777, 64, 515, po.I8_GEMM, po.BIAS_NONE, 0, -1, 2.0, 0.0, True, "i8_mfma_gemm_128x128_w8"),
    (4000, 128, 3584, po.I8_FC, po.BIAS_VECTOR, 9, -6, 1.0, 1.0, False, "i8_mfma_gemm_256x224_bk128_w8"),
    (4000, 256, 3584, po.I8_GEMM, po.BIAS_MATRIX, -4, 3, 1.0, 1.0, True, "i8_mfma_gemm_256x224_bk128_w8"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}_k{c[3]}" for c in CASES])
def test_i8_tile_gemm_bitexact(ctx, case):
    m, k, n, kind, bias_kind, zp_a, zp_y, alpha, beta, pow2, backend = case
    r = rng(m * 7 + n)
    xq = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    if pow2:
        s_w = np.full(n, 2.0 ** -8, np.float32)
        s_x, s_y = 0.0625, 2.0
    else:
        s_w = r.uniform(1e-3, 1e-2, n).astype(np.float32)
        s_x, s_y = 0.02, 0.4
    bias = None
    if bias_kind == po.BIAS_VECTOR:
        bias = r.integers(-20000, 20000, n).astype(np.int32)
    elif bias_kind == po.BIAS_MATRIX:
        bias = r.integers(-3000, 3000, (m, n)).astype(np.int32)
    trans_b = kind == po.I8_GEMM
    w_src = w if trans_b else np.ascontiguousarray(w.T)
    rc, ref, _ = po.i8_linear(kind, xq, s_x, zp_a, w_src, trans_b, s_w, None, bias, bias_kind, alpha, beta, s_y, zp_y)
    assert rc == 0
    wt = ctx.prepare_weight(dev(w_src), po.INT8, k, n, 1 if trans_b else 0, scales=s_w, version=300 + m)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    kw = {}
    if bias is not None:
        kw = dict(bias=dev(bias), bias_kind=bias_kind, bias_abs_max=int(np.abs(bias).max()))
    ctx.i8_linear(kind, dev(xq), s_x, zp_a, m, wt, out, s_y, zp_y, alpha=alpha, beta=beta, **kw)
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} mismatches ({ctx.last_backend()})"
    assert ctx.last_backend() == backend
    wt.release()


@pytest.mark.parametrize("out_dtype", [po.FP32, po.FP16, po.BF16])
@pytest.mark.parametrize("m,k,n", [(600, 512, 1000), (2048, 256, 3000), (4000, 128, 3500), (4000, 128, 3584)])
def test_i8_tile_gemm_fused_dequantize(ctx, out_dtype, m, k, n):
    r = rng(m + n + out_dtype)
    xq = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, n).astype(np.float32)
    bias = r.integers(-20000, 20000, n).astype(np.int32)
    s_x, s_y, zp_y, s_dq, zp_dq = 0.02, 0.0371, -6, 0.0125, 3
    rc, yq, _ = po.i8_linear(po.I8_GEMM, xq, s_x, 0, w, True, s_w, None, bias, po.BIAS_VECTOR, 1.0, 1.0, s_y, zp_y)
    assert rc == 0
    rc, ref = po.dequantize_linear(yq, [s_dq], [zp_dq], out_dtype)
    assert rc == 0
    wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=s_w, version=400 + m)
    tdt = torch.float32 if out_dtype == po.FP32 else torch.int16
    out = torch.empty((m, n), dtype=tdt, device="cuda")
    ctx.i8_linear_ex(po.I8_GEMM, dev(xq), s_x, 0, m, wt, out, out_dtype, s_y, zp_y, dq_scale=s_dq, dq_zp=zp_dq,
                     bias=dev(bias), bias_kind=po.BIAS_VECTOR, bias_abs_max=20000)
    assert ctx.last_backend().startswith("i8_mfma_gemm_")
    got = out.cpu().numpy()
    if out_dtype != po.FP32:
        got = got.view(np.uint16)
    assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8))
    wt.release()


def test_i8_tile_gemm_unaligned_activation_uses_small_tiles(ctx):
    """An activation pointer off 16-byte alignment keeps the K-split kernels, with the same result."""
    r = rng(77)
    m, k, n = 512, 256, 256
    buf = r.integers(-128, 128, m * k + 16).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    s_w = r.uniform(1e-3, 1e-2, n).astype(np.float32)
    xq = buf[1:1 + m * k].reshape(m, k)
    rc, ref, _ = po.i8_linear(po.I8_GEMM, xq, 0.02, 0, w, True, s_w, None, None, po.BIAS_NONE, 1.0, 1.0, 0.4, 0)
    assert rc == 0
    wt = ctx.prepare_weight(dev(w), po.INT8, k, n, 1, scales=s_w, version=500)
    dbuf = dev(buf)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    ctx.i8_linear(po.I8_GEMM, dbuf[1:1 + m * k].view(m, k), 0.02, 0, m, wt, out, 0.4, 0)
    assert ctx.last_backend().endswith("_ksplit4")
    assert np.array_equal(out.cpu().numpy(), ref)
    wt.release()


def test_i8_tile_gemm_sums_beyond_2_24(ctx):
    """Sums of magnitude above 2^24 (not exact in fp32: the integer path hands them to the fp64 pass) with an
    output scale that keeps most codes unclamped, next to small sums in the same tile."""
    r = rng(91)
    m, k, n = 512, 4096, 256
    sign_a = r.choice([-1, 1], (m, 1))
    sign_w = r.choice([-1, 1], (n, 1))
    xq = (sign_a * r.integers(100, 128, (m, k))).astype(np.int8)
    xq[::7] = r.integers(-128, 128, (len(xq[::7]), k)).astype(np.int8)  # small sums in every tile
    w = (sign_w * r.integers(100, 128, (n, k))).astype(np.int8)
    w_kn = np.ascontiguousarray(w.T)  # FC weights are [K, N]
    s_w = r.uniform(9e-4, 1.1e-3, n).astype(np.float32)
    s_x, s_y = 0.01, 6.45
    for zp_y in (0, -37):
        rc, ref, _ = po.i8_linear(po.I8_FC, xq, s_x, 0, w_kn, False, s_w, None, None, po.BIAS_NONE, 1.0, 1.0, s_y,
                                  zp_y)
        assert rc == 0
        assert np.count_nonzero(np.abs(ref.astype(int) - zp_y) < 100) > ref.size // 4
        wt = ctx.prepare_weight(dev(w_kn), po.INT8, k, n, 0, scales=s_w, version=600)
        out = torch.empty((m, n), dtype=torch.int8, device="cuda")
        ctx.i8_linear(po.I8_FC, dev(xq), s_x, 0, m, wt, out, s_y, zp_y)
        assert ctx.last_backend().startswith("i8_mfma_gemm_")
        got = out.cpu().numpy()
        assert np.array_equal(got, ref), f"zp_y={zp_y}: {np.count_nonzero(got != ref)} mismatches"
        wt.release()


@pytest.mark.parametrize("m", [100, 512])
def test_i8_linear_near_ties(ctx, m):
    """s_a * s_w / s_out = 0.5 * (1 + 2^-22): every odd sum lands a few 1e-7 .. 1e-4 from an x.5 point, inside
    the fp32 screen's margin but decided by the float-pair form (and exactly on x.5 for s_w = 1); both
    kernels (K-split for m = 100, tile for m = 512)."""
    r = rng(95 + m)
    k, n = 64, 256
    xq = r.integers(-2, 3, (m, k)).astype(np.int8)
    w = r.integers(-2, 3, (n, k)).astype(np.int8)
    s_w = np.where(np.arange(n) % 2 == 0, np.float32(1.0 + 2.0 ** -22), np.float32(1.0)).astype(np.float32)
    w_kn = np.ascontiguousarray(w.T)
    for zp_y in (0, 3, -7):
        rc, ref, _ = po.i8_linear(po.I8_FC, xq, 0.5, 0, w_kn, False, s_w, None, None, po.BIAS_NONE, 1.0, 1.0, 1.0,
                                  zp_y)
        assert rc == 0
        wt = ctx.prepare_weight(dev(w_kn), po.INT8, k, n, 0, scales=s_w, version=800 + m)
        out = torch.empty((m, n), dtype=torch.int8, device="cuda")
        ctx.i8_linear(po.I8_FC, dev(xq), 0.5, 0, m, wt, out, 1.0, zp_y)
        got = out.cpu().numpy()
        assert np.array_equal(got, ref), f"zp_y={zp_y} ({ctx.last_backend()}): {np.count_nonzero(got != ref)} mismatches"
        wt.release()


@pytest.mark.parametrize("m", [100, 512])
def test_i8_linear_value_just_above_minus_half(ctx, m):
    """A sum whose v * K is -0.5 + 1.2e-8: fl32(v * kh) rounds to -0.49999997, where p - floor(p) = p + 1 is not
    exact in fp32 (the float-pair form must use p - (floor(p) + 0.5)).  Reference code: round(17.500000012) = 18."""
    k, n = 64, 128
    xq = np.zeros((m, k), np.int8)
    xq[:, 0], xq[:, 1] = -127, -1
    w = np.zeros((n, k), np.int8)
    w[:, 0], w[:, 1] = 27, 108  # dot = -3537 in every column
    w[1::2, 1] = 107  # and -3429 - 107 = -3536 in odd columns
    s_w = np.full(n, float.fromhex("0x1.fc2cp-8"), np.float32)
    s_x, s_y = float.fromhex("0x1.2cdd28p-7"), float.fromhex("0x1.01dc72p-1")
    w_kn = np.ascontiguousarray(w.T)
    rc, ref, _ = po.i8_linear(po.I8_FC, xq, s_x, 0, w_kn, False, s_w, None, None, po.BIAS_NONE, 1.0, 1.0, s_y, 18)
    assert rc == 0 and ref[0, 0] == 18
    wt = ctx.prepare_weight(dev(w_kn), po.INT8, k, n, 0, scales=s_w, version=900 + m)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    ctx.i8_linear(po.I8_FC, dev(xq), s_x, 0, m, wt, out, s_y, 18)
    got = out.cpu().numpy()
    assert np.array_equal(got, ref), f"{ctx.last_backend()}: {np.count_nonzero(got != ref)} mismatches"
    wt.release()
