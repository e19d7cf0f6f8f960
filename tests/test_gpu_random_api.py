"""Seeded random cases over the whole operator surface, against the oracle: the FP8 linear with FP8, BF16 and
FP32 activations, FP8 / BF16 / FP32 outputs, vector and matrix bias with alpha/beta and general (non
power-of-two) output scales on every backend (m = 1 .. 700); INT8 MatMul/FC/Gemm with extreme zero points
and both kernels; QuantizeLinear, DequantizeLinear and Cast with NaN/Inf/subnormal inputs.  Same bars as
the focused tests (bit-exact for integer and cast work; fp8_linear_check for FP8 outputs).  Longer runs of
the same generators found the bias over-read of partial GEMM tiles, the LDS-staged GEMV's missing weight
batch and the float-pair requantization's rounding of p - floor(p)."""
import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import fp8_linear_check, fp8_pow2_scale, fp8_tensor, rng

pytestmark = pytest.mark.gpu


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def fp8_api_case(ctx, seed):
    r = rng(75000 + seed)
    dtype = int(r.choice([po.FP8E4M3, po.FP8E5M2]))
    m = int(r.choice([1, 2, 4, 9, 16, 40, 128, 300, 700]))
    k = 16 * int(r.integers(1, 129))
    n = int(r.integers(1, 900))
    layout = int(r.integers(0, 2))
    a_dt = int(r.choice([dtype, po.BF16, po.FP32]))
    out_dt = int(r.choice([dtype, dtype, po.BF16, po.FP32]))
    bias_kind = int(r.choice([po.BIAS_NONE, po.BIAS_VECTOR, po.BIAS_MATRIX]))
    alpha, beta = (1.0, 1.0) if r.random() < 0.5 else (float(r.choice([0.25, 0.5, 1.0])),
                                                      float(r.choice([-2.0, 0.5, 1.0, 3.0])))
    x = r.standard_normal((m, k)).astype(np.float32)
    w_nk, sw = fp8_tensor((r.standard_normal((n, k)) * 0.02).astype(np.float32), dtype)
    if a_dt == dtype:
        a_codes, s_in = fp8_tensor(x, dtype)
        a_src = a_codes
    else:
        a_src = po.bf16_encode(x) if a_dt == po.BF16 else x
        xv = po.bf16_decode(a_src) if a_dt == po.BF16 else x
        s_in = fp8_pow2_scale(float(np.max(np.abs(xv))), dtype)
        a_codes = po.cast_to_fp8(a_dt, a_src, dtype, s_in)
    s_out = fp8_pow2_scale(float(np.max(np.abs(po.fp8_sums(dtype, a_codes, s_in, w_nk, sw, True)))), dtype)
    if out_dt == dtype and r.random() < 0.4:
        s_out = float(np.float32(s_out * r.uniform(0.6, 0.95)))
    bias, sb, kw = None, 1.0, {}
    if bias_kind != po.BIAS_NONE:
        bias, sb = fp8_tensor(r.standard_normal((n,) if bias_kind == po.BIAS_VECTOR else (m, n)).astype(np.float32)
                              * 0.05, dtype)
        kw = dict(bias=dev(bias), bias_scale=sb, bias_kind=bias_kind)
    w_src = w_nk if layout == 1 else np.ascontiguousarray(w_nk.T)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, layout, version=1000 + seed)
    esz = {po.FP32: 4, po.BF16: 2}.get(out_dt, 1)
    out = torch.empty((m, n * esz), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a_src), a_dt, s_in, m, wt, sw, out, out_dt, s_out, alpha=alpha, beta=beta, **kw)
    be = ctx.last_backend()
    ref = po.fp8_gemm(dtype, a_codes, s_in, w_nk, sw, True, s_out, bias=bias, s_bias=sb, bias_kind=bias_kind,
                      alpha=alpha, beta=beta)
    raw = out.cpu().numpy().reshape(m, n * esz)
    label = f"seed={seed} a={a_dt} out={out_dt} m={m} k={k} n={n} bias={bias_kind} ({be})"
    if out_dt == dtype:
        codes = raw
    else:
        got = raw.view(np.float32) if out_dt == po.FP32 else raw.view(np.uint16)
        codes = po.cast_to_fp8(out_dt, got, dtype, s_out)
        assert np.array_equal(po.cast_from_fp8(dtype, codes, s_out, out_dt), got), label
    fp8_linear_check(dtype, codes, ref, a_codes, s_in * max(alpha, 1.0), w_nk, sw, s_out, label, backend=be)
    wt.release()


@pytest.mark.parametrize("chunk", range(20))
def test_random_fp8_api(ctx, chunk):
    for seed in range(chunk * 25 + 1, chunk * 25 + 26):
        fp8_api_case(ctx, seed)


def i8_case(ctx, seed):
    r = rng(90000 + seed)
    kind = int(r.choice([po.I8_GEMM, po.I8_FC, po.I8_MATMUL]))
    m = int(r.choice([1, 5, 64, 130, 384, 400, 777, 1024]))
    k = int(r.choice([16, 64, 192, 256, 512, 1024]))
    n = int(r.integers(1, 1200))
    zp_a, zp_y = int(r.integers(-128, 128)), int(r.integers(-128, 128))
    bias_kind = po.BIAS_NONE if kind == po.I8_MATMUL else int(r.choice([po.BIAS_NONE, po.BIAS_VECTOR,
                                                                         po.BIAS_MATRIX]))
    if kind == po.I8_FC and bias_kind == po.BIAS_MATRIX:
        bias_kind = po.BIAS_VECTOR
    alpha, beta = (1.0, 1.0) if kind != po.I8_GEMM or r.random() < 0.7 else (float(r.uniform(-3, 3)),
                                                                             float(r.uniform(-3, 3)))
    pow2 = r.random() < 0.3
    xq = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    if pow2:
        s_w = np.full(n, 2.0 ** int(r.integers(-10, -4)), np.float32)
        s_x, s_y = 2.0 ** int(r.integers(-6, -2)), 2.0 ** int(r.integers(-2, 3))
    else:
        s_w = r.uniform(1e-4, 1e-2, n).astype(np.float32)
        s_x, s_y = float(r.uniform(1e-3, 0.05)), float(r.uniform(0.01, 2.0))
    bias = None
    if bias_kind == po.BIAS_VECTOR:
        bias = r.integers(-30000, 30000, n).astype(np.int32)
    elif bias_kind == po.BIAS_MATRIX:
        bias = r.integers(-30000, 30000, (m, n)).astype(np.int32)
    trans_b = kind == po.I8_GEMM
    w_src = w if trans_b else np.ascontiguousarray(w.T)
    rc, ref, _ = po.i8_linear(kind, xq, s_x, zp_a, w_src, trans_b, s_w, None, bias, bias_kind, alpha, beta, s_y, zp_y)
    wt = ctx.prepare_weight(dev(w_src), po.INT8, k, n, 1 if trans_b else 0, scales=s_w, version=2000 + seed)
    out = torch.empty((m, n), dtype=torch.int8, device="cuda")
    kw = dict(bias=dev(bias), bias_kind=bias_kind, bias_abs_max=int(np.abs(bias).max())) if bias is not None else {}
    rc2 = ctx.i8_linear(kind, dev(xq), s_x, zp_a, m, wt, out, s_y, zp_y, alpha=alpha, beta=beta, check=False, **kw)
    if rc == 0 and rc2 == 0:
        got = out.cpu().numpy()
        assert np.array_equal(got, ref), (seed, kind, m, k, n, bias_kind, ctx.last_backend(),
                                          int(np.count_nonzero(got != ref)))
    else:
        assert rc2 != 0 or rc == 0, (seed, "HIP accepted a case the reference rejects")
    wt.release()


@pytest.mark.parametrize("chunk", range(20))
def test_random_i8_linear(ctx, chunk):
    for seed in range(chunk * 40 + 1, chunk * 40 + 41):
        i8_case(ctx, seed)


def _rand_bits(r, dt, shape):
    x = (r.standard_normal(shape) * float(r.choice([0.01, 1.0, 100.0, 1e4]))).astype(np.float32)
    sp = r.random(shape) < 0.01
    x[sp] = r.choice(np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, 3e38], np.float32), int(sp.sum()))
    if dt == po.FP32:
        return x
    return po.bf16_encode(x) if dt == po.BF16 else po.fp16_encode(x)


@pytest.mark.parametrize("seed", range(1, 901, 3))
def test_random_quantize_dequantize_cast(ctx, seed):
    for s in (seed, seed + 1, seed + 2):
        r = rng(77000 + s)
        op = s % 3
        if op == 0:
            dt = int(r.choice([po.FP32, po.BF16, po.FP16]))
            outer, ch, inner = int(r.integers(1, 9)), int(r.integers(1, 300)), int(r.integers(1, 9))
            x = _rand_bits(r, dt, (outer, ch, inner))
            if r.random() < 0.5 and ch > 1:
                sc = r.uniform(1e-3, 2.0, ch).astype(np.float32)
                if r.random() < 0.5:
                    sc = (2.0 ** r.integers(-8, 3, ch)).astype(np.float32)
                zp = r.integers(-128, 128, ch).astype(np.int32)
                args, axis = dict(channels=ch, inner=inner), 1
            else:
                sc = np.array([r.choice([float(r.uniform(1e-3, 2.0)), 2.0 ** int(r.integers(-8, 3))])], np.float32)
                zp = np.array([int(r.integers(-128, 128))], np.int32)
                args, axis = {}, -1
            out = torch.empty(x.shape, dtype=torch.int8, device="cuda")
            ctx.quantize_linear(dev(x), dt, sc, zp, out, **args)
            rc, ref = po.quantize_linear(dt, x, sc, zp, axis=axis)
            assert rc == 0 and np.array_equal(out.cpu().numpy(), ref), ("quantize", s)
        elif op == 1:
            dst = int(r.choice([po.FP32, po.BF16, po.FP16]))
            outer, ch, inner = int(r.integers(1, 9)), int(r.integers(1, 300)), int(r.integers(1, 9))
            q = r.integers(-128, 128, (outer, ch, inner)).astype(np.int8)
            if r.random() < 0.5 and ch > 1:
                sc = r.uniform(1e-4, 10.0, ch).astype(np.float32)
                zp = r.integers(-128, 128, ch).astype(np.int32)
                args, axis = dict(channels=ch, inner=inner), 1
            else:
                sc = np.array([r.uniform(1e-4, 10.0)], np.float32)
                zp = np.array([int(r.integers(-128, 128))], np.int32)
                args, axis = {}, -1
            out = torch.empty(q.shape, dtype=torch.float32 if dst == po.FP32 else torch.int16, device="cuda")
            ctx.dequantize_linear(dev(q), sc, zp, out, dst, **args)
            rc, ref = po.dequantize_linear(q, sc, zp, dst, axis=axis)
            assert rc == 0 and np.array_equal(out.cpu().numpy().view(np.uint8),
                                              np.ascontiguousarray(ref).view(np.uint8)), ("dequantize", s)
        else:
            f8 = int(r.choice([po.FP8E4M3, po.FP8E5M2]))
            nel = int(r.integers(1, 70000))
            scale = float(r.choice([1.0, 2.0 ** int(r.integers(-10, 10)), float(r.uniform(0.01, 10.0))]))
            if r.random() < 0.5:
                src = int(r.choice([po.FP32, po.BF16, po.FP16]))
                x = _rand_bits(r, src, (nel,))
                out = torch.empty(nel, dtype=torch.uint8, device="cuda")
                ctx.cast(dev(x), src, 1.0, out, f8, scale)
                assert np.array_equal(out.cpu().numpy(), po.cast_to_fp8(src, x, f8, scale)), ("cast to fp8", s)
            else:
                dst = int(r.choice([po.FP32, po.BF16]))
                codes = r.integers(0, 256, nel).astype(np.uint8)
                out = torch.empty(nel, dtype=torch.float32 if dst == po.FP32 else torch.int16, device="cuda")
                ctx.cast(dev(codes), f8, scale, out, dst, 1.0)
                ref = po.cast_from_fp8(f8, codes, scale, dst)
                assert np.array_equal(out.cpu().numpy().view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), \
                    ("cast from fp8", s)
