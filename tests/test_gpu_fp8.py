"""GPU parity of the FP8 path (Cast, decode GEMV, prefill MFMA GEMM) against the oracle.

Oracle: oracle/feather_oracle.c (Common semantics, src/kernel/common/matmul.cc:56-130, gemm.cc:62-100,
cast.cc:62-165).  Tolerance (FP8 outputs): every element within 1 FP8 code of the oracle (the fp32
accumulation order differs) or, for sums near zero, within the fp32 summation-order bound (see
tests/common.py fp8_linear_check); the exact-match rate is printed.  Cast is bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import SEEDS, fp8_code_distance, fp8_linear_check, fp8_pow2_scale, fp8_tensor, rng, same_float_bits

pytestmark = pytest.mark.gpu

FP8 = [po.FP8E4M3, po.FP8E5M2]


def dev(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


def host(t, dtype=None):
    a = t.cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


@pytest.mark.parametrize("dtype", FP8)
def test_cast_fp8_decode_all_codes(ctx, dtype):
    codes = np.arange(256, dtype=np.uint8)
    out = torch.empty(256, dtype=torch.float32, device="cuda")
    ctx.cast(dev(codes), dtype, 0.5, out, po.FP32, 1.0)
    ref = po.cast_from_fp8(dtype, codes, 0.5, po.FP32)
    got = host(out)
    bad = [(hex(c), float(got[c]), float(ref[c])) for c in range(256) if not same_float_bits(got[c:c + 1], ref[c:c + 1])]
    assert not bad, bad[:16]
    out16 = torch.empty(256, dtype=torch.int16, device="cuda")
    ctx.cast(dev(codes), dtype, 0.25, out16, po.BF16, 1.0)
    assert np.array_equal(host(out16, np.uint16), po.cast_from_fp8(dtype, codes, 0.25, po.BF16))


@pytest.mark.parametrize("dtype", FP8)
def test_cast_encode_float_patterns(ctx, dtype):
    # every sign/exponent with the top 12 mantissa bits swept and boundary low bits, plus specials
    hi = np.arange(1 << 21, dtype=np.uint32) << 11
    lows = np.array([0, 1, 0x3FF, 0x400, 0x401, 0x7FF], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).reshape(-1)
    x = bits.view(np.float32)
    for scale in (1.0, 0.0078125, 3.0):
        out = torch.empty(x.size, dtype=torch.uint8, device="cuda")
        ctx.cast(dev(x), po.FP32, 1.0, out, dtype, scale)
        ref = po.cast_to_fp8(po.FP32, x, dtype, scale)
        bad = np.nonzero(host(out) != ref)[0]
        assert bad.size == 0, f"scale {scale}: {bad.size} mismatches, first bits {bits[bad[:4]]}"


def _linear_case(seed, dtype, m, k, n, layout):
    r = rng(seed)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    a_codes, sa = fp8_tensor(x, dtype)
    w_codes, sw = fp8_tensor(w, dtype)  # [N,K]
    sums = po.fp8_sums(dtype, a_codes, sa, w_codes, sw, True)
    from tests.common import fp8_pow2_scale
    s_out = fp8_pow2_scale(float(np.max(np.abs(sums))), dtype)
    w_src = w_codes if layout == 1 else np.ascontiguousarray(w_codes.T)
    return a_codes, sa, w_codes, w_src, sw, s_out


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("m", [1, 3, 4, 16])
@pytest.mark.parametrize("layout", [0, 1])
def test_fp8_gemv_matches_oracle(ctx, dtype, m, layout):
    k, n = 1024, 3584
    a, sa, w_nk, w_src, sw, s_out = _linear_case(SEEDS[2] + m, dtype, m, k, n, layout)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, layout, version=1)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out)
    assert ctx.last_backend().startswith("fp8_gemv")
    ref = po.fp8_gemm(dtype, a, sa, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, host(out), ref, a, sa, w_nk, sw, s_out, f"gemv m={m}", backend=ctx.last_backend())
    wt.release()


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("m", [1, 5, 16])
def test_fp8_gemv_long_k_non_pow2_scale(ctx, dtype, m):
    """Down-projection shape (K = 3584: 28 MFMA steps, so each wave runs two load batches) with a
    non-power-of-two output scale, which takes the general MFMA GEMV at every m (including m = 1)."""
    k, n = 3584, 1024
    a, sa, w_nk, w_src, sw, s_out = _linear_case(SEEDS[2] + 100 + m, dtype, m, k, n, 1)
    s_out = float(np.float32(s_out * 1.37))
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=7)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out)
    assert ctx.last_backend() == "fp8_gemv_mfma"
    ref = po.fp8_gemm(dtype, a, sa, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, host(out), ref, a, sa, w_nk, sw, s_out, f"gemv long k m={m}", backend=ctx.last_backend())
    wt.release()


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("m", [1, 4, 7, 16])
def test_fp8_gemv_fused_bf16_io(ctx, dtype, m):
    """bf16 activations -> Cast(fp8) -> MatMul -> Cast(bf16), fused: equals the three-node chain."""
    k, n = 1024, 3584
    r = rng(SEEDS[2])
    x = r.standard_normal((m, k)).astype(np.float32)
    xb = po.bf16_encode(x)
    w = (r.standard_normal((k, n)) * 0.02).astype(np.float32)
    w_codes, sw = fp8_tensor(w, dtype)  # [K,N] MatMul layout
    from tests.common import fp8_pow2_scale
    s_in = fp8_pow2_scale(float(np.max(np.abs(po.bf16_decode(xb)))), dtype)
    a_codes = po.cast_to_fp8(po.BF16, xb, dtype, s_in)
    s_out = fp8_pow2_scale(float(np.max(np.abs(po.fp8_sums(dtype, a_codes, s_in, w_codes, sw, False)))), dtype)
    wt = ctx.prepare_weight(dev(w_codes), dtype, k, n, 0, version=2)
    out = torch.empty((m, n), dtype=torch.int16, device="cuda")
    ctx.fp8_linear(dev(xb), po.BF16, s_in, m, wt, sw, out, po.BF16, s_out)
    ref_codes = po.fp8_matmul(dtype, a_codes, s_in, w_codes, sw, s_out)
    ref = po.cast_from_fp8(dtype, ref_codes, s_out, po.BF16)
    got = host(out, np.uint16)
    got_codes = po.cast_to_fp8(po.BF16, got, dtype, s_out)  # bf16 of an fp8 value re-encodes exactly
    assert np.array_equal(po.cast_from_fp8(dtype, got_codes, s_out, po.BF16), got)
    fp8_linear_check(dtype, got_codes, ref_codes, a_codes, s_in, np.ascontiguousarray(w_codes.T), sw, s_out,
                     "fused bf16", backend=ctx.last_backend())
    assert np.mean(got == ref) > 0.97
    wt.release()


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("shape", [(256, 1024, 512), (100, 384, 200), (200, 320, 300), (300, 128, 520),
                                   (4096, 1024, 3584), (4000, 1152, 3584), (4096, 3584, 1024)])
def test_fp8_mfma_gemm_matches_oracle(ctx, dtype, shape):
    m, k, n = shape
    a, sa, w_nk, w_src, sw, s_out = _linear_case(SEEDS[3] + m, dtype, m, k, n, 1)
    if m * n > 1 << 21:
        # full-size case: a seeded subset of rows plus the last rows (a partial row tile when m % 256 != 0)
        rows = np.union1d(rng(7).choice(m, 96, replace=False), np.arange(m - 8, m))
    else:
        rows = np.arange(m)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=3)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out)
    assert ctx.last_backend().startswith("fp8_mfma_gemm")
    ref = po.fp8_gemm(dtype, a[rows], sa, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, host(out)[rows], ref, a[rows], sa, w_nk, sw, s_out, f"gemm {shape}", backend=ctx.last_backend())
    wt.release()


def _encode_probe_values(dtype, count, seed):
    """Activation values (in units of the activation scale) that exercise the FP8 encode: every finite
    code's value, the midpoints between neighbouring codes (round-half-even ties), values past the
    largest finite code (saturation), subnormal-range and sub-subnormal magnitudes, both zeros."""
    codes = np.arange(256, dtype=np.uint8)
    vals = po.fp8_decode(dtype, codes).astype(np.float64)
    fin = np.sort(np.unique(vals[np.isfinite(vals) & (vals >= 0)]))
    mids = (fin[:-1] + fin[1:]) / 2
    maxf = fin[-1]
    extra = np.array([maxf * 1.01, maxf * 1.2, maxf * 4, fin[1] / 2, fin[1] / 3, fin[1] / 2 * 1.0001, 0.0])
    pos = np.concatenate([fin, mids, extra])
    v = np.concatenate([pos, -pos, [-0.0]])
    r = rng(seed)
    v = np.concatenate([v, r.standard_normal(count) * maxf / 4])[:count]
    return r.permutation(v).astype(np.float32)


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("src", [po.FP32, po.BF16])
@pytest.mark.parametrize("m,staged", [(1, False), (3, False), (8, False), (3, True)])
def test_fp8_gemv_m1_activation_encode_exact(ctx, dtype, src, m, staged):
    """With an identity weight (code of 1.0 on the diagonal, w_scale 1) and out_scale = a_scale, every
    output code equals the activation's own Cast code, so the fused encode inside the decode kernels is
    checked bit-exactly against the reference Cast: the M=1 kernel (m = 1) and the register-encoding MFMA
    kernel (m = 3, 8); with `staged`, activation rows that start off a 16-byte boundary take the
    LDS-staged MFMA kernel.  K = N = 1088 (padded 1152) makes the M=1 kernel stage the row in two passes
    and walk the weight row in two chunks per lane."""
    k = n = 1088
    s_in = 0.25
    v = np.stack([_encode_probe_values(dtype, k, 31 + i) for i in range(m)])
    x = (v * np.float32(s_in)).astype(np.float32).reshape(m, k)
    xin = x if src == po.FP32 else po.bf16_encode(x)
    one = int(po.fp8_encode(dtype, np.array([1.0], np.float32))[0])
    w = np.zeros((k, n), np.uint8)
    w[np.arange(k), np.arange(n)] = one
    wt = ctx.prepare_weight(dev(w), dtype, k, n, 0, version=6)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    xd = dev(xin)
    if staged:  # same rows, one element past a 16-byte boundary
        buf = torch.zeros(xd.numel() + 8, dtype=xd.dtype, device="cuda")
        buf[1:1 + xd.numel()] = xd.reshape(-1)
        xd = buf[1:1 + xd.numel()].view(m, k)
    ctx.fp8_linear(xd, src, s_in, m, wt, 1.0, out, dtype, s_in)
    assert ctx.last_backend() == ("fp8_gemv_m1" if m == 1 else "fp8_gemv_mfma")
    a_codes = po.cast_to_fp8(src, xin, dtype, s_in)
    ref = po.fp8_matmul(dtype, a_codes, s_in, w, 1.0, s_in)
    got = host(out)
    bad = np.nonzero(got != ref)
    assert bad[0].size == 0, f"{bad[0].size} mismatches: x={x[bad][:4]} got={got[bad][:4]} ref={ref[bad][:4]}"
    wt.release()


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("out_dtype", [po.BF16, po.FP32])
@pytest.mark.parametrize("shape", [(300, 3584, 1024), (4096, 1024, 3584), (4000, 1024, 3584)])
def test_fp8_gemm_decoded_outputs(ctx, dtype, out_dtype, shape):
    """BF16 / FP32 outputs (the FP8 code decoded with out_scale, as the exported Gemm -> Cast pair) on a
    down-projection-like shape (K = 3584, 128-deep stages) and the up-projection shape (BF16: 256x224
    tiles), whole and with a partial last row tile: each output must be exactly a decoded FP8 code and those codes meet the FP8 tolerance."""
    m, k, n = shape
    a, sa, w_nk, w_src, sw, s_out = _linear_case(SEEDS[3] + 17, dtype, m, k, n, 1)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=8)
    tdt = torch.int16 if out_dtype == po.BF16 else torch.float32
    out = torch.empty((m, n), dtype=tdt, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, out_dtype, s_out)
    assert ctx.last_backend().startswith("fp8_mfma_gemm")
    got = host(out, np.uint16) if out_dtype == po.BF16 else host(out)
    codes = po.cast_to_fp8(out_dtype, got, dtype, s_out)
    assert np.array_equal(po.cast_from_fp8(dtype, codes, s_out, out_dtype).view(got.dtype), got)
    # sampled rows plus the last ones (m = 4000: a partial last row tile on the 256x224 path)
    rows = np.union1d(rng(9).choice(m, 64, replace=False), np.arange(m - 8, m))
    ref = po.fp8_gemm(dtype, a[rows], sa, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, codes[rows], ref, a[rows], sa, w_nk, sw, s_out, f"gemm out {out_dtype}", backend=ctx.last_backend())
    wt.release()


def test_fp8_gemm_bias_alpha_beta(ctx):
    dtype = po.FP8E4M3
    m, k, n = 64, 256, 96
    a, sa, w_nk, w_src, sw, s_out = _linear_case(11, dtype, m, k, n, 1)
    bias_f = rng(12).standard_normal(n).astype(np.float32) * 0.1
    bias, sb = fp8_tensor(bias_f, dtype)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=4)
    for mm in (m, 8, 1):
        out = torch.empty((mm, n), dtype=torch.uint8, device="cuda")
        ctx.fp8_linear(dev(a[:mm]), dtype, sa, mm, wt, sw, out, dtype, s_out, bias=dev(bias), bias_scale=sb,
                       bias_kind=po.BIAS_VECTOR, alpha=0.5, beta=2.0)
        ref = po.fp8_gemm(dtype, a[:mm], sa, w_nk, sw, True, s_out, bias=bias, s_bias=sb, bias_kind=po.BIAS_VECTOR,
                          alpha=0.5, beta=2.0)
        assert fp8_code_distance(host(out), ref).max() <= 1  # |sums| >> bias: no near-zero cancellation
    wt.release()


@pytest.mark.parametrize("out_dtype", [po.FP32, po.BF16])
def test_fp8_gemv_bias_alpha_beta_decoded_outputs(ctx, out_dtype):
    """Decode GEMV (m = 4 and 16, the register kernel's specialized output tail for power-of-two output
    scales) with a vector bias, alpha and beta, writing decoded FP32 / BF16: the values re-encode to codes
    within one of the oracle's, and decode exactly."""
    dtype = po.FP8E4M3
    k, n = 256, 96
    a, sa, w_nk, w_src, sw, s_out = _linear_case(13, dtype, 16, k, n, 1)
    bias_f = rng(14).standard_normal(n).astype(np.float32) * 0.1
    bias, sb = fp8_tensor(bias_f, dtype)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=5)
    for mm in (4, 16):
        esz = 4 if out_dtype == po.FP32 else 2
        out = torch.empty((mm, n * esz), dtype=torch.uint8, device="cuda")
        ctx.fp8_linear(dev(a[:mm]), dtype, sa, mm, wt, sw, out, out_dtype, s_out, bias=dev(bias), bias_scale=sb,
                       bias_kind=po.BIAS_VECTOR, alpha=0.5, beta=2.0)
        assert ctx.last_backend() == "fp8_gemv_mfma"
        ref = po.fp8_gemm(dtype, a[:mm], sa, w_nk, sw, True, s_out, bias=bias, s_bias=sb, bias_kind=po.BIAS_VECTOR,
                          alpha=0.5, beta=2.0)
        raw = host(out).reshape(mm, n * esz)
        got = raw.view(np.float32) if out_dtype == po.FP32 else raw.view(np.uint16)
        codes = po.cast_to_fp8(out_dtype, got, dtype, s_out)
        assert np.array_equal(po.cast_from_fp8(dtype, codes, s_out, out_dtype), got)
        assert fp8_code_distance(codes, ref).max() <= 1
    wt.release()


def test_fp8_gemm_bias_alpha_beta_full_size(ctx):
    """Bias, alpha and beta on the up-projection shape (256x224 tiles, power-of-two output scale with a
    bias: the unfolded epilogue); a seeded subset of rows against the oracle."""
    dtype = po.FP8E5M2
    m, k, n = 4096, 1024, 3584
    a, sa, w_nk, w_src, sw, s_out = _linear_case(13, dtype, m, k, n, 1)
    bias_f = rng(14).standard_normal(n).astype(np.float32) * 0.1
    bias, sb = fp8_tensor(bias_f, dtype)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=9)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out, bias=dev(bias), bias_scale=sb,
                   bias_kind=po.BIAS_VECTOR, alpha=0.5, beta=2.0)
    assert ctx.last_backend() == "fp8_mfma_gemm_256x224_bk128_w8"
    rows = np.union1d(rng(15).choice(m, 64, replace=False), np.arange(m - 4, m))
    ref = po.fp8_gemm(dtype, a[rows], sa, w_nk, sw, True, s_out, bias=bias, s_bias=sb, bias_kind=po.BIAS_VECTOR,
                      alpha=0.5, beta=2.0)
    # the bias is added after the sum, in the reference's order, so only the sum's accumulation order differs;
    # alpha < 1 scales that error down, so the unscaled bound of fp8_linear_check holds
    fp8_linear_check(dtype, host(out)[rows], ref, a[rows], sa, w_nk, sw, s_out, "gemm bias full size", backend=ctx.last_backend())
    wt.release()


def test_fp8_linear_rejects_bad_scale(ctx):
    dtype = po.FP8E4M3
    a, sa, w_nk, w_src, sw, s_out = _linear_case(13, dtype, 2, 64, 32, 1)
    wt = ctx.prepare_weight(dev(w_src), dtype, 64, 32, 1, version=5)
    out = torch.empty((2, 32), dtype=torch.uint8, device="cuda")
    rc = ctx.fp8_linear(dev(a), dtype, float("nan"), 2, wt, sw, out, dtype, s_out, check=False)
    assert rc == -1
    rc = ctx.fp8_linear(dev(a), dtype, sa, 2, wt, sw, out, dtype, 0.0, check=False)
    assert rc == -1
    wt.release()


def _special_case(dtype, m, k, n, seed):
    """Activations with NaN / Inf codes planted in a few rows, everything else N(0,1); returns the codes,
    the planted rows and the usual scales."""
    a, sa, w_nk, w_src, sw, s_out = _linear_case(seed, dtype, m, k, n, 1)
    a = a.copy()
    nan = 0x7F if dtype == po.FP8E4M3 else 0x7E
    plants = {3: [nan], 7: [nan | 0x80]}
    if dtype == po.FP8E5M2:
        plants[11] = [0x7C]        # +Inf: Inf * w gives +-Inf per column, NaN where w == 0
        plants[13] = [0xFC, 0x7C]  # -Inf and +Inf in one row: NaN
    for r, codes in plants.items():
        for j, c in enumerate(codes):
            a[r, 5 + 17 * j] = c
    return a, sa, w_nk, w_src, sw, s_out, sorted(plants)


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("shape", [(256, 512, 384), (4096, 256, 3584)])
@pytest.mark.parametrize("mode", ["folded", "pow2_alpha", "general"])
def test_fp8_gemm_special_values_and_saturation(ctx, dtype, shape, mode):
    """NaN/Inf inputs and outputs far beyond the largest finite code, through each epilogue scale mode:
    a power-of-two output factor folded into the MFMA block scale, a power-of-two output scale with a
    non-power-of-two alpha, and a non-power-of-two output scale.  The output scale is 1/16 of the one
    that fits the sums, so most large outputs saturate; special and saturated codes must match exactly."""
    m, k, n = shape
    a, sa, w_nk, w_src, sw, s_fit, special_rows = _special_case(dtype, m, k, n, SEEDS[3] + 7 * m + k)
    s_out = s_fit / 16 if mode != "general" else s_fit / 16 * 1.37
    alpha = 0.3 if mode == "pow2_alpha" else 1.0
    rows = np.union1d(np.arange(16), rng(9).choice(m, 48, replace=False)) if m > 1024 else np.arange(m)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=5)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out, alpha=alpha)
    assert ctx.last_backend().startswith("fp8_mfma_gemm")
    got = host(out)[rows]
    ref = po.fp8_gemm(dtype, a[rows], sa, w_nk, sw, True, s_out, alpha=alpha)
    dec = po.fp8_decode_table(dtype)
    maxf = np.nanmax(np.abs(dec[np.isfinite(dec)]))
    ref_val = dec[ref]
    must_match = ~np.isfinite(ref_val) | np.isnan(ref_val) | (np.abs(ref_val) >= maxf)
    sums = po.fp8_sums(dtype, a[rows], sa, w_nk, sw, True) * alpha / s_out
    must_match &= ~np.isfinite(sums) | (np.abs(sums) >= 2 * maxf)  # far past the top code: no rounding doubt
    assert must_match.sum() > 100
    # a NaN's sign comes from the arithmetic that made it (x86 and the GPU differ for Inf - Inf), so NaN
    # outputs are compared as NaN; Inf and saturated codes, with their signs, are compared exactly
    ref_nan = np.isnan(ref_val)
    assert np.all(np.isnan(dec[got][ref_nan]))
    mism = np.nonzero(must_match & ~ref_nan & (got != ref))
    assert mism[0].size == 0, f"{mism[0].size} special/saturated mismatches, first got {got[mism][:8]} ref {ref[mism][:8]}"
    for r in special_rows:
        i = int(np.nonzero(rows == r)[0][0])
        assert np.all(~np.isfinite(dec[got[i]]) | (np.abs(dec[got[i]]) >= maxf))
    keep = ~must_match
    ordinary = np.setdiff1d(np.arange(rows.size), [int(np.nonzero(rows == r)[0][0]) for r in special_rows])
    fp8_linear_check(dtype, np.where(keep, got, 0)[ordinary].astype(np.uint8),
                     np.where(keep, ref, 0)[ordinary].astype(np.uint8), a[rows][ordinary], sa, w_nk, sw, s_out,
                     f"special {shape} {mode}", backend=ctx.last_backend())
    wt.release()


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("m,k", [(9, 1000), (13, 260), (6, 1003)])
def test_fp8_gemv_fp32_input_ragged_k(ctx, dtype, m, k):
    """fp32 activations with a non-power-of-two input scale (the encode divides) and K not a multiple of
    the 128-deep MFMA step; k = 1003 is not a multiple of 4 either (the LDS-staged kernel).  The fused
    Cast must give the codes of Cast(fp32 -> fp8) of the same rows."""
    n = 520
    r = rng(SEEDS[2] + m * 1000 + k)
    x = r.standard_normal((m, k)).astype(np.float32)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    w_codes, sw = fp8_tensor(w, dtype)
    s_in = float(np.float32(np.max(np.abs(x)) / 300.0))
    a_codes = po.cast_to_fp8(po.FP32, x, dtype, s_in)
    from tests.common import fp8_pow2_scale
    s_out = fp8_pow2_scale(float(np.max(np.abs(po.fp8_sums(dtype, a_codes, s_in, w_codes, sw, True)))), dtype)
    wt = ctx.prepare_weight(dev(w_codes), dtype, k, n, 1, version=8)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(x), po.FP32, s_in, m, wt, sw, out, dtype, s_out)
    assert ctx.last_backend() == "fp8_gemv_mfma"
    ref = po.fp8_gemm(dtype, a_codes, s_in, w_codes, sw, True, s_out)
    fp8_linear_check(dtype, host(out), ref, a_codes, s_in, w_codes, sw, s_out, f"gemv fp32 m={m} k={k}", backend=ctx.last_backend())
    wt.release()


@pytest.mark.parametrize("dtype", FP8)
@pytest.mark.parametrize("src", [po.FP32, po.BF16])
@pytest.mark.parametrize("k", [1000, 1004, 2000, 2048])
def test_fp8_gemv_m1_k_tails(ctx, dtype, src, k):
    """The M=1 decode kernel with power-of-two scales at K that is a multiple of 16 (2048: 16-byte chunk
    loads, two chunks per lane) and that is not (1000, 1004, 2000: per-group loads, a partial last chunk):
    the fused Cast must give the codes of Cast(src -> fp8), and the outputs the FP8 tolerance."""
    n = 1040
    r = rng(SEEDS[2] + 7 * k + src)
    x = r.standard_normal((1, k)).astype(np.float32)
    xin = x if src == po.FP32 else po.bf16_encode(x)
    from tests.common import fp8_pow2_scale
    s_in = fp8_pow2_scale(float(np.max(np.abs(po.bf16_decode(po.bf16_encode(x))))), dtype)
    a_codes = po.cast_to_fp8(src, xin, dtype, s_in)
    w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
    w_codes, sw = fp8_tensor(w, dtype)
    s_out = fp8_pow2_scale(float(np.max(np.abs(po.fp8_sums(dtype, a_codes, s_in, w_codes, sw, True)))), dtype)
    wt = ctx.prepare_weight(dev(w_codes), dtype, k, n, 1, version=10)
    out = torch.empty((1, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(xin), src, s_in, 1, wt, sw, out, dtype, s_out)
    assert ctx.last_backend() == "fp8_gemv_m1"
    ref = po.fp8_gemm(dtype, a_codes, s_in, w_codes, sw, True, s_out)
    fp8_linear_check(dtype, host(out), ref, a_codes, s_in, w_codes, sw, s_out, f"gemv m1 k={k}", backend=ctx.last_backend())
    wt.release()


@pytest.mark.parametrize("bias_kind", [po.BIAS_VECTOR, po.BIAS_MATRIX])
@pytest.mark.parametrize("m,k,n", [(40, 912, 578), (300, 176, 174)])
def test_fp8_gemm_bias_partial_tiles(ctx, bias_kind, m, k, n):
    """Bias on the tile GEMM with partial tiles in M and N: the epilogue evaluates positions past m and n
    (never stored) and must read the bias only inside its m x n (or n) values; general output scale."""
    dtype = po.FP8E4M3
    a, sa, w_nk, w_src, sw, s_out = _linear_case(31, dtype, m, k, n, 1)
    s_out = float(np.float32(s_out * 0.7))  # not a power of two: the general scale mode
    shape = (n,) if bias_kind == po.BIAS_VECTOR else (m, n)
    bias, sb = fp8_tensor(rng(32).standard_normal(shape).astype(np.float32) * 0.05, dtype)
    wt = ctx.prepare_weight(dev(w_src), dtype, k, n, 1, version=11)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, s_out, bias=dev(bias), bias_scale=sb,
                   bias_kind=bias_kind, alpha=0.5, beta=2.0)
    assert ctx.last_backend().startswith("fp8_mfma_gemm_")
    ref = po.fp8_gemm(dtype, a, sa, w_nk, sw, True, s_out, bias=bias, s_bias=sb, bias_kind=bias_kind, alpha=0.5,
                      beta=2.0)
    fp8_linear_check(dtype, host(out), ref, a, sa, w_nk, sw, s_out, f"gemm bias {bias_kind} {m}x{k}x{n}",
                     backend=ctx.last_backend())
    wt.release()


@pytest.mark.parametrize("k", [128, 368, 800])
def test_fp8_gemv_m1_general_output_scale_short_k(ctx, k):
    """m = 1 with a non power-of-two output scale runs the LDS-staged MFMA GEMV; with m * kp / 4 below the
    block's 256 threads some threads stage no activations and must still issue their first weight batch."""
    dtype = po.FP8E4M3
    n = 272
    r = rng(33 + k)
    x = r.standard_normal((1, k)).astype(np.float32)
    w_nk, sw = fp8_tensor((r.standard_normal((n, k)) * 0.02).astype(np.float32), dtype)
    s_in = fp8_pow2_scale(float(np.max(np.abs(x))), dtype)
    a_codes = po.cast_to_fp8(po.FP32, x, dtype, s_in)
    s_out = float(np.float32(fp8_pow2_scale(float(np.max(np.abs(po.fp8_sums(dtype, a_codes, s_in, w_nk, sw, True)))),
                                            dtype) * 0.8))
    wt = ctx.prepare_weight(dev(w_nk), dtype, k, n, 1, version=12)
    out = torch.empty((1, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(x), po.FP32, s_in, 1, wt, sw, out, dtype, s_out)
    assert ctx.last_backend() == "fp8_gemv_mfma"
    ref = po.fp8_gemm(dtype, a_codes, s_in, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, host(out), ref, a_codes, s_in, w_nk, sw, s_out, f"gemv m1 general k={k}",
                     backend=ctx.last_backend())
    wt.release()
