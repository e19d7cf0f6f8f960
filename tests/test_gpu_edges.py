"""Edge cases of the C ABI on the GPU: empty inputs succeed without launching (the reference's Common
kernels loop zero times and return 0), empty K / N / vocabulary are declined (the Common kernel then
decides), and ragged K (not a multiple of 4, 16 or 64) takes the per-element staging paths.

Oracle for the ragged cases: oracle/feather_oracle.c, FP8 tolerance of tests/common.py.
"""
import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from tests.common import fp8_linear_check, fp8_tensor, fp8_pow2_scale, rng

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def test_empty_inputs_succeed(ctx):
    L = ctx.lib
    h = ctx.handle
    k, n = 64, 32
    w8 = dev(np.zeros((n, k), np.int8))
    wt = ctx.prepare_weight(w8, po.INT8, k, n, 1, scales=[0.01], version=50)
    wf = ctx.prepare_weight(dev(np.zeros((n, k), np.uint8)), po.FP8E4M3, k, n, 1, version=51)
    assert L.fhip_fp8_linear(h, po.FP8E4M3, None, 1.0, 0, wf.handle, 1.0, None, 1.0, 0, 1.0, 1.0, po.FP8E4M3, None,
                             1.0) == 0
    assert L.fhip_i8_linear(h, po.I8_MATMUL, None, 1.0, 0, 0, wt.handle, None, 0, 0, 1.0, 1.0, None, 1.0, 0) == 0
    assert L.fhip_cast(h, po.FP32, None, 1.0, 0, po.FP8E4M3, None, 1.0) == 0
    sc = np.array([1.0], np.float32)
    zp = np.array([0], np.int32)
    assert L.fhip_quantize_linear(h, po.FP32, None, 0, 1, 1, po._ptr(sc), po._ptr(zp), 1, None) == 0
    assert L.fhip_dequantize_linear(h, None, 0, 1, 1, po._ptr(sc), po._ptr(zp), 1, po.FP32, None) == 0
    assert L.fhip_bf16_gemv_argmax(h, None, 0, 64, None, 100, None, None) == 0
    wt.release()
    wf.release()


def test_empty_k_or_vocabulary_is_declined(ctx):
    L = ctx.lib
    h = ctx.handle
    a = dev(np.zeros((1, 64), np.int16))
    w = dev(np.zeros((16, 64), np.int16))
    tok = torch.empty(1, dtype=torch.int64, device="cuda")
    assert L.fhip_bf16_gemv_argmax(h, a.data_ptr(), 1, 64, w.data_ptr(), 0, tok.data_ptr(), None) == -2
    assert L.fhip_bf16_gemv_argmax(h, a.data_ptr(), 1, 0, w.data_ptr(), 16, tok.data_ptr(), None) == -2
    import ctypes
    out = ctypes.c_void_p()
    assert L.fhip_weight_prepare(h, w.data_ptr(), po.FP8E4M3, 0, 16, 1, None, 0, None, 0, 1, ctypes.byref(out)) == -2


@pytest.mark.parametrize("dtype", [po.FP8E4M3, po.FP8E5M2])
@pytest.mark.parametrize("m", [1, 5, 40])
def test_fp8_linear_ragged_k(ctx, dtype, m):
    """K = 99: not a multiple of 4 (per-element activation staging), 16 or 64 (zero-padded weight and
    staged GEMM operand); bf16 activations in, FP8 out."""
    k, n = 99, 70
    r = rng(60 + m)
    x = r.standard_normal((m, k)).astype(np.float32)
    xb = po.bf16_encode(x)
    w_nk, sw = fp8_tensor((r.standard_normal((n, k)) * 0.05).astype(np.float32), dtype)
    s_in = fp8_pow2_scale(float(np.abs(po.bf16_decode(xb)).max()), dtype)
    a_codes = po.cast_to_fp8(po.BF16, xb, dtype, s_in)
    s_out = fp8_pow2_scale(float(np.abs(po.fp8_sums(dtype, a_codes, s_in, w_nk, sw, True)).max()), dtype)
    wt = ctx.prepare_weight(dev(w_nk), dtype, k, n, 1, version=52)
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(dev(xb.view(np.int16)), po.BF16, s_in, m, wt, sw, out, dtype, s_out)
    ref = po.fp8_gemm(dtype, a_codes, s_in, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, out.cpu().numpy(), ref, a_codes, s_in, w_nk, sw, s_out, f"ragged k m={m}", backend=ctx.last_backend())
    wt.release()


@pytest.mark.parametrize("layout", [0, 1])
def test_weight_prepare_from_host_matches_device(ctx, layout):
    """Load-time preparation from host bytes gives the same prepared weight as the device path: the
    outputs of an FP8 linear through either are identical; the host copy is cached on its address."""
    dtype = po.FP8E4M3
    k, n, m = 1024, 700, 3
    r = rng(70 + layout)
    w_nk, sw = fp8_tensor((r.standard_normal((n, k)) * 0.02).astype(np.float32), dtype)
    src = w_nk if layout == 1 else np.ascontiguousarray(w_nk.T)
    a, sa = fp8_tensor(r.standard_normal((m, k)).astype(np.float32), dtype)
    wd = ctx.prepare_weight(dev(src), dtype, k, n, layout, version=80)
    wh = ctx.prepare_weight_host(src, dtype, k, n, layout, version=80)
    assert ctx.last_backend() == "weight_prepare_host"
    wh2 = ctx.prepare_weight_host(wh.source, dtype, k, n, layout, version=80)
    assert ctx.last_backend() == "weight_cache_hit"
    outs = []
    for wt in (wd, wh):
        out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
        ctx.fp8_linear(dev(a), dtype, sa, m, wt, sw, out, dtype, 0.5)
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    for wt in (wd, wh, wh2):
        wt.release()


def test_fp8_gemm_activations_past_the_offset_limit(ctx):
    """The prefill GEMM addresses its operands with 32-bit offsets from buffer resources; activations of
    2^31 bytes or more run as several launches over row blocks.  m*k = 2,147,500,032 here (two blocks,
    the second of 257 rows), checked on the rows around the block boundary, the last rows and a seeded
    sample."""
    dtype = po.FP8E4M3
    m, k, n = 131073, 16384, 256
    g = torch.Generator(device="cuda")
    g.manual_seed(0xFEA70F01)
    # finite e4m3 codes of magnitude <= 0.234 (0x00..0x2f) with random signs: sums stay far from saturation
    a = torch.randint(0, 0x30, (m, k), generator=g, device="cuda", dtype=torch.uint8)
    a |= (torch.randint(0, 2, (m, k), generator=g, device="cuda", dtype=torch.uint8) << 7)
    r = rng(0xFEA70F02)
    w_nk = po.fp8_encode(dtype, (r.standard_normal((n, k)) * 0.5).astype(np.float32))
    wt = ctx.prepare_weight(torch.from_numpy(w_nk).cuda(), dtype, k, n, 1, version=9)
    sa, sw, s_out = 1.0, 1.0, 2.0
    out = torch.empty((m, n), dtype=torch.uint8, device="cuda")
    ctx.fp8_linear(a, dtype, sa, m, wt, sw, out, dtype, s_out)
    assert ctx.last_backend().startswith("fp8_mfma_gemm")
    boundary = ((1 << 31) - 1) // k // 256 * 256
    rows = np.union1d(np.union1d(np.arange(boundary - 12, boundary + 12), np.arange(m - 12, m)),
                      r.choice(m, 16, replace=False))
    a_rows = a[torch.from_numpy(rows).cuda()].cpu().numpy()
    ref = po.fp8_gemm(dtype, a_rows, sa, w_nk, sw, True, s_out)
    fp8_linear_check(dtype, out.cpu().numpy()[rows], ref, a_rows, sa, w_nk, sw, s_out, "gemm past 2^31", backend=ctx.last_backend())
    del a, out
    torch.cuda.empty_cache()
    wt.release()
