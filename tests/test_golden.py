"""The oracle against the golden fixtures in tests/golden (outputs of the reference's own code, written by
tests/golden/make_golden.py).  Runs without the reference build.

Bar: codec, QuantizeInt8Value and QuantizeAccumulator bit-exact; FP8 linear within the FP8-output
tolerance of tests/common.py (the reference's x86 kernels pre-scale the LHS and sum in another order);
argmax tokens exact.
"""
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import fp8_code_distance, fp8_linear_check

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
E4, E5 = po.FP8E4M3, po.FP8E5M2


def golden(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def codec_bits():
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    return (hi[:, None] | np.array([0x0000, 0x8000], np.uint32)[None, :]).reshape(-1)


@pytest.mark.parametrize("name,dtype", [("e4m3", E4), ("e5m2", E5)])
def test_oracle_fp8_codec_matches_golden(name, dtype):
    g = golden("codec")
    x = codec_bits().view(np.float32)
    assert np.array_equal(po.fp8_encode(dtype, x), g[f"{name}_encode"])
    dec = po.fp8_decode(dtype, np.arange(256, dtype=np.uint8)).astype(np.float32)
    assert np.array_equal(dec.view(np.uint32), g[f"{name}_decode"].view(np.uint32))


def test_oracle_bf16_codec_matches_golden():
    g = golden("codec")
    assert np.array_equal(po.bf16_encode(codec_bits().view(np.float32)), g["bf16_encode"])


def test_oracle_fp16_codecs_match_golden():
    """Cast's FP16 rule (FloatToHalf: half away from zero) and DequantizeLinear's (EncodeFloat16: RNE)."""
    g = golden("codec")
    L = po.lib()
    bits = codec_bits()
    one = np.empty(1, np.uint16)
    for key, rule in (("fp16_cast_encode", 1), ("fp16_dequant_encode", 0)):
        # through the bit-pattern entry point: a Python float would quiet signalling-NaN inputs
        got = np.empty(bits.size, np.uint16)
        for i, b in enumerate(bits.tolist()):
            L.fo_fp16_encode_bits_range(rule, b, 1, po._ptr(one))
            got[i] = one[0]
        assert np.array_equal(got, g[key]), key
    assert not np.array_equal(g["fp16_cast_encode"], g["fp16_dequant_encode"])  # the two rules do differ


def test_oracle_quantize_matches_golden():
    g = golden("quant")
    x = g["q_x"]
    for i in range(3):
        _, q = po.quantize_linear(po.FP32, x, [float(g[f"q_s{i}"])], [int(g[f"q_zp{i}"])])
        assert np.array_equal(q, g[f"q_out{i}"]), i


def test_oracle_requantize_matches_golden():
    """INT8 MatMul requantization against the reference's QuantizeAccumulator on the same accumulators."""
    g = golden("quant")
    for i in range(2):
        rc, out, _ = po.i8_linear(po.I8_MATMUL, g["rq_a"], float(g["rq_s_a"]), 0, g["rq_w"], False, g[f"rq_ws{i}"],
                                  None, None, 0, 1, 1, float(g[f"rq_s_out{i}"]), int(g[f"rq_zp{i}"]))
        assert rc == 0
        assert np.array_equal(out, g[f"rq_out{i}"]), i


@pytest.mark.parametrize("name,dtype", [("e4m3", E4), ("e5m2", E5)])
def test_oracle_fp8_linear_matches_golden(name, dtype):
    g = golden("linear")
    a, w_nk = g[f"{name}_a"], g[f"{name}_w_nk"]
    sa, sw, s_out = (float(v) for v in g[f"{name}_scales"])
    ours = po.fp8_gemm(dtype, a, sa, w_nk, sw, True, s_out)
    for key in ("direct_t0", "direct_t1", "packed"):
        fp8_linear_check(dtype, ours, g[f"{name}_{key}"], a, sa, w_nk, sw, s_out, f"oracle vs reference {key}")
    assert fp8_code_distance(g[f"{name}_direct_t0"], g[f"{name}_direct_t1"]).max() <= 1


def test_oracle_argmax_matches_golden():
    g = golden("argmax")
    a, w = g["bf16_a"], g["bf16_w"]
    assert [po.bf16_gemm_argmax(a[i], w) for i in range(a.shape[0])] == g["bf16_tokens"].tolist()
    assert g["bf16_tokens"][0] == 17  # the planted exact tie with row 1020 resolves to the lower index
    for name, dtype in (("e4m3", E4), ("e5m2", E5)):
        sa, sw, s_out = (float(v) for v in g[f"{name}_scales"])
        toks = [po.fp8_gemm_argmax(dtype, g[f"{name}_a"][i], sa, g[f"{name}_w"], sw, s_out)
                for i in range(g[f"{name}_a"].shape[0])]
        assert toks == g[f"{name}_tokens"].tolist(), name


def test_oracle_int8_gemm_and_conv_match_golden():
    """The reference's x86 INT8 Gemm (zero point, alpha/beta, bias) and Conv2D (NCHW stride 2; NHWC groups
    and dilation) outputs, bit for bit."""
    g = golden("int8")
    s_a, zp_a, alpha, beta, s_out, zp_out = (float(v) for v in g["g_params"])
    rc, out, _ = po.i8_linear(po.I8_GEMM, g["g_a"], s_a, int(zp_a), g["g_w_nk"], True, g["g_ws"], None, g["g_bias"],
                              po.BIAS_VECTOR, alpha, beta, s_out, int(zp_out))
    assert rc == 0 and np.array_equal(out, g["g_out"])
    for name in ("c0", "c1"):
        layout, group, sh, sw, ph, pw, dh, dw, zp = (int(v) for v in g[f"{name}_geom"])
        rc, out = po.i8_conv2d(g[f"{name}_x"], 0.05, zp, g[f"{name}_w"], g[f"{name}_ws"], g[f"{name}_bias"], (sh, sw),
                               (ph, pw), 0.4, 3, dilation=(dh, dw), group=group, layout=layout)
        assert rc == 0 and np.array_equal(out, g[f"{name}_out"]), name
