"""Writes the golden fixtures of this directory from the reference's own code.

The outputs come from oracle/_ref/libfeather_ref.so, which `make -C oracle ref` compiles from the Feather
sources themselves: include/util/fp8.h (FloatToFp8E4M3/E5M2, Fp8*ToFloat), include/util/bf16.h
(FloatToBFloat16), include/util/fp16.h (FloatToHalf, Cast's FP16 rule), quantize_linear_utils.h (EncodeFloat16), include/quant/quantization.h (QuantizeInt8Value), src/kernel/common/int8_kernel_utils.h
(QuantizeAccumulator), src/kernel/x86/linear_fp8.cc (ComputeLinearRowMajorX86Fp8*, the packed
TransposedRhsArgmax), src/kernel/x86/linear.cc (the packed BF16 argmax) and src/kernel/x86/int8.cc (the INT8
Gemm and Conv2D kernels).  Only inputs and the
reference's outputs are stored, so the oracle and the HIP path can be checked against the reference
where that build is absent (the GPU box).

    python tests/golden/make_golden.py        # needs oracle/_ref, i.e. the Feather tree
"""
import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import pyoracle as po  # noqa: E402

E4, E5 = po.FP8E4M3, po.FP8E5M2
LOW_BITS = (0x0000, 0x8000)  # with every float32 upper half: exact values and round-half-even ties


def codec_bits():
    """Every float32 upper half (sign, exponent, top 7 mantissa bits) joined with each of LOW_BITS."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    return (hi[:, None] | np.array(LOW_BITS, np.uint32)[None, :]).reshape(-1)


def make_codec(R):
    bits = codec_bits()
    out = {}
    one8 = np.empty(1, np.uint8)
    one16 = np.empty(1, np.uint16)
    for name, d in (("e4m3", E4), ("e5m2", E5)):
        enc = np.empty(bits.size, np.uint8)
        for i, b in enumerate(bits.tolist()):
            R.ref_fp8_encode_bits_range(d, b, 1, po._ptr(one8))
            enc[i] = one8[0]
        out[f"{name}_encode"] = enc
        out[f"{name}_decode"] = np.array([R.ref_fp8_decode(d, c) for c in range(256)], np.float32)
    bf = np.empty(bits.size, np.uint16)
    for i, b in enumerate(bits.tolist()):
        R.ref_bf16_encode_bits_range(b, 1, po._ptr(one16))
        bf[i] = one16[0]
    out["bf16_encode"] = bf
    for name, rule in (("fp16_cast_encode", 1), ("fp16_dequant_encode", 0)):
        h = np.empty(bits.size, np.uint16)
        for i, b in enumerate(bits.tolist()):
            R.ref_fp16_encode_bits_range(rule, b, 1, po._ptr(one16))
            h[i] = one16[0]
        out[name] = h
    return out


def make_quant(R):
    r = np.random.default_rng(0xFEA70101)
    # QuantizeInt8Value: exact .5 ties at a power-of-two scale, saturation, signed zeros, random values
    ties = (np.arange(-300, 301, dtype=np.float32) + np.float32(0.5)) * np.float32(0.25)
    x = np.concatenate([ties, np.float32([0.0, -0.0, 1e30, -1e30, 31.75, -32.125]),
                        r.standard_normal(2000).astype(np.float32) * np.float32(40)]).astype(np.float32)
    out = {"q_x": x}
    for i, (s, zp) in enumerate(((0.25, 0), (0.25, 7), (0.3, -5))):
        q = np.empty(x.size, np.int8)
        R.ref_quantize_int8_values(po._ptr(x), x.size, s, zp, po._ptr(q))
        out[f"q_s{i}"] = np.float32(s)
        out[f"q_zp{i}"] = np.int32(zp)
        out[f"q_out{i}"] = q
    # QuantizeAccumulator (requantization of the INT8 MatMul): exact int64 accumulators of a @ w, then the
    # reference's requant; power-of-two scales make exact .5 ties (acc an odd multiple of 2^10 here)
    m, k, n = 16, 64, 48
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (k, n)).astype(np.int8)
    acc = (a.astype(np.int64) @ w.astype(np.int64)).astype(np.int32)
    out.update(rq_a=a, rq_w=w, rq_s_a=np.float32(0.0625))
    for i, (ws, s_out, zp) in enumerate(((np.full(n, 2.0 ** -6, np.float32), 2.0, 3),
                                         (r.uniform(1e-3, 1e-2, n).astype(np.float32), 0.37, -4))):
        q = np.empty((m, n), np.int8)
        assert R.ref_requantize(po._ptr(acc), m, n, 0.0625, po._ptr(ws), n, s_out, zp, po._ptr(q)) == 0
        out[f"rq_ws{i}"] = ws
        out[f"rq_s_out{i}"] = np.float32(s_out)
        out[f"rq_zp{i}"] = np.int32(zp)
        out[f"rq_out{i}"] = q
    return out


def pow2_scale(amax, dtype):
    maxf = 448.0 if dtype == E4 else 57344.0
    return float(2.0 ** np.ceil(np.log2(amax / maxf)))


def make_linear(R):
    """x86 FP8 linear (direct kernels for m = 5; the prepared M = 1 decode kernel per row)."""
    r = np.random.default_rng(0xFEA70102)
    out = {}
    m, k, n = 5, 256, 64
    for name, d in (("e4m3", E4), ("e5m2", E5)):
        x = r.standard_normal((m, k)).astype(np.float32)
        w = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
        sa, sw = pow2_scale(np.abs(x).max(), d), pow2_scale(np.abs(w).max(), d)
        a = po.fp8_encode(d, x / np.float32(sa))
        w_nk = po.fp8_encode(d, w / np.float32(sw))
        s_out = pow2_scale(float(np.abs(po.fp8_sums(d, a, sa, w_nk, sw, True)).max()), d)
        out[f"{name}_a"], out[f"{name}_w_nk"] = a, w_nk
        out[f"{name}_scales"] = np.float32([sa, sw, s_out])
        for tb in (0, 1):
            rw = w_nk if tb else np.ascontiguousarray(w_nk.T)
            y = np.empty((m, n), np.uint8)
            assert R.ref_fp8_linear(d, po._ptr(a), sa, po._ptr(rw), sw, tb, None, 1.0, 0, 1.0, 1.0, m, k, n,
                                    po._ptr(y), s_out) == 0
            out[f"{name}_direct_t{tb}"] = y
        h = R.ref_fp8_packed_create(d, po._ptr(np.ascontiguousarray(w_nk.T)), 0, k, n)
        yp = np.empty((m, n), np.uint8)
        for i in range(m):
            row = np.ascontiguousarray(a[i:i + 1])
            dst = np.empty((1, n), np.uint8)
            assert R.ref_fp8_packed_compute(h, po._ptr(row), sa, sw, 1, po._ptr(dst), s_out) == 0
            yp[i] = dst[0]
        R.ref_fp8_packed_destroy(h)
        out[f"{name}_packed"] = yp
    return out


def make_argmax(R):
    r = np.random.default_rng(0xFEA70103)
    out = {}
    k, v, rows = 128, 1031, 4
    a = po.bf16_encode(r.standard_normal((rows, k)).astype(np.float32))
    w = po.bf16_encode((r.standard_normal((v, k)) * 0.02).astype(np.float32))
    # rows 17 and 1020 are equal and lead for activation row 0: the lower index must win
    w[1020] = po.bf16_encode(np.sign(po.bf16_decode(a[0])) * np.float32(0.06))
    w[17] = w[1020]
    w[40, 3] = 0x7FC0  # a NaN row is never selected
    a[3] = a[2]
    tok = ctypes.c_int64()
    h = R.ref_bf16_argmax_create(po._ptr(w), k, v)
    toks = []
    for i in range(rows):
        assert R.ref_bf16_argmax_compute(h, po._ptr(np.ascontiguousarray(a[i])), ctypes.byref(tok)) == 0
        toks.append(tok.value)
    R.ref_bf16_argmax_destroy(h)
    out.update(bf16_a=a, bf16_w=w, bf16_tokens=np.int64(toks))
    for name, d in (("e4m3", E4), ("e5m2", E5)):
        x = r.standard_normal((rows, k)).astype(np.float32)
        wf = (r.standard_normal((v, k)) * 0.02).astype(np.float32)
        sa, sw = pow2_scale(np.abs(x).max(), d), pow2_scale(np.abs(wf).max(), d)
        ac = po.fp8_encode(d, x / np.float32(sa))
        wc = po.fp8_encode(d, wf / np.float32(sw))
        s_out = pow2_scale(float(np.abs(po.fp8_sums(d, ac, sa, wc, sw, True)).max()), d)
        h = R.ref_fp8_packed_create(d, po._ptr(wc), 1, k, v)
        toks = []
        for i in range(rows):
            assert R.ref_fp8_packed_argmax(h, po._ptr(np.ascontiguousarray(ac[i])), sa, sw, s_out, ctypes.byref(tok)) == 0
            toks.append(tok.value)
        R.ref_fp8_packed_destroy(h)
        out[f"{name}_a"], out[f"{name}_w"] = ac, wc
        out[f"{name}_scales"] = np.float32([sa, sw, s_out])
        out[f"{name}_tokens"] = np.int64(toks)
    return out


def make_int8(R):
    """The reference's x86 INT8 Gemm (transB, zero point, alpha/beta, bias) and Conv2D (NCHW stride 2; NHWC
    with groups and dilation).  Seeds are taken where the x86 conv's float requantization agrees with the
    Common kernel everywhere (they differ only within float rounding of a round-half point), so every stored
    output is also the Common result."""
    from tests.test_oracle_ref_int8 import _x86_conv, _x86_gemm
    out = {}
    r = np.random.default_rng(0xFEA70104)
    m, k, n = 24, 192, 80
    a = r.integers(-128, 128, (m, k)).astype(np.int8)
    w = r.integers(-127, 128, (n, k)).astype(np.int8)
    ws = r.uniform(1e-3, 1e-2, n).astype(np.float32)
    bias = r.integers(-20000, 20000, n).astype(np.int32)
    rc, y = _x86_gemm(a, 0.03, -4, w, ws, bias, 0.75, -1.5, 0.05, 2)
    assert rc == 0
    out.update(g_a=a, g_w_nk=w, g_ws=ws, g_bias=bias, g_params=np.float32([0.03, -4, 0.75, -1.5, 0.05, 2]), g_out=y)
    cases = (("c0", 0, 16, 32, 1, (2, 2), (1, 1), (1, 1), 0), ("c1", 1, 32, 48, 2, (1, 2), (2, 1), (2, 1), -6))
    for name, layout, c, oc, group, stride, pad, dil, zp in cases:
        for seed in range(100):
            rr = np.random.default_rng(0xFEA70105 + 1000 * seed + c)
            x = rr.integers(-128, 128, (1, c, 18, 22)).astype(np.int8)
            xl = x if layout == 0 else np.ascontiguousarray(x.transpose(0, 2, 3, 1))
            wc = rr.integers(-127, 128, (oc, c // group, 3, 3)).astype(np.int8)
            wcs = rr.uniform(1e-3, 1e-2, oc).astype(np.float32)
            cb = rr.integers(-3000, 3000, oc).astype(np.int32)
            rc, yx = _x86_conv(xl, layout, 0.05, zp, wc, group, wcs, cb, stride, pad, dil, 0.4, 3)
            rco, yo = po.i8_conv2d(xl, 0.05, zp, wc, wcs, cb, stride, pad, 0.4, 3, dilation=dil, group=group,
                                   layout=layout)
            if rc == 0 and rco == 0 and np.array_equal(yx, yo):
                break
        else:
            raise RuntimeError(f"no seed with x86 == Common for {name}")
        out.update({f"{name}_x": xl, f"{name}_w": wc, f"{name}_ws": wcs, f"{name}_bias": cb, f"{name}_out": yx,
                    f"{name}_geom": np.int32([layout, group, *stride, *pad, *dil, zp])})
    return out


def main():
    R = po.ref()
    for name, fn in (("codec", make_codec), ("quant", make_quant), ("linear", make_linear), ("argmax", make_argmax),
                     ("int8", make_int8)):
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn(R))
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
