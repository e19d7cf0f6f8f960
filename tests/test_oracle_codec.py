"""Pins of the oracle's and the shipped device codec's FP8/BF16/FP16 conversions.

- Known answers transcribed from the reference's test/fp8_test.cc:254-279.
- Exhaustive (all 2^32 float patterns) equality of the oracle encoders with the reference's own
  header codec (include/util/fp8.h, include/util/bf16.h compiled into oracle/_ref).
- Exhaustive equality of the shipped device codec (infer_amd/csrc/codec.h, host build) with the oracle.
"""
import ctypes
import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from oracle import pyoracle as po

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
E4, E5 = po.FP8E4M3, po.FP8E5M2


def enc(d, x):
    return po.lib().fo_fp8_encode(d, x)


def test_fp8_known_answers():
    inf, nan = float("inf"), float("nan")
    assert enc(E4, 1.0) == 0x38
    assert enc(E4, 0.001953125) == 0x01
    assert enc(E4, 0.015625) == 0x08
    assert enc(E4, 448.0) == 0x7E
    assert enc(E4, inf) == 0x7E
    assert enc(E4, nan) == 0x7F
    assert enc(E4, 1.0625) == 0x38
    assert enc(E4, 1.1875) == 0x3A
    assert enc(E5, 1.0) == 0x3C
    assert enc(E5, 0.0000152587890625) == 0x01
    assert enc(E5, 0.00006103515625) == 0x04
    assert enc(E5, 57344.0) == 0x7B
    assert enc(E5, inf) == 0x7C
    assert enc(E5, nan) == 0x7D
    assert enc(E5, 1.125) == 0x3C
    assert enc(E5, 1.375) == 0x3E
    dec = po.lib().fo_fp8_decode
    assert dec(E4, 0x01) == 0.001953125 and dec(E4, 0x08) == 0.015625 and dec(E4, 0x7E) == 448.0
    assert dec(E5, 0x01) == 0.0000152587890625 and dec(E5, 0x04) == 0.00006103515625 and dec(E5, 0x7B) == 57344.0
    # saturation, negative zero, sign symmetry, NaN/Inf decode
    assert enc(E4, 1e9) == 0x7E and enc(E4, -1e9) == 0xFE and enc(E5, -1e9) == 0xFB
    assert enc(E4, -0.0) == 0x80 and enc(E4, -1e-30) == 0x80
    assert np.isnan(dec(E4, 0x7F)) and np.isnan(dec(E4, 0xFF)) and np.isinf(dec(E5, 0x7C))
    assert dec(E5, 0xFC) == -inf


def test_fp8_decode_is_closed_form():
    """Every code decodes to (-1)^s 2^(e-bias) (1 + m/2^M) (normal) or 2^(1-bias) m/2^M (subnormal)."""
    for d, M, bias in ((E4, 3, 7), (E5, 2, 15)):
        for c in range(256):
            s, e, m = c >> 7, (c & 0x7F) >> M, c & ((1 << M) - 1)
            v = po.lib().fo_fp8_decode(d, c)
            if (d == E4 and e == 15 and m == 7) or (d == E5 and e == 31):
                continue
            ref = (2.0 ** (1 - bias) * m / 2 ** M) if e == 0 else 2.0 ** (e - bias) * (1 + m / 2 ** M)
            assert v == (-ref if s else ref), (d, hex(c))


def test_fp8_encode_round_trip_and_rounding_brute_force():
    """Encode is round-to-nearest-even onto the decode table (brute force over representable values)."""
    r = np.random.default_rng(1)
    for d in (E4, E5):
        table = po.fp8_decode_table(d).astype(np.float64)
        finite = np.array([c for c in range(128) if np.isfinite(table[c])])
        vals = table[finite]
        maxf = vals.max()
        x = np.concatenate([r.standard_normal(20000) * s for s in (1e-6, 1e-3, 1.0, 1e2, 1e4)]).astype(np.float32)
        x = x[np.abs(x) <= maxf]
        got = po.fp8_encode(d, x)
        ax = np.abs(x.astype(np.float64))
        # positive codes 0..max decode to increasing values: bracket |x| and pick the nearer code,
        # the even code (even mantissa) on a tie
        lo = np.searchsorted(vals, ax, side="right") - 1
        hi = np.minimum(lo + 1, len(vals) - 1)
        dlo, dhi = ax - vals[lo], vals[hi] - ax
        exp_code = np.where(dlo < dhi, finite[lo], np.where(dhi < dlo, finite[hi],
                            np.where(finite[lo] % 2 == 0, finite[lo], finite[hi])))
        assert np.array_equal(got & 0x7F, exp_code)


@pytest.mark.skipif(not po.ref_available(), reason="reference build (oracle/_ref) not present")
@pytest.mark.parametrize("kind", ["e4m3", "e5m2", "bf16", "bf16_plain", "fp16_cast", "fp16_dequant"])
def test_exhaustive_against_reference_codec(kind):
    """All 2^32 float inputs: the oracle's encoders against the reference's own -- FloatToFp8E4M3/E5M2,
    FloatToBFloat16, EncodeBFloat16 (DequantizeLinear's BF16 rule, no NaN quieting), FloatToHalf (Cast's FP16
    rule) and EncodeFloat16 (DequantizeLinear's FP16 rule)."""
    L, R = po.lib(), po.ref()
    chunk = 1 << 24

    def run(i):
        if kind == "bf16":
            a = np.empty(chunk, np.uint16)
            b = np.empty(chunk, np.uint16)
            L.fo_bf16_encode_bits_range(i * chunk, chunk, po._ptr(a))
            R.ref_bf16_encode_bits_range(i * chunk, chunk, po._ptr(b))
        elif kind == "bf16_plain":
            a = np.empty(chunk, np.uint16)
            b = np.empty(chunk, np.uint16)
            L.fo_bf16_plain_encode_bits_range(i * chunk, chunk, po._ptr(a))
            R.ref_bf16_plain_encode_bits_range(i * chunk, chunk, po._ptr(b))
        elif kind.startswith("fp16"):
            rule = 1 if kind == "fp16_cast" else 0
            a = np.empty(chunk, np.uint16)
            b = np.empty(chunk, np.uint16)
            L.fo_fp16_encode_bits_range(rule, i * chunk, chunk, po._ptr(a))
            R.ref_fp16_encode_bits_range(rule, i * chunk, chunk, po._ptr(b))
        else:
            d = E4 if kind == "e4m3" else E5
            a = np.empty(chunk, np.uint8)
            b = np.empty(chunk, np.uint8)
            L.fo_fp8_encode_bits_range(d, i * chunk, chunk, po._ptr(a))
            R.ref_fp8_encode_bits_range(d, i * chunk, chunk, po._ptr(b))
        return int(np.count_nonzero(a != b))

    with ThreadPoolExecutor(8) as ex:
        bad = sum(ex.map(run, range(256)))
    assert bad == 0
    if kind.startswith("fp16"):  # both FP16 decoders on every code
        for h in range(1 << 16):
            x = np.float32(L.fo_fp16_decode(h))
            for rule in (0, 1):
                y = np.float32(R.ref_fp16_decode(rule, h))
                assert x.tobytes() == y.tobytes() or (np.isnan(x) and np.isnan(y) and
                                                      (x.view(np.uint32) & 0xFFBFFFFF) == (y.view(np.uint32) & 0xFFBFFFFF)), hex(h)
    if kind in ("e4m3", "e5m2"):
        d = E4 if kind == "e4m3" else E5
        for c in range(256):
            x, y = np.float32(L.fo_fp8_decode(d, c)), np.float32(R.ref_fp8_decode(d, c))
            assert x.tobytes() == y.tobytes(), hex(c)


def test_shipped_device_codec_exhaustive(tmp_path):
    """infer_amd/csrc/codec.h (the kernels' codec) compiled for the host equals the oracle on every input."""
    exe = tmp_path / "codec_check"
    subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-x", "c++",
                    os.path.join(ROOT, "tests", "native", "codec_check.cc"), "-x", "c",
                    os.path.join(ROOT, "oracle", "feather_oracle.c"), "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0 and out.stdout.strip().endswith("OK"), out.stdout[-2000:]
