"""Seeded synthetic inputs shaped like BASELINE.json's configs, and comparison helpers."""
import math

import numpy as np

from oracle import pyoracle as po

SEEDS = {1: 0xFEA70001, 2: 0xFEA70002, 3: 0xFEA70003, 4: 0xFEA70004, 5: 0xFEA70005}


def rng(seed):
    return np.random.default_rng(seed)


def fp8_pow2_scale(amax, dtype):
    """Exporter rule (tools/export_qwen35_model.py:146-190): 2^ceil(log2(amax / max_finite))."""
    maxf = 448.0 if dtype == po.FP8E4M3 else 57344.0
    if not amax > 0:
        return 1.0
    return float(2.0 ** math.ceil(math.log2(amax / maxf)))


def fp8_tensor(x, dtype):
    """Encode float data with its power-of-two scale: (codes, scale)."""
    s = fp8_pow2_scale(float(np.max(np.abs(x))), dtype)
    return po.fp8_encode(dtype, np.asarray(x, np.float32) / np.float32(s)), s


def fp8_ordinal(codes):
    c = np.asarray(codes, np.int32)
    mag = c & 0x7F
    return np.where(c & 0x80, -mag, mag)


def fp8_code_distance(a, b):
    return np.abs(fp8_ordinal(a) - fp8_ordinal(b))


def bf16_bits_from_float(x):
    return po.bf16_encode(np.asarray(x, np.float32))


def same_float_bits(a, b):
    """Bitwise equality treating every NaN as equal."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.all((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b)))


def fp8_spacing_table(dtype):
    """Gap from each non-negative FP8 code to the next one (in units of the decoded value)."""
    dec = po.fp8_decode_table(dtype)
    top = 0x7E if dtype == po.FP8E4M3 else 0x7B
    gaps = np.zeros(256, np.float64)
    for c in range(top):
        gaps[c] = dec[c + 1] - dec[c]
    gaps[top:128] = gaps[top - 1]
    gaps[128:] = gaps[:128]
    return gaps


# Accumulation precision of the gfx950 FP8 MFMA (v_mfma_*_f8f6f4), measured: on sums near zero with heavy
# cancellation its result differs from the exact sum by up to ~2^-14.6 * sum_k |a_k w_k| over a 64-deep block
# (seeded comparison of 8,078 GEMMs, K = 16..4096, beyond the output code's own rounding), where fp32
# summation in any order stays within 2 * (K-1) * 2^-24 of it.  MFMA backends get this term (with 2x room).
FP8_MFMA_ACCUM_REL = 2.0 ** -13.6


def fp8_linear_check(dtype, got, ref, a_codes, sa, w_nk, sw, s_out, label="", backend=""):
    """FP8-output tolerance of the linear path.

    An element passes when its code is within 1 FP8 code of the oracle's, or -- where cancellation
    makes the accumulation error larger than an FP8 step (sums near zero) -- when the decoded values
    differ by no more than the fp32 recursive-summation bound of both orders,
    2 * (K-1) * 2^-24 * sum_k |a_k w_k|, plus one FP8 step, plus, for an MFMA backend (`backend` names
    it), the MFMA's own accumulation error FP8_MFMA_ACCUM_REL * sum_k |a_k w_k|.  A dropped, duplicated
    or mis-indexed term moves an element by ~|a_k w_k| (on average sum/K) and fails.
    Returns (exact-match rate, number of elements outside one code)."""
    d = fp8_code_distance(got, ref)
    far = np.nonzero(d > 1)
    n_far = int(far[0].size)
    if n_far:
        k = a_codes.shape[1]
        abs_sums = po.fp8_sums(dtype, a_codes & 0x7F, sa, w_nk & 0x7F, sw, True)
        dec = po.fp8_decode_table(dtype).astype(np.float64)
        gaps = fp8_spacing_table(dtype)
        g = got[far]
        r = ref[far]
        diff = np.abs(dec[g] - dec[r]) * s_out
        rel = 2.0 * (k - 1) * 2.0 ** -24 + (FP8_MFMA_ACCUM_REL if "mfma" in backend else 0.0)
        bound = rel * abs_sums[far] + np.maximum(gaps[g], gaps[r]) * s_out
        bad = diff > bound
        assert not np.any(bad), f"{label}: {int(bad.sum())} elements beyond the accumulation bound"
    exact = float(np.mean(d == 0))
    print(f"{label} exact-match {exact:.5f}, beyond-1-code (within fp32 order bound) {n_far}")
    return exact, n_far
