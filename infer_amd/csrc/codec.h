// codec.h -- FP8 (OCP e4m3fn / e5m2), BF16 and FP16 conversions with Feather's exact rounding
// and special-value rules, usable in device code and (for the CPU exhaustive check) host code.
//
// Semantics follow the reference codecs:
//   FP8 encode  include/util/fp8.h:66-211   round-to-nearest-even, finite overflow saturates to the
//               largest finite code; e4m3: Inf -> 0x7e|s, NaN -> 0x7f|s; e5m2: Inf -> 0x7c|s,
//               NaN -> 0x7d|s; values below half the smallest subnormal give a signed zero.
//   FP8 decode  include/util/fp8.h:158-200  every NaN code decodes to +qNaN (0x7fc00000).
//   BF16        include/util/bf16.h:27-46   RNE, NaN quieted by OR-ing 0x40 into the high half.
//   BF16 plain  src/kernel/common/quantize_linear_utils.h:110-117 (RNE, no NaN special case).
//   FP16        src/kernel/common/quantize_linear_utils.h:50-101.
// The encoders round the float's significand once at the FP8 quantum of its binade, using
// integer operations only (no division), so they are exact on every input.
#ifndef FHIP_CODEC_H
#define FHIP_CODEC_H

#include <stdint.h>

#if defined(__HIPCC__)
#define FHIP_HD __host__ __device__ __forceinline__
#else
#define FHIP_HD inline
#endif

namespace fhip {

FHIP_HD uint32_t f32_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __float_as_uint(f);
#else
    union { float f; uint32_t u; } v;
    v.f = f;
    return v.u;
#endif
}

FHIP_HD float bits_f32(uint32_t u) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __uint_as_float(u);
#else
    union { float f; uint32_t u; } v;
    v.u = u;
    return v.f;
#endif
}

// mant >> shift rounded to nearest, ties to even; shift in [1, 63].
FHIP_HD uint32_t round_shift_rne(uint32_t mant, int shift) {
    if (shift >= 32) return 0u;  // mant < 2^24: the value is below one half of the unit
    const uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
}

// E5M2 when `e5m2`, otherwise E4M3 (OCP fn: no infinity, single NaN mantissa).
FHIP_HD uint8_t fp8_encode(float value, bool e5m2) {
    const int mbits = e5m2 ? 2 : 3;
    const int emin = e5m2 ? -14 : -6;                       // exponent of the smallest normal
    const uint32_t max_bits = e5m2 ? 0x47600000u : 0x43e00000u;  // 57344 : 448
    const uint32_t u = f32_bits(value);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {
        const uint32_t special = a == 0x7f800000u ? (e5m2 ? 0x7cu : 0x7eu) : (e5m2 ? 0x7du : 0x7fu);
        return (uint8_t)(sign | special);
    }
    if (a > max_bits) return (uint8_t)(sign | (e5m2 ? 0x7bu : 0x7eu));
    const int fexp = (int)(a >> 23);
    const uint32_t mant = fexp == 0 ? (a & 0x7fffffu) : ((a & 0x7fffffu) | 0x800000u);
    const int e = fexp == 0 ? -126 : fexp - 127;
    if (e < emin) {
        // Subnormal FP8: count of quanta 2^(emin - mbits); a carry to 2^mbits is the smallest normal.
        return (uint8_t)(sign | round_shift_rne(mant, 23 - mbits + (emin - e)));
    }
    uint32_t q = round_shift_rne(mant, 23 - mbits);  // in [2^mbits, 2^(mbits+1)]
    int ef = e - emin + 1;                            // biased FP8 exponent field
    if (q == (2u << mbits)) {
        q >>= 1;
        ++ef;
    }
    return (uint8_t)(sign | ((uint32_t)ef << mbits) | (q & ((1u << mbits) - 1u)));
}

FHIP_HD float fp8_decode(uint8_t code, bool e5m2) {
    const int mbits = e5m2 ? 2 : 3;
    const uint32_t ef = (uint32_t)(code & 0x7f) >> mbits;
    const uint32_t m = code & ((1u << mbits) - 1u);
    const uint32_t sign = (uint32_t)(code & 0x80) << 24;
    if (e5m2 ? ef == 31u : (ef == 15u && m == 7u)) {
        if (e5m2 && m == 0u) return bits_f32(sign | 0x7f800000u);
        return bits_f32(0x7fc00000u);
    }
    if (ef == 0u) {
        // m * 2^(emin - mbits): exact in float
        const float v = (float)m * (e5m2 ? 1.52587890625e-05f : 0.001953125f);
        return bits_f32(f32_bits(v) | sign);
    }
    const uint32_t fexp = ef + (e5m2 ? 112u : 120u);  // rebias 15 -> 127 or 7 -> 127
    return bits_f32(sign | (fexp << 23) | (m << (23 - mbits)));
}

FHIP_HD uint16_t bf16_encode(float value) {
    const uint32_t u = f32_bits(value);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu) != 0u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

FHIP_HD uint16_t bf16_encode_plain(float value) {
    const uint32_t u = f32_bits(value);
    const uint32_t low = u & 0xffffu;
    uint32_t high = u >> 16;
    if (low > 0x8000u || (low == 0x8000u && (high & 1u))) ++high;
    return (uint16_t)high;
}

FHIP_HD float bf16_decode(uint16_t b) { return bits_f32((uint32_t)b << 16); }

FHIP_HD uint16_t fp16_encode(float value) {
    const uint32_t u = f32_bits(value);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t fexp = (u >> 23) & 0xffu;
    const uint32_t frac = u & 0x7fffffu;
    if (fexp == 0xffu) return (uint16_t)(sign | 0x7c00u | (frac ? 0x200u : 0u));
    const int he = (int)fexp - 112;
    if (he >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)sign;
        return (uint16_t)(sign | round_shift_rne(frac | 0x800000u, 14 - he));
    }
    const uint32_t r = round_shift_rne(frac | 0x800000u, 13);  // 11 significant bits
    if (r == 0x800u) return (uint16_t)(sign | ((uint32_t)(he + 1) << 10));
    return (uint16_t)(sign | ((uint32_t)he << 10) | (r & 0x3ffu));
}

// FP16 encode of the Cast operator (include/util/fp16.h FloatToHalf, used by src/kernel/common/cast.cc:98).
// It differs from fp16_encode above (DequantizeLinear's encoder): the magnitude is rounded half away
// from zero at the FP16 quantum, magnitudes below 2^-24 become a signed zero, and a NaN keeps its top
// 10 payload bits with the lowest bit forced on.
FHIP_HD uint16_t fp16_encode_cast(float value) {
    const uint32_t u = f32_bits(value);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t fexp = (u >> 23) & 0xffu;
    const uint32_t frac = u & 0x7fffffu;
    if (fexp == 0xffu) return (uint16_t)(sign | 0x7c00u | (frac ? ((frac >> 13) | 1u) : 0u));
    const int e = (int)fexp - 127;  // unbiased exponent
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e < -24) return (uint16_t)sign;
    if (e < -14) {
        // subnormal result: the significand (hidden bit included) keeps its top bits, half away rounds up
        const int drop = -e - 1;  // bits of the 24-bit significand below the FP16 quantum 2^-24
        const uint32_t sig = frac | 0x800000u;
        return (uint16_t)(sign | ((sig + (1u << (drop - 1))) >> drop));
    }
    // normal result: round the 23-bit fraction to 10 bits, half away; a carry bumps the exponent
    uint32_t he = (uint32_t)(e + 15);
    uint32_t f = frac + 0x1000u;
    if (f & 0x800000u) {
        f = 0;
        if (++he >= 0x1fu) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | (he << 10) | (f >> 13));
}

FHIP_HD float fp16_decode(uint16_t b) {
    const uint32_t sign = (uint32_t)(b & 0x8000u) << 16;
    const uint32_t e = (b >> 10) & 0x1fu;
    const uint32_t fr = b & 0x3ffu;
    if (e == 0u) {
        const float v = (float)fr * 5.9604644775390625e-08f;  // fr * 2^-24, exact
        return bits_f32(f32_bits(v) | sign);
    }
    if (e == 0x1fu) return bits_f32(sign | 0x7f800000u | (fr << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (fr << 13));
}

}  // namespace fhip

#endif  // FHIP_CODEC_H
