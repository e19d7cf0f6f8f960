/*
 * feather_oracle.c -- CPU restatement of Feather's Common-backend semantics for the quantized
 * linear hot path.  TEST INFRASTRUCTURE ONLY (parity checker; see feather_oracle.h).
 *
 * Parity pins (what checks each function; the tests live in tests/test_oracle_*.py):
 *   fp8/bf16 codecs      exhaustive 2^32 comparison with the reference's own header codec
 *                        (oracle/_ref, built from include/util/fp8.h, bf16.h) + the KATs of
 *                        test/fp8_test.cc:254-279
 *   cast                 test/fp8_test.cc:555-631 cases + codec pins
 *   fp8 matmul/gemm/fc   closed-form small cases (test/fp8_test.cc:768-822), fp64 brute force,
 *                        and the reference x86 FP8 linear (oracle/_ref) within 1 FP8 code
 *   int8 linear / conv   numpy int64 brute force for the accumulator, the reference's own
 *                        requantization (oracle/_ref: quant/quantization.h,
 *                        int8_kernel_utils.h) for the epilogue, and the cases of
 *                        test/common_int8_kernel_test.cc
 *   quantize/dequantize  reference QuantizeInt8Value (oracle/_ref) on every element +
 *                        test/quantization_math_test.cc, test/quantize_linear_op_test.cc cases
 *   bf16 argmax          reference x86 packed argmax (oracle/_ref) + the cases of
 *                        test/qwen_gemm_argmax_test.cc (NaN skip, first signed zero, ties)
 */
#include "feather_oracle.h"

#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------------------------
 * FP8 codec.  Restates include/util/fp8.h:66-211 (EncodeFinite/EncodeE4M3/EncodeE5M2,
 * DecodeE4M3/DecodeE5M2): OCP e4m3fn / e5m2, round-to-nearest-even, finite overflow
 * saturates to the largest finite code, e4m3: +-Inf -> 0x7e|s, NaN -> 0x7f|s;
 * e5m2: +-Inf -> 0x7c|s, NaN -> 0x7d|s.  Written here as integer arithmetic on the float's
 * bits: the value is an integer multiple of the FP8 quantum at its binade, rounded once.
 * ---------------------------------------------------------------------------------------- */
typedef struct {
    int mbits;          /* mantissa bits */
    int bias;           /* exponent bias */
    uint32_t max_bits;  /* float bits of the largest finite value */
    uint8_t max_code, inf_code, nan_code;
} fp8_format;

static const fp8_format kE4M3 = {3, 7, 0x43e00000u /* 448 */, 0x7e, 0x7e, 0x7f};
static const fp8_format kE5M2 = {2, 15, 0x47600000u /* 57344 */, 0x7b, 0x7c, 0x7d};

/* Round mant >> shift to nearest, ties to even (shift >= 1). */
static uint32_t rne_shift(uint32_t mant, int shift) {
    if (shift >= 32) return 0;            /* mant < 2^24 so the value is < 2^-8: rounds to 0 */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return q;
}

static uint8_t fp8_encode_fmt(const fp8_format* f, float value) {
    uint32_t u = f2u(value);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint8_t)(sign | (a == 0x7f800000u ? f->inf_code : f->nan_code));
    if (a > f->max_bits) return (uint8_t)(sign | f->max_code);
    int fexp = (int)(a >> 23);
    uint32_t mant = a & 0x7fffffu;
    int e;                                /* unbiased exponent of the float, value = mant * 2^(e-23) */
    if (fexp == 0) { e = -126; } else { e = fexp - 127; mant |= 0x800000u; }
    const int emin = 1 - f->bias;         /* exponent of the smallest normal FP8 */
    if (e < emin) {
        /* subnormal range: code = RNE(value / 2^(emin - mbits)), 2^mbits means min normal */
        int shift = 23 - f->mbits + (emin - e);
        return (uint8_t)(sign | rne_shift(mant, shift));
    }
    uint32_t q = rne_shift(mant, 23 - f->mbits);   /* in [2^mbits, 2^(mbits+1)] */
    if (q == (2u << f->mbits)) { q >>= 1; e++; }
    uint32_t code = ((uint32_t)(e + f->bias) << f->mbits) | (q & ((1u << f->mbits) - 1u));
    return (uint8_t)(sign | code);
}

uint8_t fo_fp8_encode(int dtype, float value) {
    return fp8_encode_fmt(dtype == FO_FP8E5M2 ? &kE5M2 : &kE4M3, value);
}

float fo_fp8_decode(int dtype, uint8_t code) {
    const int e5 = dtype == FO_FP8E5M2;
    const int mbits = e5 ? 2 : 3, bias = e5 ? 15 : 7;
    const int ef = (code & 0x7f) >> mbits, m = code & ((1 << mbits) - 1);
    const int neg = (code & 0x80) != 0;
    float v;
    if (e5 && ef == 31) v = m == 0 ? INFINITY : NAN;
    else if (!e5 && ef == 15 && m == 7) v = NAN;
    else if (ef == 0) v = ldexpf((float)m, 1 - bias - mbits);
    else v = ldexpf((float)((1 << mbits) | m), ef - bias - mbits);
    if (isnan(v)) return u2f(0x7fc00000u);   /* the reference returns a positive quiet NaN */
    return neg ? -v : v;
}

void fo_fp8_encode_array(int dtype, const float* in, uint8_t* out, int64_t count) {
    for (int64_t i = 0; i < count; ++i) out[i] = fo_fp8_encode(dtype, in[i]);
}

void fo_fp8_encode_bits_range(int dtype, uint32_t first_bits, int64_t count, uint8_t* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = fo_fp8_encode(dtype, u2f(first_bits + (uint32_t)i));
}

/* ------------------------------------------------------------------------------------------
 * BF16 / FP16 codecs.
 * ---------------------------------------------------------------------------------------- */
uint16_t fo_bf16_encode(float value) {               /* include/util/bf16.h:36-46 */
    uint32_t u = f2u(value);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float fo_bf16_decode(uint16_t bits) { return u2f((uint32_t)bits << 16); }   /* bf16.h:27-32 */

void fo_bf16_encode_array(const float* in, uint16_t* out, int64_t count) {
    #pragma omp parallel for schedule(static) if (count >= 65536)
    for (int64_t i = 0; i < count; ++i) out[i] = fo_bf16_encode(in[i]);
}

void fo_bf16_encode_bits_range(uint32_t first_bits, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = fo_bf16_encode(u2f(first_bits + (uint32_t)i));
}

void fo_fp16_encode_bits_range(int cast_rule, uint32_t first_bits, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; ++i) {
        float x = u2f(first_bits + (uint32_t)i);
        out[i] = cast_rule ? fo_fp16_encode_cast(x) : fo_fp16_encode(x);
    }
}

void fo_bf16_plain_encode_bits_range(uint32_t first_bits, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = fo_bf16_encode_plain(u2f(first_bits + (uint32_t)i));
}

uint16_t fo_bf16_encode_plain(float value) {         /* quantize_linear_utils.h:110-117 */
    uint32_t u = f2u(value);
    uint32_t low = u & 0xffffu, high = u >> 16;
    if (low > 0x8000u || (low == 0x8000u && (high & 1u))) high++;
    return (uint16_t)high;
}

uint16_t fo_fp16_encode(float value) {               /* quantize_linear_utils.h:70-101 */
    uint32_t u = f2u(value);
    uint32_t sign = (u >> 16) & 0x8000u, fexp = (u >> 23) & 0xffu, frac = u & 0x7fffffu;
    if (fexp == 0xffu) return (uint16_t)(sign | 0x7c00u | (frac ? 0x200u : 0u));
    int he = (int)fexp - 127 + 15;
    if (he >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)sign;
        return (uint16_t)(sign | rne_shift(frac | 0x800000u, 14 - he));
    }
    uint32_t r = rne_shift(frac | 0x800000u, 13);   /* 11-bit significand incl. hidden bit */
    if (r == 0x800u) return (uint16_t)(sign | ((uint32_t)(he + 1) << 10));
    return (uint16_t)(sign | ((uint32_t)he << 10) | (r & 0x3ffu));
}

/* Cast's FP16 encoder (include/util/fp16.h FloatToHalf, cast.cc:98): magnitude rounded half away
 * from zero at the FP16 quantum, |x| < 2^-24 -> signed zero, overflow -> Inf, NaN -> top 10 payload
 * bits with the lowest forced on.  Written as: the value is a multiple of the quantum q (2^-24 for
 * subnormal results, 2^(e-10) for normal ones); add q/2 to the magnitude's significand and truncate. */
uint16_t fo_fp16_encode_cast(float value) {
    uint32_t u = f2u(value);
    uint32_t sign = (u >> 16) & 0x8000u, fexp = (u >> 23) & 0xffu, frac = u & 0x7fffffu;
    int e = (int)fexp - 127;
    if (fexp == 0xffu) return (uint16_t)(sign | 0x7c00u | (frac ? ((frac >> 13) | 1u) : 0u));
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e < -24) return (uint16_t)sign;
    uint32_t sig = frac | 0x800000u;            /* 24-bit significand, value = sig * 2^(e-23) */
    int drop = e < -14 ? -e - 1 : 13;           /* significand bits below the quantum */
    uint32_t q = (sig + (1u << (drop - 1))) >> drop;   /* units of the quantum, half away */
    if (e < -14) return (uint16_t)(sign | q);   /* subnormal (q == 0x400 is the smallest normal) */
    /* normal: q in [0x400, 0x800]; 0x800 means the rounding carried into the next binade */
    uint32_t he = (uint32_t)(e + 15) + (q >> 11);
    if (he >= 0x1fu) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | (he << 10) | (q & 0x3ffu));
}

float fo_fp16_decode(uint16_t bits) {                /* quantize_linear_utils.h:50-68 */
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16, e = (bits >> 10) & 0x1fu, fr = bits & 0x3ffu;
    if (e == 0) {
        if (fr) { float v = ldexpf((float)fr, -24); return sign ? -v : v; }
        return u2f(sign);
    }
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (fr << 13));
    return u2f(sign | ((e + 112u) << 23) | (fr << 13));
}

/* ------------------------------------------------------------------------------------------
 * Cast (src/kernel/common/cast.cc:62-122): ReadFloat of the source, then the destination
 * encoder; FP8 destinations divide by the output scale, FP8 sources multiply by theirs
 * (kernel_io.h:58-78).
 * ---------------------------------------------------------------------------------------- */
static int valid_scale(float s) { return isfinite(s) && s > 0.0f; }

static float read_float(int dtype, const void* src, int64_t i) {
    switch (dtype) {
        case FO_FP32: return ((const float*)src)[i];
        case FO_BF16: return fo_bf16_decode(((const uint16_t*)src)[i]);
        case FO_FP16: return fo_fp16_decode(((const uint16_t*)src)[i]);
        default: return NAN;
    }
}

int fo_cast_to_fp8(int src_dtype, const void* src, int64_t count, int fp8_dtype, float out_scale, uint8_t* out) {
    if (!src || !out || count < 0 || !valid_scale(out_scale)) return -1;
    if (src_dtype != FO_FP32 && src_dtype != FO_BF16 && src_dtype != FO_FP16) return -1;
    for (int64_t i = 0; i < count; ++i) out[i] = fo_fp8_encode(fp8_dtype, read_float(src_dtype, src, i) / out_scale);
    return 0;
}

int fo_cast_from_fp8(int fp8_dtype, const uint8_t* src, float in_scale, int64_t count, int dst_dtype, void* out) {
    if (!src || !out || count < 0 || !valid_scale(in_scale)) return -1;
    for (int64_t i = 0; i < count; ++i) {
        float v = fo_fp8_decode(fp8_dtype, src[i]) * in_scale;
        switch (dst_dtype) {
            case FO_FP32: ((float*)out)[i] = v; break;
            case FO_BF16: ((uint16_t*)out)[i] = fo_bf16_encode(v); break;
            case FO_FP16: ((uint16_t*)out)[i] = fo_fp16_encode_cast(v); break;
            default: return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------
 * FP8 linear.  TensorIO<FP8>::Read = Dec(code) * scale (kernel_io.h:58-78), products summed
 * in fp32 in ascending K order (matmul.cc:115-122, gemm.cc:79-86, fc.cc:55-61).
 * ---------------------------------------------------------------------------------------- */
static void decode_scaled(int dtype, const uint8_t* codes, float scale, float* out, int64_t count) {
    float table[256];
    for (int c = 0; c < 256; ++c) table[c] = fo_fp8_decode(dtype, (uint8_t)c) * scale;
    for (int64_t i = 0; i < count; ++i) out[i] = table[codes[i]];
}

/* sums[i*n+j] = sum_t A[i,t]*B[t,j] with B[t,j] = b[j*k+t] (trans_b) or b[t*n+j]. */
static int fp8_sums(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb, int trans_b,
                    int64_t m, int64_t k, int64_t n, float* sums) {
    if (!a || !b || !sums || m <= 0 || k <= 0 || n <= 0 || !valid_scale(sa) || !valid_scale(sb)) return -1;
    float* av = (float*)malloc(sizeof(float) * (size_t)(m * k));
    float* bt = (float*)malloc(sizeof(float) * (size_t)(n * k));   /* [n][k] */
    if (!av || !bt) { free(av); free(bt); return -1; }
    decode_scaled(dtype, a, sa, av, m * k);
    {
        float* bv = (float*)malloc(sizeof(float) * (size_t)(n * k));
        if (!bv) { free(av); free(bt); return -1; }
        decode_scaled(dtype, b, sb, bv, n * k);
        for (int64_t j = 0; j < n; ++j)
            for (int64_t t = 0; t < k; ++t) bt[j * k + t] = trans_b ? bv[j * k + t] : bv[t * n + j];
        free(bv);
    }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
        const float* ar = av + i * k;
        for (int64_t j = 0; j < n; ++j) {
            const float* br = bt + j * k;
            float s = 0.0f;
            for (int64_t t = 0; t < k; ++t) s += ar[t] * br[t];
            sums[i * n + j] = s;
        }
    }
    free(av);
    free(bt);
    return 0;
}

int fo_fp8_gemm_f32(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb, int trans_b,
                    int64_t m, int64_t k, int64_t n, float* sums) {
    return fp8_sums(dtype, a, sa, b, sb, trans_b, m, k, n, sums);
}

static int fp8_linear_common(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb, int trans_b,
                             const uint8_t* bias, float s_bias, int bias_kind, int use_alpha, float alpha,
                             float beta, int64_t m, int64_t k, int64_t n, uint8_t* out, float s_out) {
    if (!out || !valid_scale(s_out) || (bias_kind != FO_BIAS_NONE && (!bias || !valid_scale(s_bias)))) return -1;
    float* sums = (float*)malloc(sizeof(float) * (size_t)(m * n));
    if (!sums) return -1;
    if (fp8_sums(dtype, a, sa, b, sb, trans_b, m, k, n, sums) != 0) { free(sums); return -1; }
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n; ++j) {
            float s = sums[i * n + j];
            if (use_alpha) s *= alpha;
            if (bias_kind != FO_BIAS_NONE) {
                const int64_t bi = bias_kind == FO_BIAS_VECTOR ? j : i * n + j;
                const float bv = fo_fp8_decode(dtype, bias[bi]) * s_bias;
                s += use_alpha ? beta * bv : bv;
            }
            out[i * n + j] = fo_fp8_encode(dtype, s / s_out);
        }
    }
    free(sums);
    return 0;
}

int fo_fp8_matmul(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb,
                  int64_t m, int64_t k, int64_t n, uint8_t* out, float s_out) {
    return fp8_linear_common(dtype, a, sa, b, sb, 0, NULL, 1.0f, FO_BIAS_NONE, 0, 1.0f, 1.0f, m, k, n, out, s_out);
}

int fo_fp8_gemm(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb, int trans_b,
                const uint8_t* bias, float s_bias, int bias_kind, float alpha, float beta,
                int64_t m, int64_t k, int64_t n, uint8_t* out, float s_out) {
    return fp8_linear_common(dtype, a, sa, b, sb, trans_b, bias, s_bias, bias_kind, 1, alpha, beta, m, k, n, out,
                             s_out);
}

int fo_fp8_fc(int dtype, const uint8_t* a, float sa, const uint8_t* w, float sw,
              const uint8_t* bias, float s_bias, int bias_kind,
              int64_t m, int64_t k, int64_t n, uint8_t* out, float s_out) {
    return fp8_linear_common(dtype, a, sa, w, sw, 0, bias, s_bias, bias_kind, 0, 1.0f, 1.0f, m, k, n, out, s_out);
}

/* ------------------------------------------------------------------------------------------
 * INT8 requantization (int8_kernel_utils.h:155-179, include/quant/quantization.h:94-99):
 * transformed = real / double(s_out) + zp, std::round (ties away from zero), clamp.
 * ---------------------------------------------------------------------------------------- */
/* std::max(-128.0, std::min(127.0, r)) with the std:: argument order, so NaN maps to 127 as in
 * include/quant/quantization.h:94-99. */
static int8_t clamp_i8(double r) {
    const double hi = (r < 127.0) ? r : 127.0;
    const double lo = (-128.0 < hi) ? hi : -128.0;
    return (int8_t)lo;
}

static int quantize_real(double real, float s_out, int32_t zp_out, int8_t* result) {
    if (!isfinite(real) || !valid_scale(s_out)) return -1;
    double t = real / (double)s_out + (double)zp_out;
    if (!isfinite(t)) return -1;
    *result = clamp_i8(round(t));
    return 0;
}

static int fits_i32(int64_t v) { return v >= INT32_MIN && v <= INT32_MAX; }

static int valid_qparams(const float* scales, int64_t n_scale, const int32_t* zps, int64_t n_zp) {
    if (!scales || n_scale <= 0) return 0;
    for (int64_t i = 0; i < n_scale; ++i) if (!valid_scale(scales[i])) return 0;
    if (zps) {
        if (n_zp != 1 && n_zp != n_scale) return 0;
        for (int64_t i = 0; i < n_zp; ++i) if (zps[i] < -128 || zps[i] > 127) return 0;
    }
    return 1;
}

int fo_i8_linear(int kind, const int8_t* a, float s_a, int32_t zp_a,
                 const int8_t* w, int trans_b, const float* w_scales, int64_t n_wscale,
                 const int32_t* w_zps, int64_t n_wzp,
                 const int32_t* bias, int bias_kind, float alpha, float beta,
                 int64_t m, int64_t k, int64_t n,
                 int8_t* out, float s_out, int32_t zp_out, int32_t* acc_out) {
    if (!a || !w || !out || m <= 0 || k <= 0 || n <= 0) return -1;
    if (!valid_scale(s_a) || zp_a < -128 || zp_a > 127 || !valid_scale(s_out) || zp_out < -128 || zp_out > 127)
        return -1;
    if (n_wscale != 1 && n_wscale != n) return -1;
    if (!valid_qparams(w_scales, n_wscale, w_zps, n_wzp)) return -1;
    if (kind != FO_I8_GEMM) trans_b = 0;
    if (kind == FO_I8_MATMUL) bias_kind = FO_BIAS_NONE;
    if (kind == FO_I8_GEMM && (!isfinite(alpha) || !isfinite(beta))) return -1;
    if (bias_kind != FO_BIAS_NONE && !bias) return -1;
    int status = 0;
    #pragma omp parallel for schedule(static) reduction(|:status)
    for (int64_t i = 0; i < m; ++i) {
        for (int64_t j = 0; j < n && !status; ++j) {
            const int32_t wzp = w_zps ? w_zps[n_wzp == 1 ? 0 : j] : 0;
            const float ws = w_scales[n_wscale == 1 ? 0 : j];
            int64_t dot = 0;
            for (int64_t t = 0; t < k; ++t) {
                const int32_t wv = trans_b ? w[j * k + t] : w[t * n + j];
                dot += (int64_t)((int32_t)a[i * k + t] - zp_a) * (int64_t)(wv - wzp);
                if (!fits_i32(dot)) { status = 1; break; }
            }
            if (status) break;
            if (acc_out) acc_out[i * n + j] = (int32_t)dot;
            const int32_t bv = bias_kind == FO_BIAS_NONE ? 0 : bias[bias_kind == FO_BIAS_VECTOR ? j : i * n + j];
            const double scale = (double)s_a * (double)ws;
            double real;
            if (kind == FO_I8_GEMM) {
                const double acc = (double)alpha * (double)dot + (double)beta * (double)bv;
                real = acc * scale;
            } else {
                int64_t acc = dot;
                if (kind == FO_I8_FC) {
                    acc += bv;
                    if (!fits_i32(acc)) { status = 1; break; }
                }
                real = (double)acc * scale;
            }
            if (quantize_real(real, s_out, zp_out, &out[i * n + j]) != 0) { status = 1; break; }
        }
    }
    return status ? -1 : 0;
}

/* ------------------------------------------------------------------------------------------
 * INT8 Conv2D (src/kernel/common/conv2d.cc:482-581): direct convolution, the accumulator
 * starts at the int32 bias, each partial sum must stay inside int32, requantized with
 * double(s_in) * s_w[oc].
 * ---------------------------------------------------------------------------------------- */
static int64_t img_off(int layout, int64_t b, int64_t c, int64_t y, int64_t x, int64_t C, int64_t H, int64_t W) {
    return layout == 0 ? ((b * C + c) * H + y) * W + x : ((b * H + y) * W + x) * C + c;
}

int fo_i8_conv2d(const int8_t* in, int64_t n, int64_t c, int64_t h, int64_t w, int layout,
                 float s_in, int32_t zp_in,
                 const int8_t* wt, int64_t oc, int64_t kh, int64_t kw,
                 const float* w_scales, int64_t n_wscale, const int32_t* w_zps, int64_t n_wzp,
                 const int32_t* bias,
                 int32_t stride_h, int32_t stride_w, int32_t pad_h, int32_t pad_w,
                 int32_t dil_h, int32_t dil_w, int32_t group,
                 int8_t* out, int64_t oh, int64_t ow, float s_out, int32_t zp_out) {
    if (!in || !wt || !out || stride_h <= 0 || stride_w <= 0 || dil_h <= 0 || dil_w <= 0 || group <= 0) return -1;
    if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || oc <= 0 || kh <= 0 || kw <= 0 || c % group || oc % group) return -1;
    const int64_t eh = (h + 2 * pad_h - dil_h * (kh - 1) - 1) / stride_h + 1;
    const int64_t ew = (w + 2 * pad_w - dil_w * (kw - 1) - 1) / stride_w + 1;
    if (eh <= 0 || ew <= 0 || eh != oh || ew != ow) return -1;
    if (!valid_scale(s_in) || zp_in < -128 || zp_in > 127 || !valid_scale(s_out) || zp_out < -128 || zp_out > 127)
        return -1;
    if ((n_wscale != 1 && n_wscale != oc) || !valid_qparams(w_scales, n_wscale, w_zps, n_wzp)) return -1;
    const int64_t icg = c / group, ocg = oc / group;
    int status = 0;
    #pragma omp parallel for collapse(2) schedule(static) reduction(|:status)
    for (int64_t b = 0; b < n; ++b) {
        for (int64_t o = 0; o < oc; ++o) {
            const int64_t g = o / ocg;
            const int32_t wzp = w_zps ? w_zps[n_wzp == 1 ? 0 : o] : 0;
            const double scale = (double)s_in * (double)w_scales[n_wscale == 1 ? 0 : o];
            for (int64_t y = 0; y < oh && !status; ++y) {
                for (int64_t x = 0; x < ow && !status; ++x) {
                    int64_t acc = bias ? bias[o] : 0;
                    for (int64_t ci = 0; ci < icg && !status; ++ci) {
                        const int64_t gc = g * icg + ci;
                        for (int64_t ky = 0; ky < kh && !status; ++ky) {
                            const int64_t iy = y * stride_h + ky * dil_h - pad_h;
                            if (iy < 0 || iy >= h) continue;
                            for (int64_t kx = 0; kx < kw; ++kx) {
                                const int64_t ix = x * stride_w + kx * dil_w - pad_w;
                                if (ix < 0 || ix >= w) continue;
                                const int32_t iv = in[img_off(layout, b, gc, iy, ix, c, h, w)];
                                const int32_t wv = wt[((o * icg + ci) * kh + ky) * kw + kx];
                                acc += (int64_t)(iv - zp_in) * (int64_t)(wv - wzp);
                                if (!fits_i32(acc)) { status = 1; break; }
                            }
                        }
                    }
                    if (status) break;
                    if (quantize_real((double)acc * scale, s_out, zp_out,
                                      &out[img_off(layout, b, o, y, x, oc, oh, ow)]) != 0)
                        status = 1;
                }
            }
        }
    }
    (void)ocg;
    return status ? -1 : 0;
}

/* ------------------------------------------------------------------------------------------
 * QuantizeLinear / DequantizeLinear (quantize_linear_utils.h:187-341,
 * include/quant/quantization.h:46-125).
 * ---------------------------------------------------------------------------------------- */
static int channel_geometry(const int64_t* dims, int rank, int64_t n_scale, int64_t axis, int64_t* count,
                            int64_t* stride, int64_t* channels) {
    int64_t total = 1;
    for (int r = 0; r < rank; ++r) { if (dims[r] <= 0) return -1; total *= dims[r]; }
    if (rank <= 0 || total <= 0) return -1;
    *count = total;
    *stride = 1;
    *channels = 1;
    if (n_scale == 1) return 0;
    if (axis < 0) axis += rank;
    if (axis < 0 || axis >= rank || dims[axis] != n_scale) return -1;
    for (int r = (int)axis + 1; r < rank; ++r) *stride *= dims[r];
    *channels = dims[axis];
    return 0;
}

int fo_quantize_linear(int src_dtype, const void* src, const int64_t* dims, int rank,
                       const float* scales, int64_t n_scale, const int32_t* zps, int64_t n_zp,
                       int64_t axis, int8_t* out) {
    int64_t count, stride, channels;
    if (!src || !out || !zps || n_zp <= 0) return -1;
    if (src_dtype != FO_FP32 && src_dtype != FO_FP16 && src_dtype != FO_BF16) return -1;
    if (!valid_qparams(scales, n_scale, zps, n_zp)) return -1;
    if (channel_geometry(dims, rank, n_scale, axis, &count, &stride, &channels) != 0) return -1;
    #pragma omp parallel for schedule(static) if (count >= 4096)
    for (int64_t i = 0; i < count; ++i) {
        const int64_t p = n_scale == 1 ? 0 : (i / stride) % channels;
        const float x = read_float(src_dtype, src, i);
        const double t = (double)x / (double)scales[p] + (double)zps[n_zp == 1 ? 0 : p];
        out[i] = clamp_i8(round(t));
    }
    return 0;
}

int fo_dequantize_linear(const int8_t* src, const int64_t* dims, int rank,
                         const float* scales, int64_t n_scale, const int32_t* zps, int64_t n_zp,
                         int64_t axis, int dst_dtype, void* out) {
    int64_t count, stride, channels;
    if (!src || !out || !zps || n_zp <= 0) return -1;
    if (dst_dtype != FO_FP32 && dst_dtype != FO_FP16 && dst_dtype != FO_BF16) return -1;
    if (!valid_qparams(scales, n_scale, zps, n_zp)) return -1;
    if (channel_geometry(dims, rank, n_scale, axis, &count, &stride, &channels) != 0) return -1;
    for (int64_t i = 0; i < count; ++i) {
        const int64_t p = n_scale == 1 ? 0 : (i / stride) % channels;
        const float v = (float)((int32_t)src[i] - zps[n_zp == 1 ? 0 : p]) * scales[p];
        if (dst_dtype == FO_FP32) ((float*)out)[i] = v;
        else if (dst_dtype == FO_FP16) ((uint16_t*)out)[i] = fo_fp16_encode(v);
        else ((uint16_t*)out)[i] = fo_bf16_encode_plain(v);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------
 * Greedy LM-head selection (src/kernel/common/qwen_gemm_argmax.cc:28-49): fp32 dot in K
 * order, round to BF16 (RNE, NaN quieted), skip NaN, first strict maximum (so +0/-0 and
 * equal values keep the lowest index), 0 when every value is NaN.
 * ---------------------------------------------------------------------------------------- */
static int bf16_is_nan(uint16_t b) { return (b & 0x7f80u) == 0x7f80u && (b & 0x7fu) != 0; }

int64_t fo_bf16_gemm_argmax(const uint16_t* a, const uint16_t* b, int64_t k, int64_t v, float* logits) {
    float* av = (float*)malloc(sizeof(float) * (size_t)k);
    float* sums = (float*)malloc(sizeof(float) * (size_t)v);
    if (!av || !sums) { free(av); free(sums); return -1; }
    for (int64_t t = 0; t < k; ++t) av[t] = fo_bf16_decode(a[t]);
    #pragma omp parallel for schedule(static)
    for (int64_t col = 0; col < v; ++col) {
        const uint16_t* row = b + col * k;
        float s = 0.0f;
        for (int64_t t = 0; t < k; ++t) s += av[t] * fo_bf16_decode(row[t]);
        sums[col] = s;
    }
    int64_t best = -1;
    float best_value = 0.0f;
    for (int64_t col = 0; col < v; ++col) {
        if (logits) logits[col] = sums[col];
        const uint16_t r = fo_bf16_encode(sums[col]);
        if (bf16_is_nan(r)) continue;
        const float value = fo_bf16_decode(r);
        if (best < 0 || value > best_value) { best = col; best_value = value; }
    }
    free(av);
    free(sums);
    return best < 0 ? 0 : best;
}

int64_t fo_fp8_gemm_argmax(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb,
                           int64_t k, int64_t v, float s_out) {
    if (!valid_scale(s_out)) return -1;
    float* sums = (float*)malloc(sizeof(float) * (size_t)v);
    if (!sums) return -1;
    if (fp8_sums(dtype, a, sa, b, sb, 1, 1, k, v, sums) != 0) { free(sums); return -1; }
    int64_t best = -1;
    float best_value = 0.0f;
    for (int64_t col = 0; col < v; ++col) {
        const uint8_t code = fo_fp8_encode(dtype, sums[col] / s_out);           /* Gemm output */
        const uint16_t r = fo_bf16_encode(fo_fp8_decode(dtype, code) * s_out);  /* Cast fp8 -> bf16 */
        if (bf16_is_nan(r)) continue;
        const float value = fo_bf16_decode(r);
        if (best < 0 || value > best_value) { best = col; best_value = value; }
    }
    free(sums);
    return best < 0 ? 0 : best;
}

int fo_set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
    return omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}
