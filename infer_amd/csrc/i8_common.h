// i8_common.h -- INT8 requantization and the INT8 linear epilogue, shared by the INT8 kernels (int8.hip)
// and the INT8 mode of the MFMA tile GEMM (fp8_gemm_impl.h).
//
// Requantization is the reference's, in fp64 with no contraction (each function body turns contraction
// off, so including this header changes nothing else in a translation unit):
// src/kernel/common/int8_kernel_utils.h:155-179, include/quant/quantization.h:94-99.
#ifndef FHIP_I8_COMMON_H
#define FHIP_I8_COMMON_H
#include "fhip_internal.h"
#include "codec.h"

#include <cmath>

namespace fhip {

__device__ __forceinline__ int8_t clamp_round_i8(double t) {
#pragma clang fp contract(off)
    const double r = round(t);
    const double hi = (r < 127.0) ? r : 127.0;      // std::min(127.0, r): NaN -> 127
    const double lo = (-128.0 < hi) ? hi : -128.0;  // std::max(-128.0, hi)
    return (int8_t)lo;
}

// clamp_round_i8(real / s_out + zp_out), the reference's requantization (int8_kernel_utils.h:155-179),
// without a double division on the common path.  t = real * (1 / s_out) + zp_out differs from the divided
// form by at most ~2^-51 * (|t| + |zp_out|) (the reciprocal and the product are each correctly rounded);
// round() changes value only at the x.5 points, so wherever t is farther than that from one both forms
// round to the same integer.  Only near an x.5 point (or for non-finite t) is the division done.
__device__ __forceinline__ int8_t requant_i8_fast(double real, double recip_out, double zp_out, bool& near_tie) {
#pragma clang fp contract(off)
    const double t = real * recip_out + zp_out;
    const double half_gap = fabs((t - floor(t)) - 0.5);
    near_tie = !(half_gap > 0x1p-40 * (fabs(t) + 256.0));
    return clamp_round_i8(t);
}
__device__ __forceinline__ int8_t requant_i8(double real, double s_out, double recip_out, double zp_out) {
#pragma clang fp contract(off)
    bool near_tie;
    const int8_t q = requant_i8_fast(real, recip_out, zp_out, near_tie);
    if (near_tie) return clamp_round_i8(real / s_out + zp_out);
    return q;
}

// Requantization of an exact integer sum v (|v| < 2^24) with a per-column factor K = s_a * s_w / s_out held as
// an unevaluated float pair kh + kl (K to ~2^-48): the code is clamp(round_half_away(v * K) + zp).  p = v * kh
// and its exact rounding error e (one fma) give v * K = p + c, c = e + v * kl, to ~2^-45 |p|.  With h =
// floor(p) + 0.5 (exact), p - h lies in [-0.5, 0.5) and is exact wherever |p - h| <= 0.25 (Sterbenz: p and h
// within a factor of two, or h = +-0.5 and p within 0.25 of it); elsewhere its rounding cannot change its
// sign.  (p - floor(p) itself is not exact for p in (-1, 0): p + 1 needs more bits than p.)  So d = (p - h) + c
// has the sign of v * K - h wherever |d| exceeds 2^-36 (|p| + 1), and then the code is floor(p) + (d > 0) + zp,
// the reference's value (adding the integer zp moves no x.5 point, and the reference's fp64 evaluation is
// within ~2^-50 of the exact value).
// Otherwise (an x.5 point or closer than that, or |v| >= 2^24) `unsafe` is set and the caller decides with
// the reference's arithmetic.  Magnitudes |p| >= 2^23 only ever clamp.
__device__ __forceinline__ int8_t requant_i8_split(int32_t v, float kh, float kl, int32_t zp, bool& unsafe) {
#pragma clang fp contract(off)
    const float vf = (float)v;
    const float p = vf * kh;
    const float e = __builtin_fmaf(vf, kh, -p);
    const float c = e + vf * kl;
    const float fl = floorf(p);
    const float d = (p - (fl + 0.5f)) + c;
    unsafe = !(fabsf(d) > 0x1p-36f * (fabsf(p) + 1.0f)) || (uint32_t)(v + (1 << 24)) >= (2u << 24);
    const float r = fl + (d > 0.0f ? 1.0f : 0.0f) + (float)zp;
    const float hi = r < 127.0f ? r : 127.0f;
    const float lo = hi > -128.0f ? hi : -128.0f;
    return (int8_t)(int)lo;
}

// Cheaper screen for the same requantization, for loops that can afford a per-value second step: with
// t = fl32(fl32(v) * kh) + (zp + 0.5) rounded once more, |t - (v*K + zp + 0.5)| <= 3.0000001 * 2^-24 |v*K| +
// 2^-24 |t| < 2^-12 whenever |v*K| <= 1024 (fl32(v) may itself be rounded: |v| < 2^31).  So floor(t) is the
// reference's code wherever t - floor(t) is at least 2^-11 from 0 and from 1; otherwise `unsafe` is set and the
// caller decides with requant_i8_split (and the fp64 form).  Where |v*K| > 1024 the value lies beyond +-895
// and both clamp to the same code.  About 2^-10 of uniformly spread values are flagged.
__device__ __forceinline__ int8_t requant_i8_screen(int32_t v, float kh, float zp_half, bool& unsafe) {
#pragma clang fp contract(off)
    const float t = (float)v * kh + zp_half;
    const float fl = floorf(t);
    unsafe = fabsf((t - fl) - 0.5f) > 0.5f - 0x1p-11f;
    const float hi = fl < 127.0f ? fl : 127.0f;
    const float lo = hi > -128.0f ? hi : -128.0f;
    return (int8_t)(int)lo;
}

struct I8Epilogue {
    int kind;
    const float* w_scales;   // [n] (per-tensor weights: all equal)
    const int32_t* wsum;     // [n]
    const int32_t* bias;
    int bias_kind;
    int32_t zp_a;
    float s_a;
    double alpha, beta;
    double inv_out_den;      // double(s_out), used as a divisor
    double zp_out;
    double recip_out;        // 1 / double(s_out), for requant_i8
    int8_t* out;
    int64_t ldo;
    // Fused DequantizeLinear (per tensor): out_dtype FP32/FP16/BF16 writes float((q - dq_zp) * dq_scale) with
    // DequantizeLinear's own encoders into out_any instead of the INT8 code q into out.
    int out_dtype = FHIP_INT8;
    float dq_scale = 1.0f;
    int32_t dq_zp = 0;
    void* out_any = nullptr;
    // Integer path (requant_i8_split): the sums' requantized value is (dot + bias) * K with K per column,
    // i.e. MatMul, FC, or Gemm with alpha = beta = 1, and dot + bias provably inside int32 (host-set).
    bool int_path = false;

    // K = s_a * s_w / s_out of a column as the float pair kh + kl (fp64 product, as the reference's scale).
    __device__ __forceinline__ void split_scale(float w_scale, float& kh, float& kl) const {
#pragma clang fp contract(off)
        const double kd = (double)s_a * (double)w_scale * recip_out;
        kh = (float)kd;
        kl = (float)(kd - (double)kh);
    }

    // Per-output-channel parameters, loadable ahead of the main loop.
    struct Col {
        int32_t wsum;
        int32_t bias;  // vector bias (0 without one; a matrix bias is read per element)
        float w_scale;
    };
    __device__ __forceinline__ Col col_params(int64_t col) const {
        return Col{wsum[col], bias_kind == FHIP_BIAS_VECTOR ? bias[col] : 0, w_scales[col]};
    }

    __device__ __forceinline__ void store(int32_t raw, int64_t row, int64_t col) const {
        store(raw, row, col, col_params(col));
    }

    // The real value of the integer sum `raw` at (row, col) before requantization.
    __device__ __forceinline__ double real(int32_t raw, int64_t row, int64_t col, const Col& c) const {
#pragma clang fp contract(off)
        const int32_t dot = raw - zp_a * c.wsum;
        const int32_t b = bias_kind == FHIP_BIAS_MATRIX ? bias[row * ldo + col] : c.bias;
        const double scale = (double)s_a * (double)c.w_scale;
        if (kind == FHIP_I8_GEMM) {
            const double acc = alpha * (double)dot + beta * (double)b;
            return acc * scale;
        }
        return (double)(dot + b) * scale;  // MatMul has no bias (b = 0)
    }

    // The requantized INT8 code of the integer sum `raw` at (row, col).
    __device__ __forceinline__ int8_t code(int32_t raw, int64_t row, int64_t col, const Col& c) const {
        return requant_i8(real(raw, row, col, c), inv_out_den, recip_out, zp_out);
    }

    // DequantizeLinear of a code (fused output dtypes), quantize_linear_utils.h:291-341.
    __device__ __forceinline__ float dequant(int8_t q) const {
#pragma clang fp contract(off)
        return (float)((int32_t)q - dq_zp) * dq_scale;
    }

    __device__ __forceinline__ void store(int32_t raw, int64_t row, int64_t col, const Col& c) const {
        const int8_t q = code(raw, row, col, c);
        const int64_t idx = row * ldo + col;
        if (out_dtype == FHIP_INT8) {
            out[idx] = q;
        } else {
            const float v = dequant(q);
            if (out_dtype == FHIP_FP32) static_cast<float*>(out_any)[idx] = v;
            else if (out_dtype == FHIP_FP16) static_cast<uint16_t*>(out_any)[idx] = fhip::fp16_encode(v);
            else static_cast<uint16_t*>(out_any)[idx] = fhip::bf16_encode_plain(v);
        }
    }
};

// The INT8 mode of the MFMA tile GEMM (i8_gemm_tile.hip) for large M: a [m][k] int8, 16-byte aligned,
// k % 64 == 0, m * k < 2^31; the output row stride ep.ldo equals the weight's n; ep.out_dtype INT8, FP16,
// BF16 or FP32.
int launch_i8_gemm_tile(fhip_context ctx, const int8_t* a, int64_t m, const fhip_weight_s* w, const I8Epilogue& ep);

}  // namespace fhip

#endif  // FHIP_I8_COMMON_H
