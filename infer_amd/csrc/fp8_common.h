// fp8_common.h -- pieces shared by the FP8 GEMV and GEMM kernels: operand decode, streaming loads
// and the output epilogue (the reference's alpha/beta/bias/out_scale rule and the FP8 output code).
#ifndef FHIP_FP8_COMMON_H
#define FHIP_FP8_COMMON_H

#include "fhip_internal.h"
#include "codec.h"

namespace fhip {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (non-temporal: the weight is read once per call).
__device__ __forceinline__ uint4 load_stream16(const uint8_t* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Decodes four FP8 codes packed little-endian in `w` with the hardware OCP converters.
template <bool E5>
__device__ __forceinline__ void decode4(uint32_t w, float* out) {
    v2f lo, hi;
    if constexpr (E5) {
        lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, false);
        hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, true);
    } else {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
        hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    }
    out[0] = lo.x;
    out[1] = lo.y;
    out[2] = hi.x;
    out[3] = hi.y;
}

struct Fp8Epilogue {
    float ab_scale;      // a_scale * w_scale
    float alpha, beta;
    const uint8_t* bias;
    float bias_scale;
    int bias_kind;
    float out_scale;
    float out_inv;       // 1/out_scale when out_scale is a power of two, else 0 (divide)
    int out_dtype;       // FP8 (code), BF16 or FP32 (decoded through the FP8 code)
    void* out;
    int64_t n;           // row stride of out
    bool e5;

    // Output element bits (FP8 code, BF16 bits or FP32 bits) for accumulator `acc` at (row, col).
    __device__ __forceinline__ uint32_t value(float acc, int64_t row, int64_t col) const {
        float y = acc * ab_scale;
        y *= alpha;
        if (bias_kind != FHIP_BIAS_NONE) {
            const uint8_t bc = bias[bias_kind == FHIP_BIAS_VECTOR ? col : row * n + col];
            y += beta * (fhip::fp8_decode(bc, e5) * bias_scale);
        }
        const uint8_t code = fhip::fp8_encode(out_inv != 0.0f ? y * out_inv : y / out_scale, e5);
        if (out_dtype == FHIP_BF16) return fhip::bf16_encode(fhip::fp8_decode(code, e5) * out_scale);
        if (out_dtype == FHIP_FP32) return fhip::f32_bits(fhip::fp8_decode(code, e5) * out_scale);
        return code;
    }

    __device__ __forceinline__ void store(float acc, int64_t row, int64_t col) const {
        float y = acc * ab_scale;
        if (bias_kind != FHIP_BIAS_NONE) {
            y *= alpha;
            const uint8_t bc = bias[bias_kind == FHIP_BIAS_VECTOR ? col : row * n + col];
            y += beta * (fhip::fp8_decode(bc, e5) * bias_scale);
        } else {
            y *= alpha;
        }
        const uint8_t code = fhip::fp8_encode(out_inv != 0.0f ? y * out_inv : y / out_scale, e5);
        const int64_t idx = row * n + col;
        if (out_dtype == FHIP_BF16) {
            static_cast<uint16_t*>(out)[idx] = fhip::bf16_encode(fhip::fp8_decode(code, e5) * out_scale);
        } else if (out_dtype == FHIP_FP32) {
            static_cast<float*>(out)[idx] = fhip::fp8_decode(code, e5) * out_scale;
        } else {
            static_cast<uint8_t*>(out)[idx] = code;
        }
    }
};

// Reference code for a value the hardware converter cannot encode the reference's way: beyond the
// largest finite code the reference saturates finite overflow to max finite, and maps Inf to 0x7e
// (e4m3) / 0x7c (e5m2) and NaN to 0x7f / 0x7d, each with the value's sign (include/util/fp8.h:66-211).
// In-range values keep the hardware's round-to-nearest-even code.
template <bool E5>
__device__ __forceinline__ uint32_t fixup_code(float q, uint32_t hw_code) {
    const uint32_t bits = __float_as_uint(q);
    const uint32_t mag = bits & 0x7fffffffu;
    const uint32_t sign = (bits >> 24) & 0x80u;
    const uint32_t special = mag > 0x7f800000u ? (E5 ? 0x7du : 0x7fu)
                                                : (mag == 0x7f800000u ? (E5 ? 0x7cu : 0x7eu) : (E5 ? 0x7bu : 0x7eu));
    return mag <= (E5 ? 0x47600000u : 0x43e00000u) ? hw_code : (sign | special);
}

template <bool E5>
__device__ __forceinline__ float decode_code(uint32_t code) {
    const v2f d = E5 ? __builtin_amdgcn_cvt_pk_f32_bf8((int)code, false) : __builtin_amdgcn_cvt_pk_f32_fp8((int)code, false);
    return (d.x != d.x) ? __uint_as_float(0x7fc00000u) : d.x;  // the reference decodes NaN codes to +qNaN
}

// Four values -> four FP8 codes packed little-endian.  encode4_hw: the hardware converter's codes, which
// are the reference's for finite in-range values, and whether all four are such values (NaN fails every
// comparison).  encode4: the reference's codes, with saturated / special codes patched in.
template <bool E5>
__device__ __forceinline__ uint32_t encode4_hw(const float (&q)[4], bool& in_range) {
    int pk = E5 ? __builtin_amdgcn_cvt_pk_bf8_f32(q[0], q[1], 0, false) : __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    pk = E5 ? __builtin_amdgcn_cvt_pk_bf8_f32(q[2], q[3], pk, true) : __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], pk, true);
    const float maxf = E5 ? 57344.0f : 448.0f;
    in_range = __builtin_fabsf(q[0]) <= maxf && __builtin_fabsf(q[1]) <= maxf && __builtin_fabsf(q[2]) <= maxf &&
               __builtin_fabsf(q[3]) <= maxf;
    return (uint32_t)pk;
}

template <bool E5>
__device__ __forceinline__ uint32_t encode4(const float (&q)[4]) {
    bool in_range;
    const uint32_t pk = encode4_hw<E5>(q, in_range);
    uint32_t packed = pk;
    if (__builtin_expect(!in_range, 0)) {
        packed = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) packed |= fixup_code<E5>(q[t], (pk >> (8 * t)) & 0xffu) << (8 * t);
    }
    return packed;
}

// Hardware FP8 codes of four values, and a running flag whose bit 7 of some byte ends up set when a code
// is a special one: e4m3 0x7f (NaN, which the non-saturating converter also gives for |x| >= 464 and
// Inf) or e5m2 exponent 11111 (Inf for |x| >= 61440, NaN).  Values the reference saturates but that
// round below those thresholds (448 < |x| < 464, 57344 < |x| < 61440) already get the max-finite code.
// Masked bytes are at most 0x7f / 0x7c, so adding 1 / 4 carries into bit 7 only from an all-ones field.
template <bool E5>
__device__ __forceinline__ uint32_t encode4_flag(const float (&q)[4], uint32_t& flag) {
    int pk = E5 ? __builtin_amdgcn_cvt_pk_bf8_f32(q[0], q[1], 0, false) : __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    pk = E5 ? __builtin_amdgcn_cvt_pk_bf8_f32(q[2], q[3], pk, true) : __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], pk, true);
    constexpr uint32_t kMask = E5 ? 0x7c7c7c7cu : 0x7f7f7f7fu, kOne = E5 ? 0x04040404u : 0x01010101u;
    flag |= ((uint32_t)pk & kMask) + kOne;
    return (uint32_t)pk;
}

template <bool E5>
__device__ __forceinline__ uint32_t encode1(float q) {
    const int pk = E5 ? __builtin_amdgcn_cvt_pk_bf8_f32(q, 0.0f, 0, false) : __builtin_amdgcn_cvt_pk_fp8_f32(q, 0.0f, 0, false);
    return fixup_code<E5>(q, (uint32_t)pk & 0xffu);
}

constexpr int kGemvThreads = 256;
constexpr int kGemvMaxLds = 64 * 1024;
#ifndef FHIP_GEMV_R1
#define FHIP_GEMV_R1 2
#endif


// 1/s when s is a power of two (x * (1/s) then equals x / s exactly), else 0.
float pow2_inverse(float s);

// a: FP8 codes [m][k64], k64 % 64 == 0, 16-byte aligned rows; k64 <= the weight's padded K.
int launch_fp8_gemm(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w,
                    const Fp8Epilogue& ep);
// The same per (FP8 format, output bytes): one translation unit each (fp8_gemm_e{4,5}_{fp8,bf16,fp32}.hip).
#define FHIP_GEMM_DECL(NAME) \
    int NAME(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w, const Fp8Epilogue& ep);
FHIP_GEMM_DECL(launch_fp8_gemm_e4_o1)
FHIP_GEMM_DECL(launch_fp8_gemm_e4_o2)
FHIP_GEMM_DECL(launch_fp8_gemm_e4_o4)
FHIP_GEMM_DECL(launch_fp8_gemm_e5_o1)
FHIP_GEMM_DECL(launch_fp8_gemm_e5_o2)
FHIP_GEMM_DECL(launch_fp8_gemm_e5_o4)
#undef FHIP_GEMM_DECL

}  // namespace fhip

#endif  // FHIP_FP8_COMMON_H
