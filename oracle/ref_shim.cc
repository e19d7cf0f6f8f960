// ref_shim.cc -- a C-ABI over Feather's own CPU code for the quantized linear hot path.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile (target `ref`) together with the
// reference's x86 sources straight from the Feather source tree, into oracle/_ref/libfeather_ref.so.
// It is used (a) to pin oracle/feather_oracle.c against the reference's own code and (b) as the
// CPU baseline timed by bench.py ("kind": "reference").  Nothing in the shipped library uses it.
//
// Reference code called through this shim:
//   include/util/fp8.h:66-211            FloatToFp8E4M3/E5M2, Fp8E4M3/E5M2ToFloat
//   include/util/bf16.h:27-46            FloatToBFloat16
//   include/util/fp16.h                  FloatToHalf (the Cast operator's FP16 encoder)
//   src/kernel/common/quantize_linear_utils.h:70-101   EncodeFloat16 (DequantizeLinear's FP16 encoder)
//   include/quant/quantization.h:94-99   QuantizeInt8Value
//   src/kernel/common/int8_kernel_utils.h:155-179   QuantizeReal / QuantizeAccumulator
//   src/kernel/x86/linear_fp8.{h,cc}     ComputeLinearRowMajorX86Fp8{,PackedRhs,TransposedRhs,
//                                        PackedTransposedRhs}, ComputeLinearRowMajorX86Fp8TransposedRhsArgmax
//   src/kernel/x86/linear.{h,cc}         PackedBf16TransposedRhs,
//                                        ComputeLinearRowMajorX86Bf16PackedTransposedRhsArgmax
#include <cstdint>
#include <cstring>
#include <new>

#include "util/fp8.h"
#include "util/bf16.h"
#include "util/fp16.h"
#include "quant/quantization.h"
#include "src/kernel/common/int8_kernel_utils.h"
#include "src/kernel/common/quantize_linear_utils.h"
#include "src/kernel/x86/linear_fp8.h"
#include "src/kernel/x86/linear.h"

#if defined(FEATHER_WITH_OPENMP)
#include <omp.h>
#endif

using feather::DataType;
namespace x86 = feather::kernel::x86;

namespace {
DataType Fp8Type(int dtype) { return dtype == 13 ? DataType::FP8E5M2 : DataType::FP8E4M3; }
x86::LinearBiasType BiasType(int kind) {
    return kind == 1 ? x86::LinearBiasType::kVector : (kind == 2 ? x86::LinearBiasType::kMatrix : x86::LinearBiasType::kNone);
}
float FromBits(uint32_t bits) {
    float value;
    std::memcpy(&value, &bits, sizeof(value));
    return value;
}

struct PackedFp8 {
    int dtype;
    bool transposed;
    const uint8_t* rhs;
    int64_t k, n;
    x86::PackedFp8Rhs rhs_kn;
    x86::PackedFp8TransposedRhs rhs_nk;
    x86::Fp8LinearWorkspace workspace;
};

struct PackedBf16 {
    const uint16_t* rhs;
    int64_t k, n;
    x86::PackedBf16TransposedRhs packed;
    x86::Bf16LinearWorkspace workspace;
};
}  // namespace

extern "C" {

int ref_max_threads() {
#if defined(FEATHER_WITH_OPENMP)
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void ref_fp8_encode_bits_range(int dtype, uint32_t first_bits, int64_t count, uint8_t* out) {
    const bool e5 = dtype == 13;
    for (int64_t i = 0; i < count; ++i) {
        const float value = FromBits(first_bits + static_cast<uint32_t>(i));
        out[i] = e5 ? feather::FloatToFp8E5M2(value) : feather::FloatToFp8E4M3(value);
    }
}

float ref_fp8_decode(int dtype, uint8_t code) {
    return dtype == 13 ? feather::Fp8E5M2ToFloat(code) : feather::Fp8E4M3ToFloat(code);
}

void ref_bf16_encode_bits_range(uint32_t first_bits, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = feather::FloatToBFloat16(FromBits(first_bits + static_cast<uint32_t>(i)));
}

// cast_rule 1: FloatToHalf (Cast); 0: EncodeFloat16 (DequantizeLinear)
void ref_fp16_encode_bits_range(int cast_rule, uint32_t first_bits, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; ++i) {
        const float x = FromBits(first_bits + static_cast<uint32_t>(i));
        out[i] = cast_rule ? feather::FloatToHalf(x) : feather::kernel::quantize_linear_detail::EncodeFloat16(x);
    }
}

// EncodeBFloat16 (DequantizeLinear's BF16 encoder: RNE, NaN not quieted)
void ref_bf16_plain_encode_bits_range(uint32_t first_bits, int64_t count, uint16_t* out) {
    for (int64_t i = 0; i < count; ++i)
        out[i] = feather::kernel::quantize_linear_detail::EncodeBFloat16(FromBits(first_bits + static_cast<uint32_t>(i)));
}

// FP16 decoders: decode_rule 1 = HalfToFloat (Cast, kernel_io), 0 = DecodeFloat16 (QuantizeLinear input)
float ref_fp16_decode(int decode_rule, uint16_t bits) {
    return decode_rule ? feather::HalfToFloat(bits) : feather::kernel::quantize_linear_detail::DecodeFloat16(bits);
}

void ref_quantize_int8_values(const float* in, int64_t count, float scale, int32_t zero_point, int8_t* out) {
    for (int64_t i = 0; i < count; ++i) out[i] = feather::QuantizeInt8Value(in[i], scale, zero_point);
}

// Requantizes int32 accumulators the way the Common INT8 kernels do:
// QuantizeAccumulator(acc, double(s_in) * s_w[c], {s_out, zp_out}).  Returns -1 on the
// reference's failure path (non-finite values).
int ref_requantize(const int32_t* acc, int64_t rows, int64_t channels, float s_in, const float* w_scales,
                   int64_t n_wscale, float s_out, int32_t zp_out, int8_t* out) {
    feather::kernel::int8_detail::QuantizationView output;
    output.scale = s_out;
    output.zero_point = zp_out;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t c = 0; c < channels; ++c) {
            const double scale = static_cast<double>(s_in) * w_scales[n_wscale == 1 ? 0 : c];
            if (!feather::kernel::int8_detail::QuantizeAccumulator(acc[r * channels + c], scale, output,
                                                                   &out[r * channels + c])) {
                return -1;
            }
        }
    }
    return 0;
}

// Direct x86 FP8 linear: rhs [K,N] (trans_b = 0) or [N,K] (trans_b = 1).
int ref_fp8_linear(int dtype, const uint8_t* lhs, float lhs_scale, const uint8_t* rhs, float rhs_scale, int trans_b,
                   const uint8_t* bias, float bias_scale, int bias_kind, float alpha, float beta, int64_t m,
                   int64_t k, int64_t n, uint8_t* out, float out_scale) {
    if (trans_b) {
        return x86::ComputeLinearRowMajorX86Fp8TransposedRhs(Fp8Type(dtype), lhs, lhs_scale, rhs, rhs_scale, bias,
                                                             bias_scale, alpha, beta, m, k, n, BiasType(bias_kind),
                                                             out, out_scale);
    }
    return x86::ComputeLinearRowMajorX86Fp8(Fp8Type(dtype), lhs, lhs_scale, rhs, rhs_scale, bias, bias_scale, m, k,
                                            n, BiasType(bias_kind), out, out_scale, alpha, beta);
}

// Prepared (packed, immutable-weight) x86 FP8 linear, as MatMul/Gemm<X86,FP8>::Prepare does.
void* ref_fp8_packed_create(int dtype, const uint8_t* rhs, int trans_b, int64_t k, int64_t n) {
    auto* handle = new (std::nothrow) PackedFp8{dtype, trans_b != 0, rhs, k, n, {}, {}, {}};
    if (!handle) return nullptr;
    const bool ok = trans_b ? handle->rhs_nk.Pack(Fp8Type(dtype), rhs, k, n) : handle->rhs_kn.Pack(Fp8Type(dtype), rhs, k, n);
    if (!ok) {
        delete handle;
        return nullptr;
    }
    return handle;
}

int ref_fp8_packed_compute(void* opaque, const uint8_t* lhs, float lhs_scale, float rhs_scale, int64_t m,
                           uint8_t* out, float out_scale) {
    auto* h = static_cast<PackedFp8*>(opaque);
    if (!h) return -1;
    if (h->transposed) {
        return x86::ComputeLinearRowMajorX86Fp8PackedTransposedRhs(Fp8Type(h->dtype), lhs, lhs_scale, h->rhs, rhs_scale,
                                                                   h->rhs_nk, nullptr, 1.0f, m, h->k, h->n,
                                                                   x86::LinearBiasType::kNone, out, out_scale, 1.0f,
                                                                   1.0f, 0, &h->workspace);
    }
    return x86::ComputeLinearRowMajorX86Fp8PackedRhs(Fp8Type(h->dtype), lhs, lhs_scale, h->rhs, rhs_scale, h->rhs_kn,
                                                     nullptr, 1.0f, m, h->k, h->n, x86::LinearBiasType::kNone, out,
                                                     out_scale, 1.0f, 1.0f, 0, &h->workspace);
}

int ref_fp8_packed_argmax(void* opaque, const uint8_t* lhs, float lhs_scale, float rhs_scale, float out_scale,
                          int64_t* token) {
    auto* h = static_cast<PackedFp8*>(opaque);
    if (!h || !h->transposed) return -1;
    return x86::ComputeLinearRowMajorX86Fp8TransposedRhsArgmax(Fp8Type(h->dtype), lhs, lhs_scale, h->rhs, rhs_scale,
                                                               &h->rhs_nk, h->k, h->n, out_scale, token,
                                                               &h->workspace, 0);
}

void ref_fp8_packed_destroy(void* opaque) { delete static_cast<PackedFp8*>(opaque); }

// Prepared x86 BF16 LM-head argmax (QwenGemmArgmaxKernel<X86,BF16>::Prepare + compute).
void* ref_bf16_argmax_create(const uint16_t* rhs_nk, int64_t k, int64_t n) {
    auto* handle = new (std::nothrow) PackedBf16{rhs_nk, k, n, {}, {}};
    if (!handle) return nullptr;
    if (!handle->packed.Pack(rhs_nk, k, n)) {
        delete handle;
        return nullptr;
    }
    return handle;
}

int ref_bf16_argmax_compute(void* opaque, const uint16_t* lhs, int64_t* token) {
    auto* h = static_cast<PackedBf16*>(opaque);
    if (!h) return -1;
    return x86::ComputeLinearRowMajorX86Bf16PackedTransposedRhsArgmax(lhs, h->rhs, h->packed, h->k, h->n, token,
                                                                       &h->workspace, 0);
}

void ref_bf16_argmax_destroy(void* opaque) { delete static_cast<PackedBf16*>(opaque); }

}  // extern "C"
