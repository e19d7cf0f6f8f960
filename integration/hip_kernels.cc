// hip_kernels.cc -- the `hip` device's kernels for Feather's quantized linear hot path, registered with
// KernelDispatcher::RegisterCandidate(DeviceType::HIP, ...) (include/core/kernel.h:226-237).
//
// Each class is a KernelBase (include/core/kernel.h:81-196) over one libfhip entry point (include/fhip.h):
//   * Supports() returns kUnsupported for shapes or quantization schemes libfhip does not cover, so the
//     dispatcher moves on to the next candidate (the Common kernel, unless kRequireRequested);
//   * Prepare() prepares an immutable weight once (fhip_weight_prepare, cached per session);
//   * compute() returns 0, or -1 exactly where the reference kernel fails.
// INT8 nodes that libfhip declines (a possible int32 partial-sum overflow, nonzero weight zero points) are
// refused in Supports() from the host bytes of the immutable weight and bias, so the Common kernel --
// which returns -1 exactly where a sum leaves int32 (common/gemm.cc:177-181) -- runs them.
// Tensors live as device replicas of the session's HipExecutionContext (hip_runtime.h); outputs stay on
// the device until BackendContext::ReadHost.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <memory>
#include <string>
#include <type_traits>
#include <vector>

#include "core/kernel.h"
#include "core/shape_utils.h"
#include "hip_runtime.h"
#include "src/operator/params.h"
#include "hip_fp8_linear.h"

namespace feather {
namespace kernel {
namespace {

using hip_detail::CurrentContext;
using hip_detail::HipExecutionContext;

// fhip.h's dtype codes are Feather's DataType values (include/util/types.h:32-47).
static_assert(static_cast<int>(DataType::INT8) == FHIP_INT8, "dtype code");
static_assert(static_cast<int>(DataType::FP16) == FHIP_FP16, "dtype code");
static_assert(static_cast<int>(DataType::FP32) == FHIP_FP32, "dtype code");
static_assert(static_cast<int>(DataType::INT32) == FHIP_INT32, "dtype code");
static_assert(static_cast<int>(DataType::INT64) == FHIP_INT64, "dtype code");
static_assert(static_cast<int>(DataType::BF16) == FHIP_BF16, "dtype code");
static_assert(static_cast<int>(DataType::FP8E4M3) == FHIP_FP8E4M3, "dtype code");
static_assert(static_cast<int>(DataType::FP8E5M2) == FHIP_FP8E5M2, "dtype code");

int Code(DataType dtype) { return static_cast<int>(dtype); }
bool IsFp8(DataType dtype) { return dtype == DataType::FP8E4M3 || dtype == DataType::FP8E5M2; }
bool IsFloat(DataType dtype) { return dtype == DataType::FP32 || dtype == DataType::FP16 || dtype == DataType::BF16; }

Status Unsupported(const std::string& why) { return Status::Error(StatusCode::kUnsupported, "hip: " + why); }

size_t TensorBytes(const Tensor& tensor) {
    size_t bytes = 0;
    if (!CheckedTensorBytes(tensor.dims().data(), tensor.data_type(), &bytes)) bytes = tensor.memory_size();
    return bytes;
}

bool PerTensor(const Tensor& tensor) { return HasCompatiblePerTensorQuantization(tensor.quantization()); }

int Ok(int rc) { return rc == FHIP_OK ? 0 : -1; }

// Largest |bias| of an INT32 bias (host bytes), the term fhip_i8_linear adds to its int32 overflow bound.
int32_t BiasAbsMax(const std::shared_ptr<Tensor>& bias) {
    if (bias == nullptr || !bias->IsInitialized()) return 0;
    const int32_t* values = bias->data<int32_t>();
    int64_t best = 0;
    for (int64_t i = 0; i < bias->numel(); ++i) best = std::max<int64_t>(best, std::llabs(static_cast<int64_t>(values[i])));
    return best > std::numeric_limits<int32_t>::max() ? std::numeric_limits<int32_t>::max() : static_cast<int32_t>(best);
}

// libfhip's INT8 decline rule (fhip_i8_linear / fhip_i8_conv2d return FHIP_ERR_UNSUPPORTED): weight zero
// points must be 0, and K * (128 + |zp_a|) * max|w| + |bias| must stay below 2^31, so no int32 partial sum
// can overflow.  Evaluated on the weight's and bias's host bytes.
bool I8Declined(const Tensor& w, int64_t k, int32_t zp_a, const std::shared_ptr<Tensor>& bias) {
    const auto& q = w.quantization();
    for (int32_t zp : q.zero_points)
        if (zp != 0) return true;
    if (q.zero_point_at(0) != 0) return true;
    const int8_t* values = w.data<int8_t>();
    int32_t max_abs_w = 0;
    for (int64_t i = 0; i < w.numel(); ++i) max_abs_w = std::max<int32_t>(max_abs_w, std::abs(static_cast<int32_t>(values[i])));
    const double bound = static_cast<double>(k) * (128.0 + std::abs(zp_a)) * max_abs_w + static_cast<double>(BiasAbsMax(bias));
    return !(bound < 2147483647.0);
}

// ---- FP8 MatMul / Gemm / FC (common/matmul.cc:56-130, gemm.cc:62-100, fc.cc:48-73) ----------------
struct Fp8LinearView {
    std::shared_ptr<Tensor> a, w, bias, out;
    int64_t m{0}, k{0}, n{0};
    int layout{FHIP_LAYOUT_KN};
    float alpha{1.0f}, beta{1.0f};
};

Status CheckFp8Linear(const Fp8LinearView& v, DataType dtype) {
    if (!v.a || !v.w || !v.out) return Unsupported("missing tensor");
    if (v.a->data_type() != dtype || v.w->data_type() != dtype || v.out->data_type() != dtype)
        return Unsupported("FP8 linear needs matching FP8 input, weight and output dtypes");
    if (!PerTensor(*v.a) || !PerTensor(*v.w) || !PerTensor(*v.out))
        return Unsupported("FP8 linear needs per-tensor scales");
    if (v.w->dims().size() != 2 || v.k <= 0 || v.n <= 0 || v.m < 0) return Unsupported("FP8 linear needs a 2-D weight");
    if (v.bias && v.bias->IsInitialized() && (v.bias->data_type() != dtype || !PerTensor(*v.bias)))
        return Unsupported("FP8 bias must be per-tensor FP8 of the same format");
    return Status::Ok();
}

int RunFp8Linear(const Fp8LinearView& v, DataType dtype, fhip_weight* weight) {
    auto ctx = CurrentContext();
    if (!ctx) return -1;
    if (*weight == nullptr && ctx->AcquireLinearWeight(*v.w, Code(dtype), v.k, v.n, v.layout, weight) != FHIP_OK)
        return -1;
    const void* a = nullptr;
    const void* bias = nullptr;
    void* out = nullptr;
    int bias_kind = FHIP_BIAS_NONE;
    float bias_scale = 1.0f;
    if (v.bias && v.bias->IsInitialized()) {
        bias_kind = v.bias->numel() == v.n ? FHIP_BIAS_VECTOR : FHIP_BIAS_MATRIX;
        if (bias_kind == FHIP_BIAS_MATRIX && v.bias->numel() != v.m * v.n) return -1;
        bias_scale = v.bias->quantization_scale();
        if (ctx->AcquireInput(*v.bias, &bias) != FHIP_OK) return -1;
    }
    if (ctx->AcquireInput(*v.a, &a) != FHIP_OK || ctx->AcquireOutput(*v.out, TensorBytes(*v.out), &out) != FHIP_OK)
        return -1;
    return Ok(fhip_fp8_linear(ctx->handle(), Code(dtype), a, v.a->quantization_scale(), v.m, *weight,
                              v.w->quantization_scale(), static_cast<const uint8_t*>(bias), bias_scale, bias_kind,
                              v.alpha, v.beta, Code(dtype), out, v.out->quantization_scale()));
}

template <DataType dtype>
class HipFp8MatMulKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::MatMulParam>();
        if (!p) return Unsupported("no parameters");
        return CheckFp8Linear(View(*p), dtype);
    }
    int32_t Prepare() override {
        auto* p = ParamAs<operators::MatMulParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx || !p->b->is_immutable()) return 0;
        const auto v = View(*p);
        return Ok(ctx->AcquireLinearWeight(*p->b, Code(dtype), v.k, v.n, FHIP_LAYOUT_KN, &weight_));
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::MatMulParam>();
        if (!p) return -1;
        if (!p->b->is_immutable()) weight_ = nullptr;  // a mutable weight is prepared for its current version
        return RunFp8Linear(View(*p), dtype, &weight_);
    }

 private:
    static Fp8LinearView View(const operators::MatMulParam& p) {
        Fp8LinearView v{p.a, p.b, nullptr, p.out};
        if (p.a && p.b && p.b->dims().size() == 2 && !p.a->dims().empty()) {
            v.k = p.a->dims().data().back();
            v.n = p.b->dims()[1];
            v.m = v.k > 0 && p.b->dims()[0] == v.k ? p.a->numel() / v.k : -1;
        }
        return v;
    }
    fhip_weight weight_{nullptr};
};

template <DataType dtype>
class HipFp8GemmKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::GemmParam>();
        if (!p) return Unsupported("no parameters");
        if (p->trans_a) return Unsupported("Gemm with transA");
        return CheckFp8Linear(View(*p), dtype);
    }
    int32_t Prepare() override {
        auto* p = ParamAs<operators::GemmParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx || !p->b->is_immutable()) return 0;
        const auto v = View(*p);
        return Ok(ctx->AcquireLinearWeight(*p->b, Code(dtype), v.k, v.n, v.layout, &weight_));
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::GemmParam>();
        if (!p || p->trans_a) return -1;
        if (!p->b->is_immutable()) weight_ = nullptr;
        return RunFp8Linear(View(*p), dtype, &weight_);
    }

 private:
    static Fp8LinearView View(const operators::GemmParam& p) {
        Fp8LinearView v{p.a, p.b, p.bias, p.out};
        v.alpha = p.alpha;
        v.beta = p.beta;
        v.layout = p.trans_b ? FHIP_LAYOUT_NK : FHIP_LAYOUT_KN;
        if (p.a && p.b && p.b->dims().size() == 2 && !p.a->dims().empty()) {
            v.k = p.a->dims().data().back();
            const int64_t b_k = p.trans_b ? p.b->dims()[1] : p.b->dims()[0];
            v.n = p.trans_b ? p.b->dims()[0] : p.b->dims()[1];
            v.m = v.k > 0 && b_k == v.k ? p.a->numel() / v.k : -1;
        }
        return v;
    }
    fhip_weight weight_{nullptr};
};

template <DataType dtype>
class HipFp8FcKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::FcParam>();
        if (!p) return Unsupported("no parameters");
        return CheckFp8Linear(View(*p), dtype);
    }
    int32_t Prepare() override {
        auto* p = ParamAs<operators::FcParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx || !p->w->is_immutable()) return 0;
        const auto v = View(*p);
        return Ok(ctx->AcquireLinearWeight(*p->w, Code(dtype), v.k, v.n, FHIP_LAYOUT_KN, &weight_));
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::FcParam>();
        if (!p) return -1;
        if (!p->w->is_immutable()) weight_ = nullptr;
        return RunFp8Linear(View(*p), dtype, &weight_);
    }

 private:
    static Fp8LinearView View(const operators::FcParam& p) {
        Fp8LinearView v{p.input, p.w, p.bias, p.out};
        if (p.input && p.w && p.w->dims().size() == 2 && p.input->dims().size() == 2 &&
            p.input->dims()[1] == p.w->dims()[0]) {
            v.m = p.input->dims()[0];
            v.k = p.input->dims()[1];
            v.n = p.w->dims()[1];
        }
        return v;
    }
    fhip_weight weight_{nullptr};
};

// ---- INT8 MatMul / FC / Gemm (common/matmul.cc:156-261, fc.cc:105-159, gemm.cc:136-198) ------------
struct I8LinearView {
    std::shared_ptr<Tensor> a, w, bias, out;
    int64_t m{-1}, k{0}, n{0};
    int layout{FHIP_LAYOUT_KN};
    int kind{FHIP_I8_MATMUL};
    float alpha{1.0f}, beta{1.0f};
};

Status CheckI8Linear(const I8LinearView& v) {
    if (!v.a || !v.w || !v.out) return Unsupported("missing tensor");
    if (v.a->data_type() != DataType::INT8 || v.w->data_type() != DataType::INT8 || v.out->data_type() != DataType::INT8)
        return Unsupported("INT8 linear needs INT8 input, weight and output");
    if (!PerTensor(*v.a) || !PerTensor(*v.out)) return Unsupported("per-tensor activation and output quantization only");
    if (v.m <= 0 || v.k <= 0 || v.n <= 0) return Unsupported("shape outside the HIP INT8 linear");
    if (v.bias && v.bias->IsInitialized() &&
        (v.bias->data_type() != DataType::INT32 || (v.bias->numel() != v.n && v.bias->numel() != v.m * v.n)))
        return Unsupported("INT32 [N] or [M, N] bias only");
    if (!v.w->is_immutable() || !v.w->IsInitialized()) return Unsupported("INT8 weights must be immutable");
    // only FC adds the bias inside the int32 sum; Gemm scales it in double (common/gemm.cc:187-188)
    if (I8Declined(*v.w, v.k, v.a->quantization().zero_point_at(0), v.kind == FHIP_I8_FC ? v.bias : nullptr))
        return Unsupported("INT8 sums could leave int32, or weight zero points are nonzero: Common decides");
    return Status::Ok();
}

int RunI8Linear(const I8LinearView& v, fhip_weight* weight, int32_t bias_abs_max) {
    auto ctx = CurrentContext();
    if (!ctx) return -1;
    if (*weight == nullptr && ctx->AcquireLinearWeight(*v.w, FHIP_INT8, v.k, v.n, v.layout, weight) != FHIP_OK)
        return -1;
    const void* a = nullptr;
    const void* bias = nullptr;
    void* out = nullptr;
    int bias_kind = FHIP_BIAS_NONE;
    if (v.bias && v.bias->IsInitialized()) {
        bias_kind = v.bias->numel() == v.n ? FHIP_BIAS_VECTOR : FHIP_BIAS_MATRIX;
        if (ctx->AcquireInput(*v.bias, &bias) != FHIP_OK) return -1;
    }
    if (ctx->AcquireInput(*v.a, &a) != FHIP_OK || ctx->AcquireOutput(*v.out, TensorBytes(*v.out), &out) != FHIP_OK)
        return -1;
    const auto& qa = v.a->quantization();
    const auto& qo = v.out->quantization();
    return Ok(fhip_i8_linear(ctx->handle(), v.kind, static_cast<const int8_t*>(a), qa.scale_at(0), qa.zero_point_at(0),
                             v.m, *weight, static_cast<const int32_t*>(bias), bias_kind, bias_abs_max, v.alpha, v.beta,
                             static_cast<int8_t*>(out), qo.scale_at(0), qo.zero_point_at(0)));
}

template <typename Param>
class HipI8LinearKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<Param>();
        if (!p) return Unsupported("no parameters");
        if constexpr (std::is_same<Param, operators::GemmParam>::value)
            if (p->trans_a || !std::isfinite(p->alpha) || !std::isfinite(p->beta)) return Unsupported("Gemm form");
        return CheckI8Linear(View(*p));
    }
    int32_t Prepare() override {
        auto* p = ParamAs<Param>();
        auto ctx = CurrentContext();
        if (!p || !ctx) return 0;
        const auto v = View(*p);
        if (v.bias && v.bias->is_immutable()) bias_abs_max_ = BiasAbsMax(v.bias);
        if (!v.w->is_immutable()) return 0;
        return Ok(ctx->AcquireLinearWeight(*v.w, FHIP_INT8, v.k, v.n, v.layout, &weight_));
    }
    int32_t compute() override {
        auto* p = ParamAs<Param>();
        if (!p) return -1;
        const auto v = View(*p);
        if (!v.w->is_immutable()) weight_ = nullptr;
        const int32_t bias_abs_max = v.bias && v.bias->is_immutable() && bias_abs_max_ >= 0 ? bias_abs_max_ : BiasAbsMax(v.bias);
        return RunI8Linear(v, &weight_, bias_abs_max);
    }

 private:
    static I8LinearView View(const Param& p) {
        I8LinearView v;
        if constexpr (std::is_same<Param, operators::MatMulParam>::value) {
            v = I8LinearView{p.a, p.b, nullptr, p.out};
            v.kind = FHIP_I8_MATMUL;
            if (p.a && p.b && p.b->dims().size() == 2 && !p.a->dims().empty()) {
                v.k = p.a->dims().data().back();
                v.n = p.b->dims()[1];
                v.m = v.k > 0 && p.b->dims()[0] == v.k ? p.a->numel() / v.k : -1;
            }
        } else if constexpr (std::is_same<Param, operators::FcParam>::value) {
            v = I8LinearView{p.input, p.w, p.bias, p.out};
            v.kind = FHIP_I8_FC;
            if (p.input && p.w && p.input->dims().size() == 2 && p.w->dims().size() == 2 &&
                p.input->dims()[1] == p.w->dims()[0]) {
                v.m = p.input->dims()[0];
                v.k = p.input->dims()[1];
                v.n = p.w->dims()[1];
            }
        } else {
            v = I8LinearView{p.a, p.b, p.bias, p.out};
            v.kind = FHIP_I8_GEMM;
            v.alpha = p.alpha;
            v.beta = p.beta;
            v.layout = p.trans_b ? FHIP_LAYOUT_NK : FHIP_LAYOUT_KN;
            if (p.a && p.b && p.b->dims().size() == 2 && !p.a->dims().empty()) {
                v.k = p.a->dims().data().back();
                const int64_t b_k = p.trans_b ? p.b->dims()[1] : p.b->dims()[0];
                v.n = p.trans_b ? p.b->dims()[0] : p.b->dims()[1];
                v.m = v.k > 0 && b_k == v.k ? p.a->numel() / v.k : -1;
            }
        }
        return v;
    }
    fhip_weight weight_{nullptr};
    int32_t bias_abs_max_{-1};
};

// ---- INT8 Conv2D (common/conv2d.cc:482-581) ---------------------------------------------------------
class HipI8Conv2DKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::Conv2dParam>();
        if (!p || !p->input || !p->w || !p->out) return Unsupported("missing tensor");
        if (p->input->data_type() != DataType::INT8 || p->w->data_type() != DataType::INT8 ||
            p->out->data_type() != DataType::INT8)
            return Unsupported("INT8 conv needs INT8 input, weight and output");
        if (p->input->dims().size() != 4 || p->w->dims().size() != 4 || p->out->dims().size() != 4)
            return Unsupported("4-D tensors only");
        if (!PerTensor(*p->input) || !PerTensor(*p->out)) return Unsupported("per-tensor activation quantization only");
        if (NormalizeDataLayout(p->input->layout()) != NormalizeDataLayout(p->out->layout()))
            return Unsupported("input and output layouts differ");
        if (p->bias && p->bias->IsInitialized() &&
            (p->bias->data_type() != DataType::INT32 || p->bias->numel() != p->w->dims()[0]))
            return Unsupported("INT32 [OC] bias only");
        if (!p->w->is_immutable() || !p->w->IsInitialized()) return Unsupported("INT8 weights must be immutable");
        const int64_t k = p->w->dims()[1] * p->w->dims()[2] * p->w->dims()[3];
        if (I8Declined(*p->w, k, p->input->quantization().zero_point_at(0), p->bias))
            return Unsupported("INT8 sums could leave int32, or weight zero points are nonzero: Common decides");
        return Status::Ok();
    }
    int32_t Prepare() override {
        auto* p = ParamAs<operators::Conv2dParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx) return 0;
        if (p->bias && p->bias->is_immutable()) bias_abs_max_ = BiasAbsMax(p->bias);
        if (!p->w->is_immutable()) return 0;
        return Ok(ctx->AcquireConvWeight(*p->w, p->group, &weight_));
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::Conv2dParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx) return -1;
        ImageShape4D in_shape, out_shape;
        const DataLayout layout = NormalizeDataLayout(p->input->layout());
        if (!DecodeImageShape4D(p->input->dims().data(), p->input->layout(), &in_shape) ||
            !DecodeImageShape4D(p->out->dims().data(), p->out->layout(), &out_shape))
            return -1;
        if (!p->w->is_immutable()) weight_ = nullptr;
        if (weight_ == nullptr && ctx->AcquireConvWeight(*p->w, p->group, &weight_) != FHIP_OK) return -1;
        const void* in = nullptr;
        const void* bias = nullptr;
        void* out = nullptr;
        if (p->bias && p->bias->IsInitialized() && ctx->AcquireInput(*p->bias, &bias) != FHIP_OK) return -1;
        if (ctx->AcquireInput(*p->input, &in) != FHIP_OK ||
            ctx->AcquireOutput(*p->out, TensorBytes(*p->out), &out) != FHIP_OK)
            return -1;
        const int32_t bias_abs_max =
            p->bias && p->bias->is_immutable() && bias_abs_max_ >= 0 ? bias_abs_max_ : BiasAbsMax(p->bias);
        const auto& qi = p->input->quantization();
        const auto& qo = p->out->quantization();
        return Ok(fhip_i8_conv2d(ctx->handle(), static_cast<const int8_t*>(in), in_shape.n, in_shape.c, in_shape.h,
                                 in_shape.w, layout == DataLayout::NHWC ? FHIP_NHWC : FHIP_NCHW, qi.scale_at(0),
                                 qi.zero_point_at(0), weight_, static_cast<const int32_t*>(bias), bias_abs_max,
                                 p->stride_h, p->stride_w, p->pad_h, p->pad_w, p->dilation_h, p->dilation_w,
                                 static_cast<int8_t*>(out), out_shape.h, out_shape.w, qo.scale_at(0),
                                 qo.zero_point_at(0)));
    }

 private:
    fhip_weight weight_{nullptr};
    int32_t bias_abs_max_{-1};
};

// ---- QuantizeLinear / DequantizeLinear (common/quantize_linear_utils.h:187-341) ---------------------
// Scale and zero-point tensors are small graph constants read on the host, as the Common kernel does.
bool ReadScales(const Tensor& scale, const Tensor* zero, std::vector<float>* scales, std::vector<int32_t>* zps) {
    if (scale.data_type() != DataType::FP32 || scale.numel() <= 0) return false;
    scales->assign(scale.data<float>(), scale.data<float>() + scale.numel());
    zps->clear();
    if (zero != nullptr && zero->IsInitialized() && zero->numel() > 0) {
        if (zero->data_type() == DataType::INT8) {
            for (int64_t i = 0; i < zero->numel(); ++i) zps->push_back(zero->data<int8_t>()[i]);
        } else if (zero->data_type() == DataType::INT32) {
            zps->assign(zero->data<int32_t>(), zero->data<int32_t>() + zero->numel());
        } else {
            return false;
        }
    } else {
        zps->push_back(0);
    }
    return zps->size() == 1 || zps->size() == scales->size();
}

// Element i uses parameter (i / inner) % channels for a per-channel axis.
bool ChannelGeometry(const Tensor& input, int64_t axis, size_t channels, int64_t* inner) {
    *inner = 1;
    if (channels == 1) return true;
    const auto& d = input.dims().data();
    if (axis < 0) axis += static_cast<int64_t>(d.size());
    if (axis < 0 || axis >= static_cast<int64_t>(d.size()) || d[axis] != static_cast<int64_t>(channels)) return false;
    for (size_t i = static_cast<size_t>(axis) + 1; i < d.size(); ++i) *inner *= d[i];
    return true;
}

class HipQuantizeLinearKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::QuantizeLinearParam>();
        if (!p || !p->input || !p->scale || !p->out) return Unsupported("missing tensor");
        if (!IsFloat(p->input->data_type())) return Unsupported("FP32/FP16/BF16 input only");
        return Status::Ok();
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::QuantizeLinearParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx || !p->input->IsInitialized() || p->input->numel() <= 0) return -1;
        std::vector<float> scales;
        std::vector<int32_t> zps;
        int64_t inner = 1;
        if (!ReadScales(*p->scale, p->zero_point.get(), &scales, &zps) ||
            !ChannelGeometry(*p->input, p->axis, scales.size(), &inner))
            return -1;
        const int64_t count = p->input->numel();
        p->out->Resize(p->input->dims().data());
        p->out->set_data_type(DataType::INT8);
        const void* in = nullptr;
        void* out = nullptr;
        if (ctx->AcquireInput(*p->input, &in) != FHIP_OK || ctx->AcquireOutput(*p->out, count, &out) != FHIP_OK) return -1;
        const int rc = fhip_quantize_linear(ctx->handle(), Code(p->input->data_type()), in, count,
                                            static_cast<int64_t>(scales.size()), inner, scales.data(), zps.data(),
                                            static_cast<int64_t>(zps.size()), static_cast<int8_t*>(out));
        if (rc != FHIP_OK) return -1;
        // the output's quantization metadata, as ComputeQuantizeLinear sets it (quantize_linear_utils.h:187-211)
        QuantizationParams q;
        q.enabled = true;
        q.scales = scales;
        q.zero_points = zps;
        q.scale = scales.front();
        q.zero_point = zps.front();
        q.granularity = scales.size() == 1 ? QuantizationGranularity::kPerTensor : QuantizationGranularity::kPerChannel;
        q.axis = scales.size() == 1 ? -1 : (p->axis < 0 ? p->axis + static_cast<int64_t>(p->input->dims().size()) : p->axis);
        p->out->set_quantization(q);
        return 0;
    }
};

class HipDequantizeLinearKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::DequantizeLinearParam>();
        if (!p || !p->input || !p->scale || !p->out) return Unsupported("missing tensor");
        if (p->input->data_type() != DataType::INT8 || !IsFloat(p->to)) return Unsupported("INT8 -> FP32/FP16/BF16 only");
        return Status::Ok();
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::DequantizeLinearParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx || !p->input->IsInitialized() || p->input->numel() <= 0) return -1;
        std::vector<float> scales;
        std::vector<int32_t> zps;
        int64_t inner = 1;
        if (!ReadScales(*p->scale, p->zero_point.get(), &scales, &zps) ||
            !ChannelGeometry(*p->input, p->axis, scales.size(), &inner))
            return -1;
        const int64_t count = p->input->numel();
        p->out->Resize(p->input->dims().data());
        p->out->set_data_type(p->to);
        const void* in = nullptr;
        void* out = nullptr;
        if (ctx->AcquireInput(*p->input, &in) != FHIP_OK ||
            ctx->AcquireOutput(*p->out, TensorBytes(*p->out), &out) != FHIP_OK)
            return -1;
        return Ok(fhip_dequantize_linear(ctx->handle(), static_cast<const int8_t*>(in), count,
                                         static_cast<int64_t>(scales.size()), inner, scales.data(), zps.data(),
                                         static_cast<int64_t>(zps.size()), Code(p->to), out));
    }
};

// ---- Cast between FP8 and FP32/FP16/BF16 (common/cast.cc:62-165) ------------------------------------
class HipFp8CastKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::CastParam>();
        if (!p || !p->input || !p->out) return Unsupported("missing tensor");
        const DataType from = p->input->data_type();
        const bool ok = (IsFp8(from) && (IsFloat(p->to) || IsFp8(p->to))) || (IsFloat(from) && IsFp8(p->to));
        if (!ok) return Unsupported("Cast with an FP8 side only");
        if (!PerTensor(*p->input) || !PerTensor(*p->out)) return Unsupported("per-tensor FP8 scales only");
        return Status::Ok();
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::CastParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx || !p->input->IsInitialized()) return -1;
        const int64_t count = p->input->numel();
        p->out->Resize(p->input->dims().data());
        p->out->set_data_type(p->to);
        const void* in = nullptr;
        void* out = nullptr;
        if (ctx->AcquireInput(*p->input, &in) != FHIP_OK ||
            ctx->AcquireOutput(*p->out, TensorBytes(*p->out), &out) != FHIP_OK)
            return -1;
        const float src_scale = IsFp8(p->input->data_type()) ? p->input->quantization_scale() : 1.0f;
        const float dst_scale = IsFp8(p->to) ? p->out->quantization_scale() : 1.0f;
        return Ok(fhip_cast(ctx->handle(), Code(p->input->data_type()), in, src_scale, count, Code(p->to), out, dst_scale));
    }
};

// ---- QwenGemmArgmax (operator/qwen_gemm_argmax_op.cc:28-113; common/qwen_gemm_argmax.cc:28-49) -------
template <DataType dtype>
class HipQwenGemmArgmaxKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::QwenGemmArgmaxParam>();
        if (!p || !p->a || !p->b || !p->out) return Unsupported("missing tensor");
        if (p->a->data_type() != dtype || p->b->data_type() != dtype || p->b->dims().size() != 2)
            return Unsupported("QwenGemmArgmax operand dtypes");
        if (IsFp8(dtype) && (!PerTensor(*p->a) || !PerTensor(*p->b))) return Unsupported("per-tensor FP8 scales only");
        // the library's row limits (include/fhip.h): rows of whole 16-byte chunks, at most 64 KiB, V < 2^32
        const int64_t k = p->b->dims()[1], v = p->b->dims()[0];
        const int64_t row_bytes = k * (dtype == DataType::BF16 ? 2 : 1);
        if (row_bytes % 16 != 0 || row_bytes > 65536 || v >= (int64_t(1) << 32))
            return Unsupported("QwenGemmArgmax row length or vocabulary beyond the HIP kernel's limits");
        return Status::Ok();
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::QwenGemmArgmaxParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx) return -1;
        const int64_t k = p->b->dims()[1];
        const int64_t v = p->b->dims()[0];
        if (k <= 0 || v <= 0 || p->a->numel() != k) return -1;
        const void* a = nullptr;
        const void* w = nullptr;
        void* token = nullptr;
        if (ctx->AcquireInput(*p->a, &a) != FHIP_OK || ctx->AcquireInput(*p->b, &w) != FHIP_OK ||
            ctx->AcquireOutput(*p->out, sizeof(int64_t), &token) != FHIP_OK)
            return -1;
        if constexpr (dtype == DataType::BF16) {
            return Ok(fhip_bf16_gemv_argmax(ctx->handle(), static_cast<const uint16_t*>(a), 1, k,
                                            static_cast<const uint16_t*>(w), v, static_cast<int64_t*>(token), nullptr));
        } else {
            return Ok(fhip_fp8_gemv_argmax(ctx->handle(), Code(dtype), static_cast<const uint8_t*>(a),
                                           p->a->quantization_scale(), 1, k, static_cast<const uint8_t*>(w),
                                           p->b->quantization_scale(), v, p->output_scale,
                                           static_cast<int64_t*>(token)));
        }
    }
};

// ---- the fused Cast(bf16 -> fp8) -> MatMul -> Cast(fp8 -> bf16) node (HipFp8LinearOp) ---------------
class HipFusedFp8LinearKernel final : public KernelBase {
 public:
    Status Supports() const override {
        auto* p = ParamAs<operators::HipFp8LinearParam>();
        if (!p || !p->a || !p->w || !p->out) return Unsupported("missing tensor");
        if (p->a->data_type() != DataType::BF16 || !IsFp8(p->w->data_type()) || p->w->dims().size() != 2)
            return Unsupported("fused FP8 linear needs a BF16 input and a 2-D FP8 weight");
        return Status::Ok();
    }
    int32_t Prepare() override {
        auto* p = ParamAs<operators::HipFp8LinearParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx || !p->w->is_immutable()) return 0;
        return Ok(ctx->AcquireLinearWeight(*p->w, Code(p->w->data_type()), p->w->dims()[0], p->w->dims()[1],
                                           FHIP_LAYOUT_KN, &weight_));
    }
    int32_t compute() override {
        auto* p = ParamAs<operators::HipFp8LinearParam>();
        auto ctx = CurrentContext();
        if (!p || !ctx) return -1;
        const int64_t k = p->w->dims()[0];
        const int64_t n = p->w->dims()[1];
        if (k <= 0 || p->a->dims().empty() || p->a->dims().data().back() != k) return -1;
        const int64_t m = p->a->numel() / k;
        if (!p->w->is_immutable()) weight_ = nullptr;
        if (weight_ == nullptr &&
            ctx->AcquireLinearWeight(*p->w, Code(p->w->data_type()), k, n, FHIP_LAYOUT_KN, &weight_) != FHIP_OK)
            return -1;
        const void* a = nullptr;
        void* out = nullptr;
        if (ctx->AcquireInput(*p->a, &a) != FHIP_OK ||
            ctx->AcquireOutput(*p->out, TensorBytes(*p->out), &out) != FHIP_OK)
            return -1;
        // a_dtype BF16: the first Cast's Enc(x / input_scale); out_dtype BF16: the last Cast's
        // Dec(code) * output_scale -- the three nodes value for value
        return Ok(fhip_fp8_linear(ctx->handle(), FHIP_BF16, a, p->input_scale, m, weight_, p->w->quantization_scale(),
                                  nullptr, 1.0f, FHIP_BIAS_NONE, 1.0f, 1.0f, FHIP_BF16, out, p->output_scale));
    }

 private:
    fhip_weight weight_{nullptr};
};

template <typename K>
KernelDispatcher::KernelFactory Make() {
    return [] { return std::unique_ptr<KernelBase>(new K()); };
}

// Candidates outrank the Common kernels of the same key (priority 10), as a device backend's should.
bool RegisterHipKernels() {
    auto& d = KernelDispatcher::instance();
    const DeviceType hip = DeviceType::HIP;
    const DataLayout nd = DataLayout::ND;
    d.RegisterCandidate(hip, DataType::FP8E4M3, nd, "MatMul", "hip.fp8.matmul", Make<HipFp8MatMulKernel<DataType::FP8E4M3>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::FP8E5M2, nd, "MatMul", "hip.fp8.matmul", Make<HipFp8MatMulKernel<DataType::FP8E5M2>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::FP8E4M3, nd, "Gemm", "hip.fp8.gemm", Make<HipFp8GemmKernel<DataType::FP8E4M3>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::FP8E5M2, nd, "Gemm", "hip.fp8.gemm", Make<HipFp8GemmKernel<DataType::FP8E5M2>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::FP8E4M3, nd, "FC", "hip.fp8.fc", Make<HipFp8FcKernel<DataType::FP8E4M3>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::FP8E5M2, nd, "FC", "hip.fp8.fc", Make<HipFp8FcKernel<DataType::FP8E5M2>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::INT8, nd, "MatMul", "hip.int8.matmul", Make<HipI8LinearKernel<operators::MatMulParam>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::INT8, nd, "FC", "hip.int8.fc", Make<HipI8LinearKernel<operators::FcParam>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::INT8, nd, "Gemm", "hip.int8.gemm", Make<HipI8LinearKernel<operators::GemmParam>>(), {}, 10);
    for (DataLayout layout : {DataLayout::ND, DataLayout::NCHW, DataLayout::NHWC})
        d.RegisterCandidate(hip, DataType::INT8, layout, "Conv2D", "hip.int8.conv2d", Make<HipI8Conv2DKernel>(), {}, 10);
    for (DataType dtype : {DataType::FP32, DataType::FP16, DataType::BF16})
        d.RegisterCandidate(hip, dtype, nd, "QuantizeLinear", "hip.quantize_linear", Make<HipQuantizeLinearKernel>(), {}, 10);
    d.RegisterCandidate(hip, DataType::INT8, nd, "DequantizeLinear", "hip.dequantize_linear", Make<HipDequantizeLinearKernel>(), {}, 10);
    for (DataType dtype : {DataType::FP32, DataType::FP16, DataType::BF16, DataType::FP8E4M3, DataType::FP8E5M2})
        d.RegisterCandidate(hip, dtype, nd, "Cast", "hip.fp8.cast", Make<HipFp8CastKernel>(), {}, 10);
    d.RegisterCandidate(hip, DataType::BF16, nd, "QwenGemmArgmax", "hip.qwen_gemm_argmax", Make<HipQwenGemmArgmaxKernel<DataType::BF16>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::FP8E4M3, nd, "QwenGemmArgmax", "hip.qwen_gemm_argmax", Make<HipQwenGemmArgmaxKernel<DataType::FP8E4M3>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::FP8E5M2, nd, "QwenGemmArgmax", "hip.qwen_gemm_argmax", Make<HipQwenGemmArgmaxKernel<DataType::FP8E5M2>>(), {}, 10);
    d.RegisterCandidate(hip, DataType::BF16, nd, operators::kHipFp8LinearOp, "hip.fp8.linear_bf16", Make<HipFusedFp8LinearKernel>(), {}, 10);
    return true;
}

}  // namespace

// Called from RegisterBuiltinKernels() (src/kernel/register_all.cc, FEATHER_WITH_HIP) while the
// dispatcher's initialization lock is held, like EnsureCudaKernelsRegistered().
void EnsureHipKernelsRegistered() {
    static const bool registered = RegisterHipKernels();
    (void)registered;
}

}  // namespace kernel
}  // namespace feather
