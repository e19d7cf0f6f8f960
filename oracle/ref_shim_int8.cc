// ref_shim_int8.cc -- a C-ABI over Feather's own x86 INT8 kernels (Gemm/FC and Conv2D).
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile (target `ref`) with src/kernel/x86/int8.cc and the
// Tensor pieces it needs (src/core/tensor.cc, dim.cc, memory.cc) straight from the Feather tree, into
// oracle/_ref/libfeather_ref.so.  Used to pin the oracle's INT8 Gemm and Conv2D against the reference's x86
// code and as bench.py's C1/C4 CPU baseline ("kind": "reference").  Nothing in the shipped library uses it.
//
// The kernels are reached the way Feather's executor reaches them: a KernelBase specialisation
// (GemmKernel / FcKernel / Conv2DKernel<DeviceType::X86, DataType::INT8>, src/kernel/x86/int8.cc:2353-2380)
// with a parameter struct of shared Tensors (src/operator/params.h) and compute().  A handle keeps the
// tensors and the kernel (and with it the conv's packed-weight caches) across calls, so repeated calls time
// compute() alone.
#include <cstdint>
#include <cstring>
#include <memory>
#include <vector>

#include "core/tensor.h"
#include "src/kernel/conv2d.h"
#include "src/kernel/fc.h"
#include "src/kernel/gemm.h"
#include "src/operator/params.h"

#if defined(FEATHER_WITH_OPENMP)
#include <omp.h>
#endif

using feather::DataLayout;
using feather::DataType;
using feather::DeviceType;
using feather::QuantizationGranularity;
using feather::QuantizationParams;
using feather::Tensor;

namespace {

QuantizationParams PerTensor(float scale, int32_t zero_point) {
    QuantizationParams q;
    q.enabled = true;
    q.scale = scale;
    q.zero_point = zero_point;
    q.scales = {scale};
    q.zero_points = {zero_point};
    return q;
}

QuantizationParams PerChannel(const float* scales, int64_t channels, int64_t axis) {
    QuantizationParams q;
    q.enabled = true;
    q.scales.assign(scales, scales + channels);
    q.zero_points.assign(static_cast<size_t>(channels), 0);
    q.scale = q.scales.front();
    q.zero_point = 0;
    q.granularity = channels == 1 ? QuantizationGranularity::kPerTensor : QuantizationGranularity::kPerChannel;
    q.axis = channels == 1 ? -1 : axis;
    return q;
}

template <typename T>
std::shared_ptr<Tensor> MakeTensor(const T* data, const std::vector<int64_t>& shape, DataType dtype) {
    size_t count = 1;
    for (int64_t d : shape) count *= static_cast<size_t>(d);
    auto t = std::make_shared<Tensor>();
    t->Assign<T>(data ? std::vector<T>(data, data + count) : std::vector<T>(count, T(0)), shape);
    t->set_data_type(dtype);
    return t;
}

struct I8Gemm {
    std::shared_ptr<feather::operators::GemmParam> param;
    feather::kernel::GemmKernel<DeviceType::X86, DataType::INT8> kernel;
};

struct I8Conv {
    std::shared_ptr<feather::operators::Conv2dParam> param;
    feather::kernel::Conv2DKernel<DeviceType::X86, DataType::INT8> kernel;
};

}  // namespace

extern "C" {

// Gemm(transB = 1), INT8 in/out, per-tensor activation/output, per-output-channel weight scales (axis 0),
// INT32 bias [N] or none.  `threads` > 0 sets the OpenMP thread count for the calls (the x86 Gemm itself
// is single-threaded, src/kernel/x86/int8.cc:514-572).
void* ref_i8_gemm_create(const int8_t* a, float s_a, int32_t zp_a, int64_t m, int64_t k, const int8_t* w_nk,
                         const float* s_w, int64_t n_scale, int64_t n, const int32_t* bias, float alpha, float beta,
                         float s_out, int32_t zp_out) {
    auto* h = new I8Gemm();
    h->param = std::make_shared<feather::operators::GemmParam>();
    auto& p = *h->param;
    p.a = MakeTensor<int8_t>(a, {m, k}, DataType::INT8);
    p.a->set_quantization(PerTensor(s_a, zp_a));
    p.b = MakeTensor<int8_t>(w_nk, {n, k}, DataType::INT8);
    p.b->set_quantization(PerChannel(s_w, n_scale, 0));
    if (bias) p.bias = MakeTensor<int32_t>(bias, {n}, DataType::INT32);
    p.out = MakeTensor<int8_t>(nullptr, {m, n}, DataType::INT8);
    p.out->set_quantization(PerTensor(s_out, zp_out));
    p.alpha = alpha;
    p.beta = beta;
    p.trans_a = false;
    p.trans_b = true;
    h->kernel.SetParamOwner(h->param);
    return h;
}

int ref_i8_gemm_compute(void* opaque) {
    auto* h = static_cast<I8Gemm*>(opaque);
    return h->kernel.compute();
}

// The kernel owns the parameter snapshot it was given; its output tensor is read back here.
void ref_i8_gemm_output(void* opaque, int8_t* out) {
    auto* h = static_cast<I8Gemm*>(opaque);
    auto* p = h->kernel.ParamAs<feather::operators::GemmParam>();
    std::memcpy(out, p->out->raw_data(), static_cast<size_t>(p->out->numel()));
}

void ref_i8_gemm_destroy(void* opaque) { delete static_cast<I8Gemm*>(opaque); }

// Conv2D, INT8, NCHW (layout 0) or NHWC (layout 1) activations, weight [OC, C/group, KH, KW],
// per-tensor activation/output, per-output-channel weight scales, INT32 bias [OC] or none.
void* ref_i8_conv2d_create(const int8_t* x, int64_t n, int64_t c, int64_t h, int64_t w, int layout, float s_in,
                           int32_t zp_in, const int8_t* wt, int64_t oc, int64_t kh, int64_t kw, int32_t group,
                           const float* s_w, const int32_t* bias, int32_t stride_h, int32_t stride_w, int32_t pad_h,
                           int32_t pad_w, int32_t dil_h, int32_t dil_w, int64_t oh, int64_t ow, float s_out,
                           int32_t zp_out) {
    auto* hd = new I8Conv();
    hd->param = std::make_shared<feather::operators::Conv2dParam>();
    auto& p = *hd->param;
    const DataLayout lay = layout == 1 ? DataLayout::NHWC : DataLayout::NCHW;
    const std::vector<int64_t> in_shape = layout == 1 ? std::vector<int64_t>{n, h, w, c} : std::vector<int64_t>{n, c, h, w};
    const std::vector<int64_t> out_shape =
        layout == 1 ? std::vector<int64_t>{n, oh, ow, oc} : std::vector<int64_t>{n, oc, oh, ow};
    p.input = MakeTensor<int8_t>(x, in_shape, DataType::INT8);
    p.input->set_layout(lay);
    p.input->set_quantization(PerTensor(s_in, zp_in));
    p.w = MakeTensor<int8_t>(wt, {oc, c / group, kh, kw}, DataType::INT8);
    p.w->set_quantization(PerChannel(s_w, oc, 0));
    if (bias) p.bias = MakeTensor<int32_t>(bias, {oc}, DataType::INT32);
    p.out = MakeTensor<int8_t>(nullptr, out_shape, DataType::INT8);
    p.out->set_layout(lay);
    p.out->set_quantization(PerTensor(s_out, zp_out));
    p.stride_h = stride_h;
    p.stride_w = stride_w;
    p.pad_h = pad_h;
    p.pad_w = pad_w;
    p.dilation_h = dil_h;
    p.dilation_w = dil_w;
    p.group = group;
    hd->kernel.SetParamOwner(hd->param);
    return hd;
}

int ref_i8_conv2d_compute(void* opaque) { return static_cast<I8Conv*>(opaque)->kernel.compute(); }

void ref_i8_conv2d_output(void* opaque, int8_t* out) {
    auto* hd = static_cast<I8Conv*>(opaque);
    auto* p = hd->kernel.ParamAs<feather::operators::Conv2dParam>();
    std::memcpy(out, p->out->raw_data(), static_cast<size_t>(p->out->numel()));
}

void ref_i8_conv2d_destroy(void* opaque) { delete static_cast<I8Conv*>(opaque); }

// 1 when this host has AVX-VNNI, i.e. the x86 conv takes its VNNI 4-pixel path (int8.cc:397-446).
int ref_has_avx_vnni(void) { return __builtin_cpu_supports("avxvnni") ? 1 : 0; }

void ref_set_threads(int threads) {
#if defined(FEATHER_WITH_OPENMP)
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

}  // extern "C"
