// hip_fp8_linear.h -- the fused FP8 projection of the `hip` device: one node for the exported
// Cast(bf16 -> fp8) -> MatMul(fp8) -> Cast(fp8 -> bf16) chain of the Qwen FP8 export, and the graph pass
// that forms it.
//
// The node computes, value for value, what the three nodes compute (Enc(x / input_scale), the FP8 MatMul
// with its output scale, Dec(code) * output_scale) in one libfhip launch (fhip_fp8_linear with BF16 input
// and output), so the two memory-bound Casts around every projection disappear.  Its reference precedent is
// the CUDA backend's unused LaunchFp8MatMulToBf16KernelCuda (src/kernel/cuda/linear_kernels.cuh:839-862);
// the pass follows QwenGemmArgmaxFusionPass (src/pass/qwen_gemm_argmax_fusion_pass.cc:65-181).
#ifndef FEATHER_HIP_FP8_LINEAR_H
#define FEATHER_HIP_FP8_LINEAR_H

#include <memory>
#include <string>

#include "core/operator.h"
#include "pass/graph_pass.h"
#include "src/operator/params.h"

namespace feather {
namespace operators {

constexpr const char* kHipFp8LinearOp = "HipFp8Linear";

struct HipFp8LinearParam : ParamBase {
    std::shared_ptr<Tensor> a;    // BF16 activations [..., K] (the first Cast's input)
    std::shared_ptr<Tensor> w;    // FP8 weight [K, N] (the MatMul's immutable weight, with its scale)
    std::shared_ptr<Tensor> out;  // BF16 [..., N] (the last Cast's output)
    float input_scale{1.0f};      // scale of the first Cast's FP8 output
    float output_scale{1.0f};     // scale of the MatMul's FP8 output
    template <typename Visitor> void VisitTensors(Visitor&& visit) {
        visit(a);
        visit(w);
        visit(out);
    }
};

class HipFp8LinearOp : public OpBase {
 public:
    HipFp8LinearOp(std::string name, const HipFp8LinearParam& param);
    int32_t CheckShape() const override;
    int32_t InferOutputShapes() override;
    void AttachKernel(std::unique_ptr<KernelBase> kernel) override;
    std::unique_ptr<KernelBase> DetachKernel() override { return std::move(kernel_); }
    bool HasKernel() const override { return kernel_ != nullptr; }
    const KernelBase* kernel() const override { return kernel_.get(); }
    int32_t Run() override;

 private:
    void SyncIO();
    HipFp8LinearParam param_;
    std::unique_ptr<KernelBase> kernel_;
};

void EnsureHipFp8LinearOperatorRegistered();

}  // namespace operators

// Replaces Cast(bf16 -> fp8) -> MatMul -> Cast(fp8 -> bf16) with one HipFp8Linear node on graphs whose
// kernel device is HIP.  Matches only chains whose intermediate values have no other user and whose
// MatMul weight is an immutable 2-D FP8 tensor with a per-tensor scale.
class HipFp8LinearFusionPass : public GraphPass {
 public:
    const std::string& name() const override;
    int32_t Run(StaticGraph* graph) override;
    bool SupportsDevice(DeviceType device) const override { return device == DeviceType::HIP; }
};

}  // namespace feather

#endif  // FEATHER_HIP_FP8_LINEAR_H
