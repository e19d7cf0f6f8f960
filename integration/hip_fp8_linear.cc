// hip_fp8_linear.cc -- HipFp8LinearOp, its operator builder, and HipFp8LinearFusionPass
// (hip_fp8_linear.h).
#include "hip_fp8_linear.h"

#include <cmath>
#include <utility>

#include "core/operator_registry.h"
#include "core/shape_utils.h"
#include "core/static_graph.h"

namespace feather {
namespace kernel {
void EnsureHipKernelsRegistered();
}

namespace operators {
namespace {

bool FloatAttribute(const model::NodeDesc& node, const std::string& key, float* value) {
    const auto it = node.attributes.find(key);
    if (it == node.attributes.end()) return false;
    const auto* v = std::get_if<float>(&it->second);
    if (v == nullptr) return false;
    *value = *v;
    return true;
}

// Builder of the "HipFp8Linear" node: inputs {a (BF16), w (FP8)}, output {out (BF16)}, float attributes
// input_scale and output_scale.  Follows the QwenGemmArgmax builder (src/operator/qwen_gemm_argmax_op.cc:28-62).
std::shared_ptr<OpBase> BuildHipFp8LinearOp(const model::NodeDesc& node, OperatorRegistry::TensorMap& tensors,
                                            const OperatorRegistry::BuildContext& context) {
    if (node.inputs.size() != 2 || node.outputs.size() != 1) return nullptr;
    HipFp8LinearParam param;
    param.a = tensors[node.inputs[0]];
    param.w = tensors[node.inputs[1]];
    param.out = tensors[node.outputs[0]];
    if (!FloatAttribute(node, "input_scale", &param.input_scale) ||
        !FloatAttribute(node, "output_scale", &param.output_scale))
        return nullptr;
    if (param.a == nullptr || param.w == nullptr || param.out == nullptr) return nullptr;
    auto op = std::make_shared<HipFp8LinearOp>(node.name.empty() ? kHipFp8LinearOp : node.name, param);
    if (op->CheckShape() != 0 || op->InferOutputShapes() != 0) return nullptr;
    kernel::EnsureHipKernelsRegistered();
    auto kernel = CreateKernelForTensor(context.device, kHipFp8LinearOp, {param.a}, DataType::BF16);
    if (kernel == nullptr) return nullptr;
    op->AttachKernel(std::move(kernel));
    return op;
}

bool g_registered = [] {
    OperatorRegistry::instance().Register(kHipFp8LinearOp, BuildHipFp8LinearOp);
    return true;
}();

bool ValidScale(float s) { return std::isfinite(s) && s > 0.0f; }

}  // namespace

void EnsureHipFp8LinearOperatorRegistered() { (void)g_registered; }

HipFp8LinearOp::HipFp8LinearOp(std::string name, const HipFp8LinearParam& param)
    : OpBase(std::move(name), kHipFp8LinearOp), param_(param) {
    SyncIO();
}

void HipFp8LinearOp::SyncIO() {
    SetInputs({param_.a, param_.w});
    SetOutputs({param_.out});
}

int32_t HipFp8LinearOp::CheckShape() const {
    if (!param_.a || !param_.w || !param_.out || !param_.a->IsInitialized() || !param_.w->IsInitialized() ||
        param_.a->data_type() != DataType::BF16 ||
        (param_.w->data_type() != DataType::FP8E4M3 && param_.w->data_type() != DataType::FP8E5M2) ||
        param_.w->dims().size() != 2 || param_.a->dims().empty() ||
        param_.a->dims().data().back() != param_.w->dims()[0] || !ValidScale(param_.input_scale) ||
        !ValidScale(param_.output_scale) || !HasCompatiblePerTensorQuantization(param_.w->quantization()))
        return -1;
    return 0;
}

int32_t HipFp8LinearOp::InferOutputShapes() {
    if (CheckShape() != 0) return -1;
    auto dims = param_.a->dims().data();
    dims.back() = param_.w->dims()[1];
    size_t bytes = 0;
    if (!CheckedTensorBytes(dims, DataType::BF16, &bytes)) return -1;
    if (!param_.out->IsInitialized() || param_.out->memory_size() < bytes) param_.out = std::make_shared<Tensor>(bytes);
    param_.out->Resize(dims);
    param_.out->set_data_type(DataType::BF16);
    SyncIO();
    return 0;
}

void HipFp8LinearOp::AttachKernel(std::unique_ptr<KernelBase> kernel) {
    kernel_ = std::move(kernel);
    if (kernel_ != nullptr) kernel_->SetParamOwner(std::make_shared<HipFp8LinearParam>(param_));
}

int32_t HipFp8LinearOp::Run() { return InferOutputShapes() == 0 && kernel_ != nullptr ? kernel_->compute() : -1; }

}  // namespace operators

namespace {

const std::string kPassName = "HipFp8LinearFusionPass";

bool IsFp8(DataType dtype) { return dtype == DataType::FP8E4M3 || dtype == DataType::FP8E5M2; }
bool ValidScale(float s) { return std::isfinite(s) && s > 0.0f; }

// `value` is produced by `node` and read by exactly one node, `user`, and is not a graph output.
bool SoleEdge(const StaticGraph& graph, const std::string& value, const std::string& user) {
    const auto users = graph.GetUsers(value);
    return !graph.IsGraphOutputValue(value) && users.size() == 1 && users[0] == user;
}

struct Chain {
    const StaticNode* first_cast{nullptr};
    const StaticNode* matmul{nullptr};
    float input_scale{1.0f};
    float output_scale{1.0f};
};

// `last` is Cast(fp8 -> bf16) fed by MatMul(x8, W) fed by Cast(bf16 -> fp8).
bool MatchChain(const StaticGraph& graph, const StaticNode& last, Chain* chain) {
    if (last.removed || last.op_type != "Cast" || last.inputs.size() != 1 || last.outputs.size() != 1) return false;
    const auto* matmul = graph.GetNode(graph.GetProducer(last.inputs[0]));
    if (matmul == nullptr || matmul->removed || matmul->op_type != "MatMul" || matmul->inputs.size() != 2 ||
        matmul->outputs.size() != 1 || !SoleEdge(graph, last.inputs[0], last.name))
        return false;
    const auto* first = graph.GetNode(graph.GetProducer(matmul->inputs[0]));
    if (first == nullptr || first->removed || first->op_type != "Cast" || first->inputs.size() != 1 ||
        first->outputs.size() != 1 || !SoleEdge(graph, matmul->inputs[0], matmul->name))
        return false;
    const auto x = graph.GetTensor(first->inputs[0]);
    const auto x8 = graph.GetTensor(first->outputs[0]);
    const auto w = graph.GetTensor(matmul->inputs[1]);
    const auto y8 = graph.GetTensor(matmul->outputs[0]);
    const auto y = graph.GetTensor(last.outputs[0]);
    if (!x || !x8 || !w || !y8 || !y || x->data_type() != DataType::BF16 || y->data_type() != DataType::BF16 ||
        !IsFp8(x8->data_type()) || x8->data_type() != w->data_type() || y8->data_type() != w->data_type() ||
        w->dims().size() != 2 || !w->is_immutable() || !HasCompatiblePerTensorQuantization(x8->quantization()) ||
        !HasCompatiblePerTensorQuantization(w->quantization()) ||
        !HasCompatiblePerTensorQuantization(y8->quantization()) || !ValidScale(x8->quantization_scale()) ||
        !ValidScale(y8->quantization_scale()))
        return false;
    chain->first_cast = first;
    chain->matmul = matmul;
    chain->input_scale = x8->quantization_scale();
    chain->output_scale = y8->quantization_scale();
    return true;
}

}  // namespace

const std::string& HipFp8LinearFusionPass::name() const { return kPassName; }

int32_t HipFp8LinearFusionPass::Run(StaticGraph* graph) {
    if (graph == nullptr) return -1;
    if (graph->KernelDevice() != DeviceType::HIP) return 0;
    operators::EnsureHipFp8LinearOperatorRegistered();
    for (const auto& node : graph->nodes()) {
        Chain chain;
        if (!MatchChain(*graph, node, &chain)) continue;
        model::NodeDesc replacement;
        replacement.name = node.name;
        replacement.op_type = operators::kHipFp8LinearOp;
        replacement.inputs = {chain.first_cast->inputs[0], chain.matmul->inputs[1]};
        replacement.outputs = node.outputs;
        replacement.attributes["input_scale"] = chain.input_scale;
        replacement.attributes["output_scale"] = chain.output_scale;
        const std::string matmul = chain.matmul->name, first = chain.first_cast->name;
        if (!graph->ReplaceNodeDesc(replacement) || !graph->RemoveNode(matmul) || !graph->RemoveNode(first)) return -1;
    }
    return 0;
}

}  // namespace feather
