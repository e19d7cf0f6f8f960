// hip_backend_context.cc -- HipBackendContext: the BackendContext (include/core/backend.h:43-96) of a
// session whose nodes run on DeviceType::HIP.  A session gets it from
// SessionOptions::backend_factory = feather::CreateHipBackendContext (include/core/execution_plan.h:34).
//
// Like CUDA's context (src/kernel/backend.cc:52-187) it keeps activations device-resident between
// nodes and defers host reads to ReadHost; Capture records the run into a HIP graph through
// fhip_capture_begin/end, and ExecutionCapture::Launch replays it on the session's stream.
#include <memory>
#include <stdexcept>
#include <unordered_map>

#include "core/backend.h"
#include "core/shape_utils.h"
#include "hip_runtime.h"

namespace feather {
namespace {

using kernel::hip_detail::ExecutionContextScope;
using kernel::hip_detail::HipExecutionContext;

class HipCapture final : public ExecutionCapture {
 public:
    HipCapture(std::shared_ptr<HipExecutionContext> context, fhip_graph graph)
        : context_(std::move(context)), graph_(graph) {}
    ~HipCapture() override {
        (void)context_->Synchronize();
        (void)fhip_graph_destroy(graph_);
    }
    Status Launch() override {
        ExecutionContextScope scope(context_);
        return fhip_graph_launch(context_->handle(), graph_) == FHIP_OK
                   ? Status::Ok()
                   : Status::Error(StatusCode::kExecutionFailed, "HIP graph launch failed: " + context_->LastError());
    }

 private:
    std::shared_ptr<HipExecutionContext> context_;
    fhip_graph graph_{nullptr};
};

class HipBackendContext final : public BackendContext {
    struct ActiveScope final : Scope {
        explicit ActiveScope(const std::shared_ptr<HipExecutionContext>& context) : scope(context) {}
        ExecutionContextScope scope;
    };

 public:
    explicit HipBackendContext(std::shared_ptr<HipExecutionContext> context) : context_(std::move(context)) {}
    ~HipBackendContext() override { Clear(); }

    BackendCapabilities Capabilities(DeviceType device) const override {
        // device-resident tensors, one stream per session: like CUDA (src/kernel/backend.cc:73-76)
        return device == DeviceType::HIP ? BackendCapabilities{true, false, false, false}
                                         : BackendContext::Capabilities(device);
    }
    std::unique_ptr<Scope> Enter() override { return std::make_unique<ActiveScope>(context_); }
    // Host consumers synchronize explicitly through ReadHost, so execution needs no extra scope.
    std::unique_ptr<Scope> EnterExecution() override { return Enter(); }

    Status Capture(const std::function<Status()>& run, std::unique_ptr<ExecutionCapture>* result) override {
        if (!result || !run) return Status::Error(StatusCode::kInvalidArgument, "invalid capture destination or callback");
        auto scope = Enter();
        if (fhip_capture_begin(context_->handle()) != FHIP_OK)
            return Status::Error(StatusCode::kUnsupported, "HIP capture unavailable: " + context_->LastError());
        Status status;
        try {
            status = run();
        } catch (const std::exception& error) {
            status = Status::Error(StatusCode::kExecutionFailed, error.what());
        }
        fhip_graph graph = nullptr;
        const int ended = fhip_capture_end(context_->handle(), &graph);
        if (!status.ok() || ended != FHIP_OK || graph == nullptr) {
            if (graph != nullptr) (void)fhip_graph_destroy(graph);
            return status.ok() ? Status::Error(StatusCode::kUnsupported, "HIP graph capture failed: " + context_->LastError())
                               : status;
        }
        *result = std::make_unique<HipCapture>(context_, graph);
        return Status::Ok();
    }
    Status Synchronize() override {
        return Result(context_->Synchronize(), "HIP synchronization failed");
    }
    void SetWorkspaceLimit(size_t bytes) override { context_->SetWorkspaceLimit(bytes); }
    void SetFp8WeightCacheLimit(size_t bytes) override { context_->SetWeightCacheLimit(bytes); }
    Status ReadHost(Tensor& tensor) override { return Result(context_->SyncToHost(tensor), "HIP host read failed"); }
    void HostWritten(Tensor& tensor) override { context_->Invalidate(tensor); }
    void MarkPersistent(const Tensor& tensor, bool persistent) override { context_->MarkPersistent(tensor, persistent); }
    bool IsPersistent(const Tensor& tensor) const override { return context_->IsPersistent(tensor); }
    void Release(const Tensor& tensor) override { context_->Release(tensor); }
    void RegisterTensor(std::shared_ptr<Tensor> tensor) override {
        if (tensor) registered_.emplace(tensor.get(), std::move(tensor));
    }
    void Clear() override {
        for (const auto& entry : registered_) context_->Release(*entry.second);
        registered_.clear();
    }
    Status CopyState(Tensor& input, const Tensor& output) override {
        size_t bytes = 0;
        if (!CheckedTensorBytes(input.dims().data(), input.data_type(), &bytes) || input.dims() != output.dims() ||
            input.data_type() != output.data_type())
            return Status::Error(StatusCode::kInvalidArgument, "incompatible state copy");
        return Result(context_->CopyReplica(input, output, bytes), "HIP state copy failed");
    }

 private:
    Status Result(int code, const char* message) const {
        return code == FHIP_OK ? Status::Ok()
                               : Status::Error(StatusCode::kExecutionFailed,
                                               std::string(message) + ": " + context_->LastError());
    }
    std::shared_ptr<HipExecutionContext> context_;
    std::unordered_map<const Tensor*, std::shared_ptr<Tensor>> registered_;
};

}  // namespace

// SessionOptions::backend_factory for HIP sessions.  Throws when no HIP device can be opened, so a
// session is never silently created on a context that cannot run its nodes.
std::unique_ptr<BackendContext> CreateHipBackendContext(int device) {
    auto context = HipExecutionContext::Create(device);
    if (!context) throw std::runtime_error("libfhip: no HIP context on device " + std::to_string(device));
    return std::make_unique<HipBackendContext>(std::move(context));
}

}  // namespace feather
