// hip_runtime.h -- the Feather-side runtime of the `hip` device: one HipExecutionContext per session
// owns a libfhip context (include/fhip.h), the device replicas of the session's tensors and their
// prepared weights.  It is the HIP counterpart of the CUDA execution context
// (src/kernel/cuda/runtime.h:39-157): tensors are identified by Storage id, byte offset and size, and a
// replica is uploaded again only when the host copy's mutation version moved.
//
// Compiled inside the Feather tree (src/kernel/hip/) with FEATHER_WITH_HIP; links libfhip.so.
#ifndef FEATHER_KERNEL_HIP_RUNTIME_H
#define FEATHER_KERNEL_HIP_RUNTIME_H

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>

#include "core/tensor.h"
#include "fhip.h"

namespace feather {
namespace kernel {
namespace hip_detail {

class HipExecutionContext {
 public:
    // A context on HIP device `device`; nullptr when libfhip cannot create one.
    static std::shared_ptr<HipExecutionContext> Create(int device = 0);
    ~HipExecutionContext();
    HipExecutionContext(const HipExecutionContext&) = delete;
    HipExecutionContext& operator=(const HipExecutionContext&) = delete;

    fhip_context handle() const { return ctx_; }
    std::string LastError() const;

    // Device bytes of `tensor` for reading.  The host bytes are uploaded when the replica is missing or
    // older than the tensor's mutation version; a replica written by an earlier HIP node is used as is.
    int AcquireInput(const Tensor& tensor, const void** device);
    // Device bytes for writing `bytes` of `tensor`; the host copy is stale until SyncToHost.
    int AcquireOutput(Tensor& tensor, size_t bytes, void** device);
    // Downloads the replica when the device copy is newer than the host copy (BackendContext::ReadHost).
    int SyncToHost(Tensor& tensor);
    // The host wrote the tensor: its replica no longer holds the current bytes (HostWritten).
    void Invalidate(const Tensor& tensor);
    void Release(const Tensor& tensor);
    void MarkPersistent(const Tensor& tensor, bool persistent);
    bool IsPersistent(const Tensor& tensor) const;
    // Device-to-device copy of one tensor's replica into another's (BackendContext::CopyState).
    int CopyReplica(Tensor& dst, const Tensor& src, size_t bytes);

    // Prepared weights (Prepare(): fhip_weight_prepare / fhip_conv_weight_prepare), cached by the
    // tensor's storage identity, offset, mutation version and preparation (dtype, layout, group).
    int AcquireLinearWeight(const Tensor& w, int dtype, int64_t k, int64_t n, int layout, fhip_weight* out);
    int AcquireConvWeight(const Tensor& w, int32_t group, fhip_weight* out);

    void SetWorkspaceLimit(size_t bytes);
    void SetWeightCacheLimit(size_t bytes);
    int Synchronize();
    void Clear();  // frees every non-persistent replica

 private:
    explicit HipExecutionContext(fhip_context ctx) : ctx_(ctx) {}
    using Key = std::tuple<uint64_t, size_t, size_t>;  // storage id, byte offset, bytes
    struct Replica {
        void* device{nullptr};
        size_t bytes{0};
        uint64_t host_version{0};  // host mutation version the device bytes equal (when !device_newer)
        bool device_newer{false};  // written by a HIP kernel after the last upload/download
        bool persistent{false};
    };
    using WeightKey = std::tuple<uint64_t, size_t, uint64_t, int, int, int64_t>;
    static Key KeyOf(const Tensor& tensor, size_t bytes);
    void ReleaseStaleWeights(const WeightKey& fresh);
    Replica* Find(const Tensor& tensor);
    int Ensure(const Tensor& tensor, size_t bytes, Replica** out);

    fhip_context ctx_{nullptr};
    mutable std::recursive_mutex mu_;
    std::map<Key, Replica> replicas_;
    std::map<WeightKey, fhip_weight> weights_;
};

// Thread-local active context, set by HipBackendContext::Enter()/EnterExecution() for the kernels of
// its session (the role ExecutionContextScope plays for CUDA, runtime.h:44-53).
class ExecutionContextScope {
 public:
    explicit ExecutionContextScope(std::shared_ptr<HipExecutionContext> context);
    ~ExecutionContextScope();
    ExecutionContextScope(const ExecutionContextScope&) = delete;
    ExecutionContextScope& operator=(const ExecutionContextScope&) = delete;

 private:
    std::shared_ptr<HipExecutionContext> previous_;
};

// The context of the calling thread's session, or nullptr outside any HIP session.
std::shared_ptr<HipExecutionContext> CurrentContext();

}  // namespace hip_detail
}  // namespace kernel
}  // namespace feather

#endif  // FEATHER_KERNEL_HIP_RUNTIME_H
