// hip_runtime.cc -- HipExecutionContext (hip_runtime.h): tensor replicas and prepared weights of one
// session on top of libfhip's C ABI.
#include "hip_runtime.h"

#include <utility>
#include <vector>

#include "core/shape_utils.h"

namespace feather {
namespace kernel {
namespace hip_detail {
namespace {

thread_local std::shared_ptr<HipExecutionContext> t_current;

size_t TensorBytes(const Tensor& tensor) {
    size_t bytes = 0;
    if (!CheckedTensorBytes(tensor.dims().data(), tensor.data_type(), &bytes)) bytes = tensor.memory_size();
    return bytes;
}

}  // namespace

std::shared_ptr<HipExecutionContext> HipExecutionContext::Create(int device) {
    fhip_context ctx = nullptr;
    if (fhip_context_create(device, &ctx) != FHIP_OK || ctx == nullptr) return nullptr;
    return std::shared_ptr<HipExecutionContext>(new HipExecutionContext(ctx));
}

HipExecutionContext::~HipExecutionContext() {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    (void)fhip_synchronize(ctx_);
    for (auto& entry : weights_) (void)fhip_weight_release(entry.second);
    weights_.clear();
    for (auto& entry : replicas_) (void)fhip_memory_free(ctx_, entry.second.device);
    replicas_.clear();
    (void)fhip_context_destroy(ctx_);
}

std::string HipExecutionContext::LastError() const {
    const char* message = fhip_last_error(ctx_);
    return message ? message : "";
}

HipExecutionContext::Key HipExecutionContext::KeyOf(const Tensor& tensor, size_t bytes) {
    const auto storage = tensor.storage();
    return Key{storage ? storage->id() : 0, tensor.offset(), bytes};
}

HipExecutionContext::Replica* HipExecutionContext::Find(const Tensor& tensor) {
    const auto it = replicas_.find(KeyOf(tensor, TensorBytes(tensor)));
    return it == replicas_.end() ? nullptr : &it->second;
}

int HipExecutionContext::Ensure(const Tensor& tensor, size_t bytes, Replica** out) {
    auto& replica = replicas_[KeyOf(tensor, bytes)];
    if (replica.device == nullptr && bytes != 0) {
        const int rc = fhip_memory_alloc(ctx_, bytes, &replica.device);
        if (rc != FHIP_OK) {
            replicas_.erase(KeyOf(tensor, bytes));
            return rc;
        }
        replica.bytes = bytes;
        replica.host_version = ~uint64_t(0);  // nothing uploaded yet
    }
    *out = &replica;
    return FHIP_OK;
}

int HipExecutionContext::AcquireInput(const Tensor& tensor, const void** device) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    const size_t bytes = TensorBytes(tensor);
    Replica* replica = nullptr;
    int rc = Ensure(tensor, bytes, &replica);
    if (rc != FHIP_OK) return rc;
    if (!replica->device_newer && replica->host_version != tensor.mutation_version()) {
        rc = fhip_memory_upload(ctx_, replica->device, tensor.raw_data(), bytes);
        if (rc != FHIP_OK) return rc;
        replica->host_version = tensor.mutation_version();
    }
    *device = replica->device;
    return FHIP_OK;
}

int HipExecutionContext::AcquireOutput(Tensor& tensor, size_t bytes, void** device) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    Replica* replica = nullptr;
    const int rc = Ensure(tensor, bytes, &replica);
    if (rc != FHIP_OK) return rc;
    replica->device_newer = true;
    *device = replica->device;
    return FHIP_OK;
}

int HipExecutionContext::SyncToHost(Tensor& tensor) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    Replica* replica = Find(tensor);
    if (replica == nullptr || !replica->device_newer) return FHIP_OK;
    // mutable_data keeps copy-on-write and bumps the storage version; the replica equals the new version
    void* host = tensor.mutable_data(tensor.memory_size());
    const int rc = fhip_memory_download(ctx_, host, replica->device, replica->bytes);
    if (rc != FHIP_OK) return rc;
    replica->device_newer = false;
    replica->host_version = tensor.mutation_version();
    return FHIP_OK;
}

void HipExecutionContext::Invalidate(const Tensor& tensor) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    if (Replica* replica = Find(tensor)) {
        replica->device_newer = false;
        replica->host_version = ~uint64_t(0);
    }
}

void HipExecutionContext::Release(const Tensor& tensor) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    const auto it = replicas_.find(KeyOf(tensor, TensorBytes(tensor)));
    if (it == replicas_.end() || it->second.persistent) return;
    (void)fhip_memory_free(ctx_, it->second.device);
    replicas_.erase(it);
}

void HipExecutionContext::MarkPersistent(const Tensor& tensor, bool persistent) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    Replica* replica = nullptr;
    if (Ensure(tensor, TensorBytes(tensor), &replica) == FHIP_OK) replica->persistent = persistent;
}

bool HipExecutionContext::IsPersistent(const Tensor& tensor) const {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    const auto it = replicas_.find(KeyOf(tensor, TensorBytes(tensor)));
    return it != replicas_.end() && it->second.persistent;
}

int HipExecutionContext::CopyReplica(Tensor& dst, const Tensor& src, size_t bytes) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    const void* from = nullptr;
    void* to = nullptr;
    int rc = AcquireInput(src, &from);
    if (rc != FHIP_OK) return rc;
    rc = AcquireOutput(dst, bytes, &to);
    if (rc != FHIP_OK) return rc;
    return fhip_memory_copy(ctx_, to, from, bytes);
}

// A mutated weight gets a new prepared copy under its new version; the copies of its older versions are
// released so a weight updated in place does not accumulate prepared copies.
void HipExecutionContext::ReleaseStaleWeights(const WeightKey& fresh) {
    for (auto it = weights_.begin(); it != weights_.end();) {
        const auto& k = it->first;
        if (std::get<0>(k) == std::get<0>(fresh) && std::get<1>(k) == std::get<1>(fresh) &&
            std::get<3>(k) == std::get<3>(fresh) && std::get<4>(k) == std::get<4>(fresh) &&
            std::get<2>(k) != std::get<2>(fresh)) {
            (void)fhip_weight_release(it->second);
            it = weights_.erase(it);
        } else {
            ++it;
        }
    }
}

int HipExecutionContext::AcquireLinearWeight(const Tensor& w, int dtype, int64_t k, int64_t n, int layout,
                                             fhip_weight* out) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    const auto storage = w.storage();
    const WeightKey key{storage ? storage->id() : 0, w.offset(), w.mutation_version(), dtype, layout, k};
    const auto hit = weights_.find(key);
    if (hit != weights_.end()) {
        *out = hit->second;
        return FHIP_OK;
    }
    // An immutable weight (a WeightStore view of the mmapped model file, src/model/weight_store.cc:77-104) is
    // prepared straight from its host bytes: no raw device replica is kept beside the prepared copy.
    const bool from_host = w.is_immutable();
    const void* device = nullptr;
    int rc = FHIP_OK;
    if (!from_host) {
        rc = AcquireInput(w, &device);
        if (rc != FHIP_OK) return rc;
    }
    const auto& q = w.quantization();
    std::vector<float> scales;
    std::vector<int32_t> zero_points;
    if (dtype == FHIP_INT8) {
        // per-output-channel (or per-tensor) QuantizationParams of the weight, include/util/types.h:56-90
        scales = q.scales.empty() ? std::vector<float>{q.scale_at(0)} : q.scales;
        zero_points = q.zero_points.empty() ? std::vector<int32_t>{q.zero_point_at(0)} : q.zero_points;
    }
    fhip_weight handle = nullptr;
    const float* sp = scales.empty() ? nullptr : scales.data();
    const int32_t* zp = zero_points.empty() ? nullptr : zero_points.data();
    rc = from_host ? fhip_weight_prepare_host(ctx_, w.raw_data(), dtype, k, n, layout, sp, static_cast<int64_t>(scales.size()),
                                              zp, static_cast<int64_t>(zero_points.size()), w.mutation_version(), &handle)
                   : fhip_weight_prepare(ctx_, device, dtype, k, n, layout, sp, static_cast<int64_t>(scales.size()), zp,
                                         static_cast<int64_t>(zero_points.size()), w.mutation_version(), &handle);
    if (rc != FHIP_OK) return rc;
    ReleaseStaleWeights(key);
    weights_[key] = handle;
    *out = handle;
    return FHIP_OK;
}

int HipExecutionContext::AcquireConvWeight(const Tensor& w, int32_t group, fhip_weight* out) {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    const auto& d = w.dims().data();
    if (d.size() != 4) return FHIP_ERR_INVALID;
    const auto storage = w.storage();
    const WeightKey key{storage ? storage->id() : 0, w.offset(), w.mutation_version(), FHIP_INT8, -1 - group, d[1]};
    const auto hit = weights_.find(key);
    if (hit != weights_.end()) {
        *out = hit->second;
        return FHIP_OK;
    }
    const void* device = nullptr;
    int rc = AcquireInput(w, &device);
    if (rc != FHIP_OK) return rc;
    const auto& q = w.quantization();
    const std::vector<float> scales = q.scales.empty() ? std::vector<float>{q.scale_at(0)} : q.scales;
    const std::vector<int32_t> zero_points =
        q.zero_points.empty() ? std::vector<int32_t>{q.zero_point_at(0)} : q.zero_points;
    fhip_weight handle = nullptr;
    rc = fhip_conv_weight_prepare(ctx_, static_cast<const int8_t*>(device), d[0], d[1], d[2], d[3], group,
                                  scales.data(), static_cast<int64_t>(scales.size()), zero_points.data(),
                                  static_cast<int64_t>(zero_points.size()), w.mutation_version(), &handle);
    if (rc != FHIP_OK) return rc;
    ReleaseStaleWeights(key);
    weights_[key] = handle;
    *out = handle;
    return FHIP_OK;
}

void HipExecutionContext::SetWorkspaceLimit(size_t bytes) { (void)fhip_set_workspace_limit(ctx_, bytes); }
void HipExecutionContext::SetWeightCacheLimit(size_t bytes) { (void)fhip_set_weight_cache_limit(ctx_, bytes); }
int HipExecutionContext::Synchronize() { return fhip_synchronize(ctx_); }

void HipExecutionContext::Clear() {
    std::lock_guard<std::recursive_mutex> lock(mu_);
    for (auto it = replicas_.begin(); it != replicas_.end();) {
        if (it->second.persistent) {
            ++it;
            continue;
        }
        (void)fhip_memory_free(ctx_, it->second.device);
        it = replicas_.erase(it);
    }
}

ExecutionContextScope::ExecutionContextScope(std::shared_ptr<HipExecutionContext> context)
    : previous_(t_current) {
    t_current = std::move(context);
}

ExecutionContextScope::~ExecutionContextScope() { t_current = std::move(previous_); }

std::shared_ptr<HipExecutionContext> CurrentContext() { return t_current; }

}  // namespace hip_detail
}  // namespace kernel
}  // namespace feather
