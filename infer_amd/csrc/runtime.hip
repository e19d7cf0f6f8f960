// runtime.hip -- context, stream, workspace budget, prepared-weight cache and execution capture of
// the MI355X backend (C ABI in include/fhip.h).
//
// Reference counterparts: BackendContext (include/core/backend.h:43-96) and the CUDA runtime it
// adapts (src/kernel/backend.cc:52-187; src/kernel/cuda/runtime.h:39-157, runtime.cu:702-858).
// The weight cache follows the contract of x86 PackedFp8Rhs / prepared_weight_cache.h:26-81 and
// CUDA's packed-weight cache (linear_kernels.cuh:528-567): a prepared copy is keyed by the source
// pointer, dtype, shape, layout and the tensor's mutation version, so a mutated tensor never hits
// a stale copy.
#include "fhip_internal.h"

#include <algorithm>
#include <cstring>

namespace fhip {

int set_error(fhip_context ctx, int code, const std::string& msg) {
    if (ctx) ctx->last_error = msg;
    return code;
}

int check_hip(fhip_context ctx, hipError_t err, const char* what) {
    if (err == hipSuccess) return FHIP_OK;
    return set_error(ctx, FHIP_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

int acquire_workspace(fhip_context ctx, size_t bytes, void** ptr) {
    if (bytes == 0) bytes = 256;
    if (bytes > ctx->workspace_limit) {
        return set_error(ctx, FHIP_ERR_BUDGET, "workspace request " + std::to_string(bytes) +
                                                   " B exceeds the limit " + std::to_string(ctx->workspace_limit));
    }
    if (bytes <= ctx->workspace_size) {
        *ptr = ctx->workspace;
        return FHIP_OK;
    }
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "workspace must grow outside capture; warm up first");
    size_t grown = std::max(bytes, ctx->workspace_size * 2);
    grown = std::min(grown, ctx->workspace_limit);
    grown = (grown + 255) & ~size_t(255);
    if (ctx->workspace) {
        if (ctx->live_graphs > 0) {
            // a captured graph may still replay with this address: keep the buffer until it is destroyed
            ctx->retired_workspaces.push_back(ctx->workspace);
        } else {
            hipError_t e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) return check_hip(ctx, e, "hipStreamSynchronize");
            (void)hipFree(ctx->workspace);
        }
        ctx->workspace = nullptr;
        ctx->workspace_size = 0;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, grown);
    if (e != hipSuccess) return check_hip(ctx, e, "hipMalloc(workspace)");
    ctx->workspace = p;
    ctx->workspace_size = grown;
    *ptr = p;
    return FHIP_OK;
}

}  // namespace fhip

using namespace fhip;

namespace {

struct DeviceGuard {
    int previous = -1;
    explicit DeviceGuard(int device) {
        if (hipGetDevice(&previous) != hipSuccess) previous = -1;
        if (previous != device) (void)hipSetDevice(device);
    }
    ~DeviceGuard() {
        if (previous >= 0) (void)hipSetDevice(previous);
    }
};

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Prepared linear weight: [Np][Kp] row-major, K contiguous, zero padded, Np multiple of 256 and
// Kp multiple of 128 so the GEMM/GEMV kernels load whole 16-byte chunks and whole tiles.
// wsum[n] = sum_k (w - zp_w) (INT8 only) feeds the activation zero-point correction.
__global__ void prepare_linear_weight_kernel(const uint8_t* __restrict__ src, int64_t k, int64_t n, int layout,
                                             int64_t kp, uint8_t* __restrict__ dst) {
    const int64_t row = blockIdx.x;  // output channel (padded range)
    for (int64_t kk = threadIdx.x; kk < kp; kk += blockDim.x) {
        uint8_t v = 0;
        if (row < n && kk < k) v = layout == FHIP_LAYOUT_NK ? src[row * k + kk] : src[kk * n + row];
        dst[row * kp + kk] = v;
    }
}

__global__ void weight_channel_stats_kernel(const int8_t* __restrict__ w, int64_t k, int64_t kp, int64_t n,
                                            const int32_t* __restrict__ zps, int per_channel_zp,
                                            int32_t* __restrict__ wsum, int32_t* __restrict__ max_abs) {
    const int64_t row = blockIdx.x;
    if (row >= n) return;
    const int32_t zp = zps ? zps[per_channel_zp ? row : 0] : 0;
    int64_t s = 0;
    int32_t m = 0;
    for (int64_t kk = threadIdx.x; kk < k; kk += blockDim.x) {
        const int32_t v = (int32_t)w[row * kp + kk] - zp;
        s += v;
        m = max(m, abs(v));
    }
    __shared__ long long ssum[256];
    __shared__ int smax[256];
    ssum[threadIdx.x] = s;
    smax[threadIdx.x] = m;
    __syncthreads();
    for (int off = blockDim.x / 2; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off) {
            ssum[threadIdx.x] += ssum[threadIdx.x + off];
            smax[threadIdx.x] = max(smax[threadIdx.x], smax[threadIdx.x + off]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        wsum[row] = (int32_t)ssum[0];   // |sum| <= k * 255 fits for k < 2^23 (checked on the host)
        atomicMax(max_abs, smax[0]);
    }
}

// Conv weight [OC][IC][KH][KW] -> tap-major [OC][KH*KW][IC] (channels contiguous per tap).
__global__ void conv_tap_major_kernel(const int8_t* __restrict__ src, int64_t ic, int64_t taps,
                                      int8_t* __restrict__ dst) {
    const int64_t oc = blockIdx.x;
    for (int64_t i = threadIdx.x; i < ic * taps; i += blockDim.x) {
        const int64_t t = i / ic, c = i - t * ic;
        dst[(oc * taps + t) * ic + c] = src[(oc * ic + c) * taps + t];
    }
}

void free_weight(fhip_weight w) {
    if (!w) return;
    if (w->tap_major) (void)hipFree(w->tap_major);
    if (w->data) (void)hipFree(w->data);
    if (w->scales) (void)hipFree(w->scales);  // one allocation holds scales, zps, wsum and max|w|
    delete w;
}

fhip_weight find_cached(fhip_context ctx, const void* src, int dtype, int64_t k, int64_t n, int layout, WeightKind kind,
                        uint64_t version) {
    for (fhip_weight w : ctx->weights) {
        if (w->src == src && w->dtype == dtype && w->k == k && w->n == n && w->src_layout == layout &&
            w->kind == kind && w->version == version) {
            return w;
        }
    }
    return nullptr;
}

// Shared tail of the two prepare entry points: budget, allocation, re-layout, statistics.
int prepare_common(fhip_context ctx, fhip_weight w, const void* src, int64_t rows_src_k, int64_t rows_src_n,
                   int layout, const float* scales, int64_t n_scale, const int32_t* zps, int64_t n_zp) {
    const int64_t np = round_up(w->n, 256);
    const int64_t kp = round_up(w->k, 128);
    const size_t data_bytes = (size_t)(np * kp);
    const bool int8 = w->dtype == FHIP_INT8;
    const size_t extra = int8 ? (size_t)np * 12 + 256 : 0;
    if (ctx->weight_bytes + data_bytes + extra > ctx->weight_cache_limit) {
        return set_error(ctx, FHIP_ERR_BUDGET, "prepared weight would exceed the weight cache limit");
    }
    int rc;
    if ((rc = check_hip(ctx, hipMalloc(&w->data, data_bytes), "hipMalloc(weight)")) != FHIP_OK) return rc;
    w->bytes = data_bytes + extra;
    prepare_linear_weight_kernel<<<(unsigned)np, 256, 0, ctx->stream>>>(static_cast<const uint8_t*>(src), rows_src_k,
                                                                        rows_src_n, layout, kp,
                                                                        static_cast<uint8_t*>(w->data));
    FHIP_CHECK_LAUNCH(ctx, "prepare_linear_weight_kernel");
    if (int8) {
        // scales [np] f32, zps [np] i32, wsum [np] i32, max_abs i32
        void* meta = nullptr;
        if ((rc = check_hip(ctx, hipMalloc(&meta, extra), "hipMalloc(weight meta)")) != FHIP_OK) return rc;
        w->scales = static_cast<float*>(meta);
        w->zps = reinterpret_cast<int32_t*>(static_cast<char*>(meta) + np * 4);
        int32_t* wsum = reinterpret_cast<int32_t*>(static_cast<char*>(meta) + np * 8);
        w->wsum = wsum;
        int32_t* max_abs = reinterpret_cast<int32_t*>(static_cast<char*>(meta) + np * 12);
        std::vector<float> hs(np, 1.0f);
        std::vector<int32_t> hz(np, 0);
        for (int64_t i = 0; i < w->n; ++i) {
            hs[i] = scales[n_scale == 1 ? 0 : i];
            hz[i] = zps ? zps[n_zp == 1 ? 0 : i] : 0;
        }
        w->per_channel = n_scale > 1;
        w->max_scale = *std::max_element(hs.begin(), hs.begin() + w->n);
        w->scale0 = scales[0];
        w->zp0 = zps ? zps[0] : 0;
        w->any_zp = std::any_of(hz.begin(), hz.end(), [](int32_t z) { return z != 0; });
        if ((rc = check_hip(ctx, hipMemcpy(w->scales, hs.data(), np * 4, hipMemcpyHostToDevice), "copy scales")) ||
            (rc = check_hip(ctx, hipMemcpy(w->zps, hz.data(), np * 4, hipMemcpyHostToDevice), "copy zps")) ||
            (rc = check_hip(ctx, hipMemsetAsync(wsum, 0, np * 4 + 4, ctx->stream), "clear wsum"))) {
            return rc;
        }
        weight_channel_stats_kernel<<<(unsigned)w->n, 256, 0, ctx->stream>>>(
            static_cast<const int8_t*>(w->data), w->k, kp, w->n, w->zps, 1, wsum, max_abs);
        FHIP_CHECK_LAUNCH(ctx, "weight_channel_stats_kernel");
        int32_t host_max = 0;
        if ((rc = check_hip(ctx, hipMemcpyAsync(&host_max, max_abs, 4, hipMemcpyDeviceToHost, ctx->stream),
                            "read max|w|")) ||
            (rc = check_hip(ctx, hipStreamSynchronize(ctx->stream), "sync prepare"))) {
            return rc;
        }
        w->max_abs_w = host_max;
    } else {
        rc = check_hip(ctx, hipStreamSynchronize(ctx->stream), "sync prepare");
        if (rc) return rc;
    }
    return FHIP_OK;
}

}  // namespace

extern "C" {

int fhip_version(void) { return 1; }

int fhip_context_create(int device, fhip_context* out) {
    if (!out) return FHIP_ERR_INVALID;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return FHIP_ERR_HIP;
    DeviceGuard guard(device);
    auto* ctx = new fhip_context_s();
    ctx->device = device;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        ctx->cus = cus;
    if (hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return FHIP_ERR_HIP;
    }
    ctx->stream = ctx->own_stream;
    if (hipMalloc(reinterpret_cast<void**>(&ctx->scratch), sizeof(ArgmaxScratch)) != hipSuccess ||
        hipMemset(ctx->scratch, 0, sizeof(ArgmaxScratch)) != hipSuccess) {
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return FHIP_ERR_HIP;
    }
    if (fhip::noalloc_setup(ctx) != FHIP_OK) {
        (void)hipFree(ctx->scratch);
        (void)hipStreamDestroy(ctx->own_stream);
        delete ctx;
        return FHIP_ERR_HIP;
    }
    *out = ctx;
    return FHIP_OK;
}

int fhip_context_destroy(fhip_context ctx) {
    if (!ctx) return FHIP_ERR_INVALID;
    DeviceGuard guard(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (fhip_weight w : ctx->weights) free_weight(w);
    ctx->weights.clear();
    if (ctx->workspace) (void)hipFree(ctx->workspace);
    for (void* p : ctx->retired_workspaces) (void)hipFree(p);
    ctx->retired_workspaces.clear();
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return FHIP_OK;
}

int fhip_context_set_stream(fhip_context ctx, void* stream) {
    if (!ctx) return FHIP_ERR_INVALID;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "cannot change the stream during capture");
    hipStream_t next = stream ? static_cast<hipStream_t>(stream) : ctx->own_stream;
    if (next != ctx->stream && ctx->stream) {
        // The argmax tickets, partial keys and workspace belong to the context, not to a stream: work
        // still queued on the old stream must finish before the new stream can reuse them.
        DeviceGuard guard(ctx->device);
        int rc = check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(previous stream)");
        if (rc != FHIP_OK) return rc;
    }
    ctx->stream = next;
    return FHIP_OK;
}

void* fhip_context_stream(fhip_context ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int fhip_set_workspace_limit(fhip_context ctx, size_t bytes) {
    if (!ctx) return FHIP_ERR_INVALID;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    ctx->workspace_limit = bytes;
    return FHIP_OK;
}

int fhip_set_weight_cache_limit(fhip_context ctx, size_t bytes) {
    if (!ctx) return FHIP_ERR_INVALID;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    ctx->weight_cache_limit = bytes;
    return FHIP_OK;
}

int fhip_weight_cache_bytes(fhip_context ctx, size_t* bytes) {
    if (!ctx || !bytes) return FHIP_ERR_INVALID;
    *bytes = ctx->weight_bytes;
    return FHIP_OK;
}

int fhip_synchronize(fhip_context ctx) {
    if (!ctx) return FHIP_ERR_INVALID;
    DeviceGuard guard(ctx->device);
    return check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

int fhip_memory_alloc(fhip_context ctx, size_t bytes, void** out) {
    if (!ctx || !out) return FHIP_ERR_INVALID;
    *out = nullptr;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "memory_alloc during capture");
    if (bytes == 0) return FHIP_OK;
    DeviceGuard guard(ctx->device);
    return check_hip(ctx, hipMalloc(out, bytes), "hipMalloc(tensor)");
}

int fhip_memory_free(fhip_context ctx, void* ptr) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (!ptr) return FHIP_OK;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "memory_free during capture");
    DeviceGuard guard(ctx->device);
    // work still queued on the context's stream may use the allocation
    int rc = check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(before free)");
    if (rc != FHIP_OK) return rc;
    return check_hip(ctx, hipFree(ptr), "hipFree(tensor)");
}

int fhip_memory_upload(fhip_context ctx, void* dst, const void* host, size_t bytes) {
    if (!ctx || (bytes && (!dst || !host))) return FHIP_ERR_INVALID;
    if (bytes == 0) return FHIP_OK;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "memory_upload during capture");
    DeviceGuard guard(ctx->device);
    // ordered after the work already on the stream; the host bytes are consumed before the call returns
    int rc = check_hip(ctx, hipMemcpyAsync(dst, host, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync(H2D)");
    if (rc != FHIP_OK) return rc;
    return check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(upload)");
}

int fhip_memory_download(fhip_context ctx, void* host, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!host || !src))) return FHIP_ERR_INVALID;
    if (bytes == 0) return FHIP_OK;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "memory_download during capture");
    DeviceGuard guard(ctx->device);
    int rc = check_hip(ctx, hipMemcpyAsync(host, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync(D2H)");
    if (rc != FHIP_OK) return rc;
    return check_hip(ctx, hipStreamSynchronize(ctx->stream), "hipStreamSynchronize(download)");
}

int fhip_memory_copy(fhip_context ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return FHIP_ERR_INVALID;
    if (bytes == 0) return FHIP_OK;
    DeviceGuard guard(ctx->device);
    return check_hip(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream), "hipMemcpyAsync(D2D)");
}

const char* fhip_last_error(fhip_context ctx) { return ctx ? ctx->last_error.c_str() : "null context"; }
const char* fhip_last_backend(fhip_context ctx) { return ctx ? ctx->last_backend : ""; }

}  // extern "C"

namespace {

// Argument checks shared by the two linear-weight prepare entry points.
int check_linear_weight_args(fhip_context ctx, const void* src, int dtype, int64_t k, int64_t n, int src_layout,
                             const float* scales, int64_t n_scale, const int32_t* zero_points, int64_t n_zp) {
    if ((k == 0 || n == 0) && src_layout >= FHIP_LAYOUT_KN && src_layout <= FHIP_LAYOUT_NK)
        return set_error(ctx, FHIP_ERR_UNSUPPORTED, "weight_prepare: empty weight (the Common kernel handles it)");
    if (!src || k <= 0 || n <= 0 || (src_layout != FHIP_LAYOUT_KN && src_layout != FHIP_LAYOUT_NK))
        return set_error(ctx, FHIP_ERR_INVALID, "weight_prepare: bad arguments");
    if (dtype != FHIP_FP8E4M3 && dtype != FHIP_FP8E5M2 && dtype != FHIP_INT8)
        return set_error(ctx, FHIP_ERR_UNSUPPORTED, "weight_prepare: dtype must be FP8E4M3, FP8E5M2 or INT8");
    if (k >= (int64_t(1) << 23) || n >= (int64_t(1) << 31))
        return set_error(ctx, FHIP_ERR_UNSUPPORTED, "weight_prepare: k or n too large");
    if (dtype == FHIP_INT8) {
        if (!scales || (n_scale != 1 && n_scale != n) || (zero_points && n_zp != 1 && n_zp != n))
            return set_error(ctx, FHIP_ERR_INVALID, "weight_prepare: INT8 scales/zero points do not match N");
        for (int64_t i = 0; i < n_scale; ++i)
            if (!valid_scale(scales[i])) return set_error(ctx, FHIP_ERR_INVALID, "weight_prepare: invalid scale");
        for (int64_t i = 0; zero_points && i < n_zp; ++i)
            if (zero_points[i] < -128 || zero_points[i] > 127)
                return set_error(ctx, FHIP_ERR_INVALID, "weight_prepare: zero point outside [-128, 127]");
    }
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "weight_prepare during capture");
    return FHIP_OK;
}

// A new prepared weight from device bytes `src`, cached under `key` (the caller's identity of the bytes).
int make_linear_weight(fhip_context ctx, const void* src, const void* key, int dtype, int64_t k, int64_t n,
                       int src_layout, const float* scales, int64_t n_scale, const int32_t* zero_points, int64_t n_zp,
                       uint64_t version, fhip_weight* out) {
    auto* w = new fhip_weight_s();
    w->ctx = ctx;
    w->dtype = dtype;
    w->k = k;
    w->n = n;
    w->src_layout = src_layout;
    w->src = key;
    w->version = version;
    int rc = prepare_common(ctx, w, src, k, n, src_layout, scales, n_scale, zero_points, n_zp);
    if (rc != FHIP_OK) {
        free_weight(w);
        return rc;
    }
    ctx->weight_bytes += w->bytes;
    ctx->weights.push_back(w);
    *out = w;
    return FHIP_OK;
}

}  // namespace

extern "C" {

int fhip_weight_prepare(fhip_context ctx, const void* src, int dtype, int64_t k, int64_t n, int src_layout,
                        const float* scales, int64_t n_scale, const int32_t* zero_points, int64_t n_zp,
                        uint64_t version, fhip_weight* out) {
    if (!ctx || !out) return FHIP_ERR_INVALID;
    *out = nullptr;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    DeviceGuard guard(ctx->device);
    int rc = check_linear_weight_args(ctx, src, dtype, k, n, src_layout, scales, n_scale, zero_points, n_zp);
    if (rc != FHIP_OK) return rc;
    if (fhip_weight hit = find_cached(ctx, src, dtype, k, n, src_layout, kLinearWeight, version)) {
        hit->refs++;
        *out = hit;
        ctx->last_backend = "weight_cache_hit";
        return FHIP_OK;
    }
    rc = make_linear_weight(ctx, src, src, dtype, k, n, src_layout, scales, n_scale, zero_points, n_zp, version, out);
    if (rc == FHIP_OK) ctx->last_backend = "weight_prepare";
    return rc;
}

int fhip_weight_prepare_host(fhip_context ctx, const void* host_src, int dtype, int64_t k, int64_t n, int src_layout,
                             const float* scales, int64_t n_scale, const int32_t* zero_points, int64_t n_zp,
                             uint64_t version, fhip_weight* out) {
    if (!ctx || !out) return FHIP_ERR_INVALID;
    *out = nullptr;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    DeviceGuard guard(ctx->device);
    int rc = check_linear_weight_args(ctx, host_src, dtype, k, n, src_layout, scales, n_scale, zero_points, n_zp);
    if (rc != FHIP_OK) return rc;
    if (fhip_weight hit = find_cached(ctx, host_src, dtype, k, n, src_layout, kLinearWeight, version)) {
        hit->refs++;
        *out = hit;
        ctx->last_backend = "weight_cache_hit";
        return FHIP_OK;
    }
    // Upload into a transient device copy and re-lay it out with the device path; the prepared weight is
    // keyed on the host bytes, and the transient copy is freed before returning.
    const size_t bytes = (size_t)k * (size_t)n;
    void* tmp = nullptr;
    rc = check_hip(ctx, hipMalloc(&tmp, bytes), "hipMalloc(weight upload)");
    if (rc != FHIP_OK) return rc;
    rc = check_hip(ctx, hipMemcpyAsync(tmp, host_src, bytes, hipMemcpyHostToDevice, ctx->stream), "weight upload");
    if (rc == FHIP_OK)
        rc = make_linear_weight(ctx, tmp, host_src, dtype, k, n, src_layout, scales, n_scale, zero_points, n_zp,
                                version, out);
    const int rs = check_hip(ctx, hipStreamSynchronize(ctx->stream), "weight upload sync");
    (void)hipFree(tmp);
    if (rc == FHIP_OK && rs != FHIP_OK) {
        fhip_weight_release(*out);
        *out = nullptr;
        rc = rs;
    }
    if (rc == FHIP_OK) ctx->last_backend = "weight_prepare_host";
    return rc;
}

int fhip_conv_weight_prepare(fhip_context ctx, const int8_t* src, int64_t oc, int64_t icg, int64_t kh, int64_t kw,
                             int32_t group, const float* scales, int64_t n_scale, const int32_t* zero_points,
                             int64_t n_zp, uint64_t version, fhip_weight* out) {
    if (!ctx || !out) return FHIP_ERR_INVALID;
    *out = nullptr;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    DeviceGuard guard(ctx->device);
    if (!src || oc <= 0 || icg <= 0 || kh <= 0 || kw <= 0 || group <= 0 || oc % group != 0 || !scales ||
        (n_scale != 1 && n_scale != oc) || (zero_points && n_zp != 1 && n_zp != oc))
        return set_error(ctx, FHIP_ERR_INVALID, "conv_weight_prepare: bad arguments");
    for (int64_t i = 0; i < n_scale; ++i)
        if (!valid_scale(scales[i])) return set_error(ctx, FHIP_ERR_INVALID, "conv_weight_prepare: invalid scale");
    for (int64_t i = 0; zero_points && i < n_zp; ++i)
        if (zero_points[i] < -128 || zero_points[i] > 127)
            return set_error(ctx, FHIP_ERR_INVALID, "conv_weight_prepare: zero point outside [-128, 127]");
    const int64_t k = icg * kh * kw;
    if (k >= (int64_t(1) << 23)) return set_error(ctx, FHIP_ERR_UNSUPPORTED, "conv_weight_prepare: kernel too large");
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "conv_weight_prepare during capture");
    if (fhip_weight hit = find_cached(ctx, src, FHIP_INT8, k, oc, FHIP_LAYOUT_NK, kConvWeight, version)) {
        if (hit->kh == kh && hit->kw == kw && hit->group == group) {
            hit->refs++;
            *out = hit;
            return FHIP_OK;
        }
    }
    auto* w = new fhip_weight_s();
    w->ctx = ctx;
    w->kind = kConvWeight;
    w->dtype = FHIP_INT8;
    w->k = k;
    w->n = oc;
    w->src_layout = FHIP_LAYOUT_NK;  // [OC][ICg*KH*KW] is already the GEMM [N][K] view
    w->src = src;
    w->version = version;
    w->icg = icg;
    w->kh = kh;
    w->kw = kw;
    w->group = group;
    int rc = prepare_common(ctx, w, src, k, oc, FHIP_LAYOUT_NK, scales, n_scale, zero_points, n_zp);
    if (rc == FHIP_OK && group == 1 && icg % 64 == 0) {
        const size_t bytes = (size_t)(oc * k);
        if (ctx->weight_bytes + w->bytes + bytes <= ctx->weight_cache_limit &&
            (rc = check_hip(ctx, hipMalloc(&w->tap_major, bytes), "hipMalloc(conv tap-major)")) == FHIP_OK) {
            conv_tap_major_kernel<<<(unsigned)oc, 256, 0, ctx->stream>>>(src, icg, kh * kw,
                                                                          static_cast<int8_t*>(w->tap_major));
            rc = check_hip(ctx, hipGetLastError(), "conv_tap_major_kernel");
            if (rc == FHIP_OK) rc = check_hip(ctx, hipStreamSynchronize(ctx->stream), "sync conv prepare");
            w->bytes += bytes;
        }
    }
    if (rc != FHIP_OK) {
        free_weight(w);
        return rc;
    }
    ctx->weight_bytes += w->bytes;
    ctx->weights.push_back(w);
    *out = w;
    return FHIP_OK;
}

int fhip_weight_release(fhip_weight w) {
    if (!w) return FHIP_ERR_INVALID;
    fhip_context ctx = w->ctx;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (--w->refs > 0) return FHIP_OK;
    DeviceGuard guard(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    ctx->weights.erase(std::remove(ctx->weights.begin(), ctx->weights.end(), w), ctx->weights.end());
    ctx->weight_bytes -= w->bytes;
    free_weight(w);
    return FHIP_OK;
}

int fhip_weight_matches(fhip_weight w, const void* src, uint64_t version) {
    return w && w->src == src && w->version == version ? 1 : 0;
}

// ---- execution capture ---------------------------------------------------------------------

// A graph keeps its context's workspace address alive (see retired_workspaces); destroy graphs before
// their context.
struct fhip_graph_s {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int device = 0;
    fhip_context ctx = nullptr;
};

int fhip_capture_begin(fhip_context ctx) {
    if (!ctx) return FHIP_ERR_INVALID;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "capture already active");
    DeviceGuard guard(ctx->device);
    int rc = check_hip(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    if (rc == FHIP_OK) ctx->capturing = true;
    return rc;
}

int fhip_capture_end(fhip_context ctx, fhip_graph* out) {
    if (!ctx || !out) return FHIP_ERR_INVALID;
    std::lock_guard<std::recursive_mutex> lock(ctx->mu);
    if (!ctx->capturing) return set_error(ctx, FHIP_ERR_STATE, "no capture active");
    DeviceGuard guard(ctx->device);
    ctx->capturing = false;
    auto* g = new fhip_graph_s();
    g->device = ctx->device;
    g->ctx = ctx;
    int rc = check_hip(ctx, hipStreamEndCapture(ctx->stream, &g->graph), "hipStreamEndCapture");
    if (rc == FHIP_OK) rc = check_hip(ctx, hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0), "hipGraphInstantiate");
    if (rc != FHIP_OK) {
        if (g->graph) (void)hipGraphDestroy(g->graph);
        delete g;
        return rc;
    }
    ctx->live_graphs++;
    *out = g;
    return FHIP_OK;
}

int fhip_graph_launch(fhip_context ctx, fhip_graph g) {
    if (!ctx || !g) return FHIP_ERR_INVALID;
    DeviceGuard guard(ctx->device);
    return check_hip(ctx, hipGraphLaunch(g->exec, ctx->stream), "hipGraphLaunch");
}

int fhip_graph_destroy(fhip_graph g) {
    if (!g) return FHIP_ERR_INVALID;
    DeviceGuard guard(g->device);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (fhip_context ctx = g->ctx) {
        std::lock_guard<std::recursive_mutex> lock(ctx->mu);
        if (--ctx->live_graphs == 0 && !ctx->retired_workspaces.empty()) {
            (void)hipStreamSynchronize(ctx->stream);
            for (void* p : ctx->retired_workspaces) (void)hipFree(p);
            ctx->retired_workspaces.clear();
        }
    }
    delete g;
    return FHIP_OK;
}

}  // extern "C"
