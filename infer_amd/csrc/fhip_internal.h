// fhip_internal.h -- state shared by the runtime and the kernel translation units of libfhip.
#ifndef FHIP_INTERNAL_H
#define FHIP_INTERNAL_H

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fhip.h"

// Persistent per-context device scratch: the argmax block-completion counters, two levels (blocks
// count in per-group counters, the last block of each group counts in `done`) so that no single
// address takes an atomic from every block.  Each counter has its own 128-byte line.  Every kernel
// that uses them leaves them zeroed on exit, so calls and graph replays need no memset.
constexpr int kArgmaxMaxRows = 16;
// Longest LM-head row (K * element size) the argmax kernels take: the m = 1 kernel keeps the activation
// row in LDS beside its weight rings.
constexpr int kArgmaxMaxRowBytes = 65536;
constexpr int kTicketGroups = 32;
struct ArgmaxScratch {
    unsigned int done;
    unsigned int pad[31];
    unsigned int group_done[kTicketGroups][32];  // [g][0] is the counter
};

// Size of the static device array behind fhip_bf16_gemv_argmax_noalloc (ticket counters plus one
// 16-key block of partial keys per workgroup; the C5 head at 2 blocks per CU on 256 CUs needs 72 KiB).
constexpr size_t kNoAllocScratchBytes = size_t(128) << 10;

struct fhip_weight_s;

struct fhip_context_s {
    int device = 0;
    int cus = 256;  // compute units of the device (grid sizing)
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    size_t workspace_limit = SIZE_MAX;
    size_t weight_cache_limit = SIZE_MAX;
    size_t weight_bytes = 0;
    void* workspace = nullptr;
    size_t workspace_size = 0;
    // Workspaces replaced by a larger one while captured graphs were alive: a graph holds the address
    // of the buffer it was captured with, so those buffers are freed only when no graph of this
    // context remains (fhip_graph_destroy) or with the context.
    std::vector<void*> retired_workspaces;
    int live_graphs = 0;
    ArgmaxScratch* scratch = nullptr;
    bool capturing = false;
    std::string last_error;
    const char* last_backend = "";
    std::recursive_mutex mu;
    std::vector<fhip_weight_s*> weights;
};

enum WeightKind { kLinearWeight = 0, kConvWeight = 1 };

struct fhip_weight_s {
    fhip_context ctx = nullptr;
    int refs = 1;
    WeightKind kind = kLinearWeight;
    int dtype = 0;
    int64_t k = 0, n = 0;        // GEMM view: n output channels, k reduction length
    int src_layout = 0;
    const void* src = nullptr;
    uint64_t version = 0;
    // Conv geometry (kind == kConvWeight): n = oc, k = icg*kh*kw
    int64_t icg = 0, kh = 0, kw = 0;
    int32_t group = 1;
    void* data = nullptr;        // prepared layout, see the kernel files
    size_t bytes = 0;
    float* scales = nullptr;     // [n] device (INT8)
    int32_t* zps = nullptr;      // [n] device (INT8)
    int32_t* wsum = nullptr;     // [n] device: sum_k (w - zp_w) per output channel (INT8)
    void* tap_major = nullptr;   // conv (group 1): [OC][KH*KW][IC] copy for the LDS-window kernel
    bool per_channel = false;
    float scale0 = 1.0f;
    int32_t zp0 = 0;
    bool any_zp = false;
    int32_t max_abs_w = 127;     // max |w - zp| over the weight, for the int32 overflow bound
    float max_scale = 1.0f;      // max per-channel scale (finiteness bound of the requantization)
};

namespace fhip {

int set_error(fhip_context ctx, int code, const std::string& msg);
int check_hip(fhip_context ctx, hipError_t err, const char* what);
// Device workspace of at least `bytes`, within the budget (grown only outside capture).
int acquire_workspace(fhip_context ctx, size_t bytes, void** ptr);

// Looks up this device's copy of the no-alloc scratch array (hipGetSymbolAddress), once per device,
// with ctx->device current.  Called by fhip_context_create.
int noalloc_setup(fhip_context ctx);

inline bool valid_scale(float s) { return s > 0.0f && s < __builtin_huge_valf(); }

}  // namespace fhip

#define FHIP_CHECK_LAUNCH(ctx, name)                                                   \
    do {                                                                              \
        hipError_t _e = hipGetLastError();                                            \
        if (_e != hipSuccess) return fhip::check_hip((ctx), _e, name);                \
    } while (0)

#endif  // FHIP_INTERNAL_H
