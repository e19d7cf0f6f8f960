// Host check of the Feather-side HIP runtime (integration/hip_runtime.cc): the replica and prepared-weight
// bookkeeping of HipExecutionContext, run against a host stand-in for libfhip's C ABI below (device memory
// is host memory; every call is counted).  Built with the Feather Tensor sources by
// tests/test_integration_compile.py where the Feather tree is present; prints "OK" or the failed check.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <vector>

#include "core/tensor.h"
#include "fhip.h"
#include "hip_runtime.h"

// ---- host stand-in of the C ABI --------------------------------------------------------------------
namespace {
struct Calls {
    int alloc = 0, free = 0, upload = 0, download = 0, copy = 0, prepare = 0, prepare_host = 0, release = 0;
    const void* last_host_src = nullptr;
    uint64_t last_version = 0;
} g;
struct fake_weight {
    int refs = 1;
};
}  // namespace

struct fhip_context_s {
    int device;
};
struct fhip_weight_s : fake_weight {};

extern "C" {
int fhip_context_create(int device, fhip_context* out) {
    *out = new fhip_context_s{device};
    return FHIP_OK;
}
int fhip_context_destroy(fhip_context ctx) {
    delete ctx;
    return FHIP_OK;
}
int fhip_synchronize(fhip_context) { return FHIP_OK; }
const char* fhip_last_error(fhip_context) { return ""; }
int fhip_set_workspace_limit(fhip_context, size_t) { return FHIP_OK; }
int fhip_set_weight_cache_limit(fhip_context, size_t) { return FHIP_OK; }
int fhip_memory_alloc(fhip_context, size_t bytes, void** out) {
    ++g.alloc;
    *out = bytes ? std::malloc(bytes) : nullptr;
    return FHIP_OK;
}
int fhip_memory_free(fhip_context, void* p) {
    if (p) ++g.free;
    std::free(p);
    return FHIP_OK;
}
int fhip_memory_upload(fhip_context, void* dst, const void* host, size_t bytes) {
    ++g.upload;
    std::memcpy(dst, host, bytes);
    return FHIP_OK;
}
int fhip_memory_download(fhip_context, void* host, const void* src, size_t bytes) {
    ++g.download;
    std::memcpy(host, src, bytes);
    return FHIP_OK;
}
int fhip_memory_copy(fhip_context, void* dst, const void* src, size_t bytes) {
    ++g.copy;
    std::memcpy(dst, src, bytes);
    return FHIP_OK;
}
int fhip_weight_prepare(fhip_context, const void*, int, int64_t, int64_t, int, const float*, int64_t, const int32_t*,
                        int64_t, uint64_t version, fhip_weight* out) {
    ++g.prepare;
    g.last_version = version;
    *out = new fhip_weight_s();
    return FHIP_OK;
}
int fhip_weight_prepare_host(fhip_context, const void* host_src, int, int64_t, int64_t, int, const float*, int64_t,
                             const int32_t*, int64_t, uint64_t version, fhip_weight* out) {
    ++g.prepare_host;
    g.last_host_src = host_src;
    g.last_version = version;
    *out = new fhip_weight_s();
    return FHIP_OK;
}
int fhip_conv_weight_prepare(fhip_context, const int8_t*, int64_t, int64_t, int64_t, int64_t, int32_t, const float*,
                             int64_t, const int32_t*, int64_t, uint64_t, fhip_weight* out) {
    ++g.prepare;
    *out = new fhip_weight_s();
    return FHIP_OK;
}
int fhip_weight_release(fhip_weight w) {
    ++g.release;
    delete w;
    return FHIP_OK;
}
}  // extern "C"

// ---- checks ---------------------------------------------------------------------------------------
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            std::printf("FAILED line %d: %s\n", __LINE__, #cond);                \
            return 1;                                                            \
        }                                                                        \
    } while (0)

using feather::DataType;
using feather::Tensor;
using feather::kernel::hip_detail::HipExecutionContext;

static std::shared_ptr<Tensor> make(std::vector<float> v, std::vector<int64_t> shape) {
    auto t = std::make_shared<Tensor>();
    t->Assign<float>(v, shape);
    t->set_data_type(DataType::FP32);
    return t;
}

int main() {
    auto ctx = HipExecutionContext::Create(0);
    CHECK(ctx != nullptr);
    auto x = make({1, 2, 3, 4}, {2, 2});

    // an input is uploaded once per host version
    const void* dx = nullptr;
    CHECK(ctx->AcquireInput(*x, &dx) == FHIP_OK && g.upload == 1 && g.alloc == 1);
    CHECK(std::memcmp(dx, x->raw_data(), 16) == 0);
    CHECK(ctx->AcquireInput(*x, &dx) == FHIP_OK && g.upload == 1);
    x->mutable_data<float>()[0] = 9.0f;  // a host write bumps the mutation version
    CHECK(ctx->AcquireInput(*x, &dx) == FHIP_OK && g.upload == 2 && g.alloc == 1);
    CHECK(static_cast<const float*>(dx)[0] == 9.0f);

    // an output stays on the device until read, then the host holds the kernel's bytes
    auto y = make({0, 0, 0, 0}, {2, 2});
    void* dy = nullptr;
    CHECK(ctx->AcquireOutput(*y, 16, &dy) == FHIP_OK);
    static_cast<float*>(dy)[3] = 7.5f;  // "the kernel writes"
    CHECK(ctx->SyncToHost(*y) == FHIP_OK && g.download == 1);
    CHECK(y->data<float>()[3] == 7.5f);
    CHECK(ctx->SyncToHost(*y) == FHIP_OK && g.download == 1);        // nothing newer on the device
    const void* dy_in = nullptr;
    CHECK(ctx->AcquireInput(*y, &dy_in) == FHIP_OK && g.upload == 2);  // the replica is current: no upload
    CHECK(dy_in == dy);

    // a host write reported through HostWritten is uploaded before the next read
    y->mutable_data<float>()[0] = -1.0f;
    ctx->Invalidate(*y);
    CHECK(ctx->AcquireInput(*y, &dy_in) == FHIP_OK && g.upload == 3 && static_cast<const float*>(dy_in)[0] == -1.0f);

    // device-to-device state copy
    auto z = make({0, 0, 0, 0}, {2, 2});
    CHECK(ctx->CopyReplica(*z, *x, 16) == FHIP_OK && g.copy == 1);
    CHECK(ctx->SyncToHost(*z) == FHIP_OK && z->data<float>()[0] == 9.0f);

    // persistent replicas survive Release and Clear; others are freed
    ctx->MarkPersistent(*x, true);
    CHECK(ctx->IsPersistent(*x));
    const int frees = g.free;
    ctx->Release(*x);
    CHECK(g.free == frees);
    ctx->Release(*y);
    CHECK(g.free == frees + 1);

    // an immutable weight is prepared from its host bytes once; a mutable one from its replica, per version
    auto w = make(std::vector<float>(64, 0.5f), {8, 8});
    w->set_immutable(true);
    fhip_weight h1 = nullptr, h2 = nullptr;
    CHECK(ctx->AcquireLinearWeight(*w, FHIP_FP8E4M3, 8, 8, FHIP_LAYOUT_KN, &h1) == FHIP_OK);
    CHECK(g.prepare_host == 1 && g.last_host_src == w->raw_data() && g.prepare == 0);
    CHECK(ctx->AcquireLinearWeight(*w, FHIP_FP8E4M3, 8, 8, FHIP_LAYOUT_KN, &h2) == FHIP_OK && h1 == h2);
    CHECK(g.prepare_host == 1);
    auto mw = make(std::vector<float>(64, 0.25f), {8, 8});
    fhip_weight m1 = nullptr, m2 = nullptr;
    CHECK(ctx->AcquireLinearWeight(*mw, FHIP_FP8E4M3, 8, 8, FHIP_LAYOUT_NK, &m1) == FHIP_OK && g.prepare == 1);
    const int uploads = g.upload;
    mw->mutable_data<float>()[0] = 3.0f;
    CHECK(ctx->AcquireLinearWeight(*mw, FHIP_FP8E4M3, 8, 8, FHIP_LAYOUT_NK, &m2) == FHIP_OK && g.prepare == 2);
    CHECK(m1 != m2 && g.release == 1 && g.upload == uploads + 1 && g.last_version == mw->mutation_version());

    ctx.reset();  // the context releases the rest
    CHECK(g.release == 3);
    std::printf("OK\n");
    return 0;
}
