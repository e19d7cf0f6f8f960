// bench_ceilings.hip -- measured hardware ceilings that bench.py reports beside the published MI355X peaks.
//
// Not part of the operator library (libfhip.so) and not called by it: a separate diagnostic library,
// bench_ceilings.so (built beside bench.py by __graft_entry__.build()), that bench.py loads to put the FP8 GEMM's roofline fraction in context.
//   * fhipc_mfma_fp8_rate: sustained v_mfma_scale_f32_32x32x64_f8f6f4 rate on every CU when the operand
//     registers hold given FP8 codes (bench.py passes the C3 activation codes).  MFMA power, and with
//     it the clock the chip sustains, depends on the operand bits: all-zero operands run faster than
//     realistic ones.
//   * fhipc_l2_stream: L2 -> LDS streaming rate of buffer_load ... lds over an L2-resident buffer, the
//     path the FP8 GEMM stages its operands through.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr;

constexpr int kThreads = 512;

template <bool E5>
__global__ __launch_bounds__(kThreads) void mfma_rate_kernel(const uint8_t* __restrict__ codes, int n_codes, int iters,
                                                             float* __restrict__ sink) {
    // each lane takes two 32-byte operand slices from the code buffer (wrapping), as a GEMM lane would
    const int t = blockIdx.x * kThreads + threadIdx.x;
    const int64_t oa = ((int64_t)t * 64) % (n_codes - 64 + 1);
    const int64_t ob = ((int64_t)t * 64 + 32) % (n_codes - 64 + 1);
    v8i a, b;
    for (int i = 0; i < 8; ++i) {
        a[i] = *reinterpret_cast<const int*>(codes + (oa & ~int64_t(3)) + 4 * i);
        b[i] = *reinterpret_cast<const int*>(codes + (ob & ~int64_t(3)) + 4 * i);
    }
    constexpr int fmt = E5 ? 1 : 0;
    v16f c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c0, fmt, fmt, 0, 127, 0, 127);
        c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c1, fmt, fmt, 0, 127, 0, 127);
        c2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, a, c2, fmt, fmt, 0, 127, 0, 127);
        c3 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, b, c3, fmt, fmt, 0, 127, 0, 127);
    }
    float s = 0.0f;
    for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
    if (threadIdx.x == 0) sink[blockIdx.x] = s;  // keeps the MFMAs live
}

__global__ __launch_bounds__(kThreads) void l2_stream_kernel(const uint8_t* __restrict__ src, int bytes, int iters) {
    extern __shared__ __align__(16) uint8_t sm[];
    const int tid = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)src, 0, bytes, 0x00020000);
    constexpr int kPass = kThreads * 16 * 8;  // 64 KB per pass: 8 loads of 16 bytes per thread
    int off = (int)(((int64_t)blockIdx.x * 7919 * 1024) % bytes) & ~(kPass - 1);
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int r = 0; r < 8; ++r)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(sm + (r * kThreads + (tid & ~63)) * 16), 16,
                                                     off + (r * kThreads + tid) * 16, 0, 0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        off += kPass;
        if (off >= bytes) off = 0;
    }
}

int cu_count(int* cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -3;
    return hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? 0 : -3;
}

// Times `launch` (enqueued on `s`) with events; one untimed launch first.
template <typename F>
int time_launch(hipStream_t s, F&& launch, float* ms) {
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess) return -3;
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return -3;
    }
    launch();
    int rc = hipEventRecord(e0, s) == hipSuccess ? 0 : -3;
    if (rc == 0) launch();
    if (rc == 0 && hipEventRecord(e1, s) != hipSuccess) rc = -3;
    if (rc == 0 && hipEventSynchronize(e1) != hipSuccess) rc = -3;
    if (rc == 0 && hipGetLastError() != hipSuccess) rc = -3;
    if (rc == 0 && hipEventElapsedTime(ms, e0, e1) != hipSuccess) rc = -3;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

}  // namespace

extern "C" {

// Sustained FP8 MFMA rate (TFLOP/s) of one 512-thread block per CU running `iters` x 4 independent
// 32x32x64 MFMAs whose operands are taken from `codes` (device memory, n_codes >= 64 bytes).
int fhipc_mfma_fp8_rate(const uint8_t* codes, int64_t n_codes, int e5, int iters, float* tflops) {
    if (!codes || n_codes < 64 || n_codes > (int64_t(1) << 30) || iters <= 0 || !tflops) return -1;
    int cus = 0;
    if (cu_count(&cus) != 0) return -3;
    float* sink = nullptr;
    if (hipMalloc(&sink, sizeof(float) * cus) != hipSuccess) return -3;
    hipStream_t s = nullptr;
    float ms = 0.0f;
    const int rc = time_launch(s, [&] {
        if (e5) mfma_rate_kernel<true><<<cus, kThreads, 0, s>>>(codes, (int)n_codes, iters, sink);
        else mfma_rate_kernel<false><<<cus, kThreads, 0, s>>>(codes, (int)n_codes, iters, sink);
    }, &ms);
    (void)hipFree(sink);
    if (rc != 0 || ms <= 0.0f) return rc ? rc : -3;
    const double flop = (double)cus * (kThreads / 64) * iters * 4 * (2.0 * 32 * 32 * 64);
    *tflops = (float)(flop / (ms * 1e-3) / 1e12);
    return 0;
}

// L2 -> LDS streaming rate (TB/s, all CUs, one 512-thread block per CU) of 16-byte buffer_load ... lds
// over `buf` (device memory of `bytes` bytes, a multiple of 64 KB, small enough to stay L2-resident).
int fhipc_l2_stream(const uint8_t* buf, int64_t bytes, int iters, float* tbs) {
    if (!buf || bytes < 65536 || bytes % 65536 != 0 || bytes > (int64_t(1) << 30) || iters <= 0 || !tbs) return -1;
    int cus = 0;
    if (cu_count(&cus) != 0) return -3;
    hipStream_t s = nullptr;
    float ms = 0.0f;
    const int rc = time_launch(s, [&] { l2_stream_kernel<<<cus, kThreads, 65536, s>>>(buf, (int)bytes, iters); }, &ms);
    if (rc != 0 || ms <= 0.0f) return rc ? rc : -3;
    *tbs = (float)((double)cus * iters * 65536 / (ms * 1e-3) / 1e12);
    return 0;
}

}  // extern "C"
