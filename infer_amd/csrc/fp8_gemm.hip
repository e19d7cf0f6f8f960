// fp8_gemm.hip -- FP8 (e4m3 / e5m2) prefill GEMM on gfx950 MFMA: entry from fhip_fp8_linear.
//
// The kernel and its tile choice are in fp8_gemm_impl.h; fp8_gemm_<fmt>_<out>.hip instantiate them per
// (FP8 format, output width).  This file picks the instantiation and splits activations too large for the
// kernel's 32-bit offsets into row blocks.
#include "fp8_common.h"

namespace {

int launch(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w,
           const fhip::Fp8Epilogue& ep) {
    const int ob = ep.out_dtype == FHIP_FP32 ? 4 : (ep.out_dtype == FHIP_BF16 ? 2 : 1);
    if (ep.e5) {
        if (ob == 1) return fhip::launch_fp8_gemm_e5_o1(ctx, a, m, k64, w, ep);
        if (ob == 2) return fhip::launch_fp8_gemm_e5_o2(ctx, a, m, k64, w, ep);
        return fhip::launch_fp8_gemm_e5_o4(ctx, a, m, k64, w, ep);
    }
    if (ob == 1) return fhip::launch_fp8_gemm_e4_o1(ctx, a, m, k64, w, ep);
    if (ob == 2) return fhip::launch_fp8_gemm_e4_o2(ctx, a, m, k64, w, ep);
    return fhip::launch_fp8_gemm_e4_o4(ctx, a, m, k64, w, ep);
}

}  // namespace

int fhip::launch_fp8_gemm(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w,
                          const Fp8Epilogue& ep) {
    // The kernel addresses the activations with 32-bit offsets (buffer resources), so activations of
    // 2^31 bytes or more run as several launches over row blocks (multiples of 256 rows).
    const int64_t limit = (int64_t(1) << 31) - 1;
    const int64_t max_rows = limit / k64 / 256 * 256;
    if (m * k64 <= limit || max_rows == 0)
        return launch(ctx, a, m, k64, w, ep);
    const int64_t out_bytes = ep.out_dtype == FHIP_FP32 ? 4 : (ep.out_dtype == FHIP_BF16 ? 2 : 1);
    for (int64_t r0 = 0; r0 < m; r0 += max_rows) {
        Fp8Epilogue e = ep;
        e.out = static_cast<uint8_t*>(ep.out) + r0 * ep.n * out_bytes;
        if (ep.bias_kind == FHIP_BIAS_MATRIX) e.bias = ep.bias + r0 * ep.n;
        const int64_t rows = m - r0 < max_rows ? m - r0 : max_rows;
        const int rc = launch(ctx, a + r0 * k64, rows, k64, w, e);
        if (rc != FHIP_OK) return rc;
    }
    return FHIP_OK;
}
