// i8_gemm_tile.hip -- the INT8 linear for large M on the MFMA tile GEMM of fp8_gemm_impl.h (its I8 mode:
// v_mfma_i32_32x32x32_i8, int32 accumulators, I8Epilogue requantization in the epilogue).
#include "fp8_gemm_impl.h"

namespace {

template <int OB>
int launch_i8(fhip_context ctx, const uint8_t* a, int64_t m, const fhip_weight_s* w, const I8Epilogue& iep) {
    Fp8Epilogue ep{};  // the tile kernel's final store reads only out and n from it
    ep.bias_kind = FHIP_BIAS_NONE;
    ep.out = iep.out_any;
    ep.n = w->n;
    const int64_t n = w->n, k = w->k;
    const bool big = ((m + 255) / 256) * ((n + 255) / 256) >= 192 && OB != 4;
    if (k % 128 == 0) {
        // N a multiple of 224 (Qwen's 3584 = 16 x 224): 256x224 tiles (two wave columns of 128 and 96), so the
        // tile count is a multiple of 16 rather than 14
        if (big && n % 224 == 0)
            return launch_tile<false, OB, 256, 224, 4, 2, 128, 2, 96, true>(ctx, a, m, k, w, ep,
                                                                           "i8_mfma_gemm_256x224_bk128_w8", &iep);
        if (big)
            return launch_tile<false, OB, 256, 256, 4, 2, 128, 2, 0, true>(ctx, a, m, k, w, ep,
                                                                          "i8_mfma_gemm_256x256_bk128_w8", &iep);
        return launch_tile<false, OB, 128, 128, 2, 4, 128, 4, 0, true>(ctx, a, m, k, w, ep,
                                                                      "i8_mfma_gemm_128x128_bk128_w8", &iep);
    }
    if (big) return launch_tile<false, OB, 256, 256, 4, 2, 64, 4, 0, true>(ctx, a, m, k, w, ep, "i8_mfma_gemm_256x256_w8", &iep);
    return launch_tile<false, OB, 128, 128, 2, 4, 64, 4, 0, true>(ctx, a, m, k, w, ep, "i8_mfma_gemm_128x128_w8", &iep);
}

}  // namespace

int fhip::launch_i8_gemm_tile(fhip_context ctx, const int8_t* a, int64_t m, const fhip_weight_s* w,
                              const I8Epilogue& ep) {
    const uint8_t* a8 = reinterpret_cast<const uint8_t*>(a);
    if (ep.out_dtype == FHIP_INT8) return launch_i8<1>(ctx, a8, m, w, ep);
    if (ep.out_dtype == FHIP_FP32) return launch_i8<4>(ctx, a8, m, w, ep);
    return launch_i8<2>(ctx, a8, m, w, ep);
}
