// fp8_gemm_e5_fp32.hip -- the FP8 GEMM (fp8_gemm_impl.h) for e5m2 operands and FP32 outputs.
#include "fp8_gemm_impl.h"

int fhip::launch_fp8_gemm_e5_o4(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w,
                                  const Fp8Epilogue& ep) {
    return launch<true, 4>(ctx, a, m, k64, w, ep);
}
