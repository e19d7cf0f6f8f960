// fp8_gemm_e4_bf16.hip -- the FP8 GEMM (fp8_gemm_impl.h) for e4m3 operands and BF16 outputs.
#include "fp8_gemm_impl.h"

int fhip::launch_fp8_gemm_e4_o2(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w,
                                  const Fp8Epilogue& ep) {
    return launch<false, 2>(ctx, a, m, k64, w, ep);
}
