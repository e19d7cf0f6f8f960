// wave.h -- wave64 reductions on CDNA registers (no LDS traffic).
//
// Within each 16-lane row four DPP steps (quad xor 1, quad xor 2, half-row mirror, row mirror)
// leave the row's sum in every lane of the row; the four row sums are then read with readlane into
// scalar registers.  The result is wave-uniform.
#ifndef FHIP_WAVE_H
#define FHIP_WAVE_H

#include <hip/hip_runtime.h>

namespace fhip {

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum of v over the 64 lanes, identical in every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

}  // namespace fhip

#endif  // FHIP_WAVE_H
