// fp8_linear.hip -- FP8 (e4m3 / e5m2) linear of the Qwen FP8 export on gfx950, and the Cast kernel.
//
// Semantics (per output element), following src/kernel/common/matmul.cc:56-130, gemm.cc:62-100,
// fc.cc:48-73 and kernel_io.h:58-78:
//     y   = alpha * sum_k (Dec(a)*a_scale) * (Dec(w)*w_scale)  [+ beta * Dec(bias)*bias_scale]
//     out = Enc(y / out_scale)                                   (FP8 code)
// fp32 accumulation.  The products Dec(a)*Dec(w) are exact in fp32, so the kernels accumulate the
// unscaled products and apply a_scale*w_scale once; the result differs from the reference's
// K-ordered fp32 sum only by accumulation order (<= 1 FP8 code after the output encode).
//
// Two paths:
//   * fp8_gemv1_kernel  -- one decode row with power-of-two scales (the fused Cast -> MatMul -> Cast):
//                          bandwidth-bound; weight rows stream with 16-byte loads, products accumulate
//                          on the VALU, a cross-lane butterfly reduces.
//   * fp8_gemv_mfma_kernel -- any m <= 16: weight columns straight from HBM as MFMA B operands,
//                          activations staged once per block in LDS as FP8 codes.
//   * fp8_gemm_kernel (fp8_gemm.hip) -- prefill (m > 16): MFMA, fp32 accumulation.
// Weights come prepared as [Np][Kp] (K contiguous, zero padded; runtime.hip).
#include "fp8_common.h"

#include <cmath>
#include "codec.h"
#include "wave.h"

using namespace fhip;

namespace {

// Activation staging: the block encodes its activation rows once into LDS as FP8 codes.  Every
// thread takes groups of 4 elements (one 4/8/16-byte load for FP8/BF16/FP32) and issues all of its
// loads before encoding any, so the staging costs one memory latency and a short encode chain.
// `a_vec` = 1 when k % 4 == 0 and the rows are 16-byte aligned; otherwise a per-element path runs.
// Scales: `inv` holds 1/s when s is a power of two (x * (1/s) is then exactly x / s, both being the
// correctly rounded value of the same real number); otherwise inv = 0 and the kernel divides.
__device__ __forceinline__ float scale_down(float x, float s, float inv) { return inv != 0.0f ? x * inv : x / s; }

template <bool E5, int ADT>
__device__ __forceinline__ uint8_t encode_act(uint32_t bits, float a_scale, float a_inv) {
    const float x = ADT == 1 ? fhip::bits_f32(bits << 16) : fhip::bits_f32(bits);
    return fhip::fp8_encode(scale_down(x, a_scale, a_inv), E5);
}

// `after_first_loads` runs once, right after the first batch of activation loads is issued: the caller
// issues its weight stream there, so the (in-order) wait for the activations does not also wait for it.
template <bool E5, int ADT, int MT, class F>
__device__ __forceinline__ void stage_activations(const void* __restrict__ a, int a_vec, float a_scale, float a_inv,
                                                  int64_t m, int64_t k, int64_t kp, int mt, uint8_t* xs, int tid,
                                                  F&& after_first_loads) {
    bool first = true;
    constexpr int kBatch = MT == 1 ? 1 : (MT <= 4 ? 4 : 16);  // MT rows of up to 1024 codes: one batch
    constexpr int esz = ADT == 0 ? 1 : (ADT == 1 ? 2 : 4);
    const int64_t groups = (int64_t)mt * kp / 4;
    const int64_t gpr = kp / 4;  // groups per row
    if (a_vec) {
        for (int64_t g0 = tid; g0 < groups; g0 += (int64_t)kGemvThreads * kBatch) {
            uint32_t raw[kBatch][4];
            // Loads are unconditional (out-of-range groups read element 0 and are masked afterwards), so
            // the batch issues back to back and costs one memory round trip.
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int64_t g = g0 + (int64_t)u * kGemvThreads;
                const int64_t r = g / gpr, kk = (g - r * gpr) * 4;
                const bool live = g < groups && r < m && kk < k;
                const uint8_t* src = static_cast<const uint8_t*>(a) + (live ? (r * k + kk) * esz : 0);
                uint32_t v4[4];
                if constexpr (ADT == 0) {
                    v4[0] = *reinterpret_cast<const uint32_t*>(src);
                    v4[1] = v4[2] = v4[3] = 0u;
                } else if constexpr (ADT == 1) {
                    const uint2 v = *reinterpret_cast<const uint2*>(src);
                    v4[0] = v.x & 0xffffu;
                    v4[1] = v.x >> 16;
                    v4[2] = v.y & 0xffffu;
                    v4[3] = v.y >> 16;
                } else {
                    const uint4 v = *reinterpret_cast<const uint4*>(src);
                    v4[0] = v.x;
                    v4[1] = v.y;
                    v4[2] = v.z;
                    v4[3] = v.w;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) raw[u][i] = live ? v4[i] : 0u;
            }
            if (first) {
                after_first_loads();
                first = false;
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int64_t g = g0 + (int64_t)u * kGemvThreads;
                if (g >= groups) continue;
                uint32_t c;
                if constexpr (ADT == 0) {
                    c = raw[u][0];
                } else {
                    float q[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        q[i] = scale_down(ADT == 1 ? fhip::bits_f32(raw[u][i] << 16) : fhip::bits_f32(raw[u][i]),
                                          a_scale, a_inv);
                    c = encode4<E5>(q);
                }
                *reinterpret_cast<uint32_t*>(xs + g * 4) = c;
            }
        }
        // a thread with no activation group (mt * kp / 4 < threads) still issues its first weight batch
        if (first) after_first_loads();
    } else {
        after_first_loads();
        for (int64_t idx = tid; idx < (int64_t)mt * kp; idx += kGemvThreads) {
            const int64_t r = idx / kp, kk = idx - r * kp;
            uint8_t code = 0;
            if (r < m && kk < k) {
                const int64_t e = r * k + kk;
                if constexpr (ADT == 0) code = static_cast<const uint8_t*>(a)[e];
                else if constexpr (ADT == 1) code = encode_act<E5, 1>(static_cast<const uint16_t*>(a)[e], a_scale, a_inv);
                else code = encode_act<E5, 2>(fhip::f32_bits(static_cast<const float*>(a)[e]), a_scale, a_inv);
            }
            xs[idx] = code;
        }
    }
}

// ---- Decode GEMV on MFMA (any m <= 16) -----------------------------------------------------------
// A block owns 16 output columns; its 4 waves split K (wave w takes the 128-deep steps w, w+4, ...).
// v_mfma_scale_f32_16x16x128_f8f6f4 with unit scales multiplies the activation rows (A, staged as FP8
// codes in LDS, rows >= m zero) by the weight columns (B, straight from HBM into registers): no
// per-element decode, and the MFMA does the K reduction inside each step.  Lane l supplies row/column
// l%16 and the 32-byte K slice l/16 of the step, for A and B alike.  The four partial 16x16 tiles are
// summed through LDS and every thread finishes one output.  The first batch of weight loads is issued
// right after the activation loads, so the weight stream and the staging overlap.
constexpr int kGemvUnroll = 4;  // steps per wave whose weight loads are in flight together

template <bool E5, int ADT, int MT>
__global__ __launch_bounds__(kGemvThreads) void fp8_gemv_mfma_kernel(const void* __restrict__ a, int a_vec,
                                                                      float a_scale, float a_inv, int64_t m, int64_t k,
                                                                      const uint8_t* __restrict__ w, int64_t kp,
                                                                      int64_t n, Fp8Epilogue ep) {
    extern __shared__ __align__(16) uint8_t xs[];  // [m][kp] FP8 codes
    __shared__ float red[4][16][17];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t col0 = (int64_t)blockIdx.x * 16;
    const int steps = (int)(kp / 128);
    const int fr = lane & 15;
    const int fq = lane >> 4;
    const uint8_t* wcol = w + (col0 + fr) * kp + fq * 32;  // rows past n: zero padding of the prepared weight
    uint4 wb[kGemvUnroll][2];
    auto load_batch = [&](int s0) {
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            const int s = s0 + 4 * u;
            const uint8_t* p = wcol + (int64_t)(s < steps ? s : steps - 1) * 128;  // clamped: unconditional
            wb[u][0] = load_stream16(p);
            wb[u][1] = load_stream16(p + 16);
        }
    };
    stage_activations<E5, ADT, MT>(a, a_vec, a_scale, a_inv, m, k, kp, (int)m, xs, tid, [&] { load_batch(wave); });
    __syncthreads();

    const int fmt = E5 ? 1 : 0;
    const bool arow = fr < m;
    const uint8_t* xrow = xs + (arow ? fr : 0) * kp + fq * 32;
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = wave; s0 < steps; s0 += 4 * kGemvUnroll) {
        if (s0 != wave) load_batch(s0);
#pragma unroll
        for (int u = 0; u < kGemvUnroll; ++u) {
            const int s = s0 + 4 * u;
            if (s >= steps) break;  // wave-uniform
            uint4 x0 = make_uint4(0, 0, 0, 0), x1 = x0;
            if (arow) {
                x0 = *reinterpret_cast<const uint4*>(xrow + s * 128);
                x1 = *reinterpret_cast<const uint4*>(xrow + s * 128 + 16);
            }
            const v8i av = v8i{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
            const v8i bv = v8i{(int)wb[u][0].x, (int)wb[u][0].y, (int)wb[u][0].z, (int)wb[u][0].w,
                               (int)wb[u][1].x, (int)wb[u][1].y, (int)wb[u][1].z, (int)wb[u][1].w};
            acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, fmt, fmt, 0, 127, 0, 127);
        }
    }
    // C fragment of lane l: column l%16, rows 4*(l/16) .. +3.
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][fq * 4 + r][fr] = acc[r];
    __syncthreads();
    const int row = tid >> 4, cc = tid & 15;
    const int64_t col = col0 + cc;
    if (row < m && col < n) ep.store(red[0][row][cc] + red[1][row][cc] + red[2][row][cc] + red[3][row][cc], row, col);
}

// Same MFMA GEMV without the LDS staging, for 16-byte aligned activation rows whose length is a multiple of
// 16 bytes' worth of elements (k % (16 / element size) == 0): each lane
// loads and encodes exactly the 32 activations of its own A-operand slice (row l%16, K slice l/16 of the
// step) in registers.  The staging kernel has every thread of a block encode the whole activation
// matrix into LDS in serial batches and wait at a barrier; here the activation loads of a batch of
// steps are issued together, ahead of that batch's weight loads, and no barrier precedes the MFMAs.
// POW2: a_inv != 0 (power-of-two activation scale), so x / s is x * (1/s) exactly and no division is compiled.
// Encoding: the hardware converter's codes for the whole batch with a running special-code flag
// (encode4_flag, no branch); a lane whose batch met a value beyond the largest finite code, Inf or NaN
// re-encodes the batch with the reference's saturated / special codes (encode4) in one cold branch.
// NW waves split K (wave w takes the steps w, w + NW, ...), U steps per load batch; the NW partial 16x16
// tiles are summed through LDS.
// OB: 0 = the general epilogue (ep.store); 1, 2, 4 = output bytes (FP8 code, BF16, FP32) for a power-of-two
// output scale, with the M = 1 kernel's hardware-converter encode -- a short, branch-free tail in place of
// the general one's software codec and division (the tail runs once per launch with a cold instruction cache).
template <bool E5, int ADT, int U, bool POW2, int NW, int OB = 0>
__global__ __launch_bounds__(NW * 64) void fp8_gemv_mfma_reg_kernel(const void* __restrict__ a, float a_scale,
                                                                          float a_inv, int64_t m, int64_t k,
                                                                          const uint8_t* __restrict__ w, int64_t kp,
                                                                          int64_t n, Fp8Epilogue ep) {
    __shared__ float red[NW][16][17];
    constexpr int esz = ADT == 0 ? 1 : (ADT == 1 ? 2 : 4);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t col0 = (int64_t)blockIdx.x * 16;
    const int steps = (int)(kp / 128);
    const int fr = lane & 15;
    const int fq = lane >> 4;
    const uint8_t* wcol = w + (col0 + fr) * kp + fq * 32;  // rows past n: zero padding of the prepared weight
    const bool arow = fr < m;
    const uint8_t* arow_p = static_cast<const uint8_t*>(a) + (arow ? (int64_t)fr * k * esz : 0);
    const int fmt = E5 ? 1 : 0;
    v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    // 16-byte activation loads cover 16 / esz elements: two groups of 4 (bf16), one (fp32), four (fp8)
    constexpr int kPer16 = 16 / esz / 4;      // groups per 16-byte load
    constexpr int kLoads = 8 / kPer16;        // 16-byte loads per lane per step
    for (int s0 = wave; s0 < steps; s0 += NW * U) {
        // activation loads of this batch first (L2 hits: their wait then leaves the weight loads in flight);
        // lanes of rows past m issue none
        uint4 raw[U][kLoads];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + NW * u < steps ? s0 + NW * u : steps - 1;
#pragma unroll
            for (int j = 0; j < kLoads; ++j) {
                const int64_t kk = (int64_t)s * 128 + fq * 32 + j * kPer16 * 4;
                raw[u][j] = make_uint4(0, 0, 0, 0);
                if (arow && kk < k) raw[u][j] = *reinterpret_cast<const uint4*>(arow_p + kk * esz);
            }
        }
        uint4 wb[U][2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = s0 + NW * u;
            const uint8_t* p = wcol + (int64_t)(s < steps ? s : steps - 1) * 128;  // clamped: unconditional
            wb[u][0] = load_stream16(p);
            wb[u][1] = load_stream16(p + 16);
        }
        // activation codes of the whole batch: hot pass with the hardware converter, one cold fix-up branch
        auto act = [&](int u, int g, int i) -> float {
            const uint4 v = raw[u][g / kPer16];
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
            uint32_t bits;
            if constexpr (ADT == 1) {
                const uint32_t d = w4[(g % 2) * 2 + (i >> 1)];
                bits = i & 1 ? d & 0xffff0000u : d << 16;
            } else {
                bits = w4[i];
            }
            const float x = fhip::bits_f32(bits);
            return POW2 ? x * a_inv : x / a_scale;
        };
        uint32_t c[U][8];
        if constexpr (ADT == 0) {
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    const uint4 v = raw[u][g / kPer16];
                    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
                    c[u][g] = w4[g % 4];
                }
        } else {
            uint32_t flag = 0;
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    const float q[4] = {act(u, g, 0), act(u, g, 1), act(u, g, 2), act(u, g, 3)};
                    c[u][g] = encode4_flag<E5>(q, flag);  // zero inputs (rows past m, K past k) encode to 0
                }
            if (__builtin_expect((flag & 0x80808080u) != 0, 0)) {
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int g = 0; g < 8; ++g) {
                        const float q[4] = {act(u, g, 0), act(u, g, 1), act(u, g, 2), act(u, g, 3)};
                        c[u][g] = encode4<E5>(q);
                    }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (s0 + NW * u >= steps) break;  // wave-uniform
            const v8i av = v8i{(int)c[u][0], (int)c[u][1], (int)c[u][2], (int)c[u][3], (int)c[u][4], (int)c[u][5],
                               (int)c[u][6], (int)c[u][7]};
            const v8i bv = v8i{(int)wb[u][0].x, (int)wb[u][0].y, (int)wb[u][0].z, (int)wb[u][0].w,
                               (int)wb[u][1].x, (int)wb[u][1].y, (int)wb[u][1].z, (int)wb[u][1].w};
            acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, fmt, fmt, 0, 127, 0, 127);
        }
    }
    // C fragment of lane l: column l%16, rows 4*(l/16) .. +3.
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][fq * 4 + r][fr] = acc[r];
    __syncthreads();
    if (tid < 256) {
        const int row = tid >> 4, cc = tid & 15;
        const int64_t col = col0 + cc;
        float sum = red[0][row][cc];
#pragma unroll
        for (int q = 1; q < NW; ++q) sum += red[q][row][cc];
        if (row < m && col < n) {
            if constexpr (OB == 0) {
                ep.store(sum, row, col);
            } else {
                // the general epilogue's order: acc*ab_scale, *alpha, [+ beta*bias], then * (1/out_scale)
                float y = sum * ep.ab_scale;
                y *= ep.alpha;
                if (ep.bias_kind != FHIP_BIAS_NONE) {
                    const uint8_t bc = ep.bias[ep.bias_kind == FHIP_BIAS_VECTOR ? col : row * ep.n + col];
                    y += ep.beta * (fhip::fp8_decode(bc, E5) * ep.bias_scale);
                }
                const uint32_t code = encode1<E5>(y * ep.out_inv);
                const int64_t idx = row * ep.n + col;
                if constexpr (OB == 1) static_cast<uint8_t*>(ep.out)[idx] = (uint8_t)code;
                else if constexpr (OB == 2) static_cast<uint16_t*>(ep.out)[idx] = fhip::bf16_encode(decode_code<E5>(code) * ep.out_scale);
                else static_cast<float*>(ep.out)[idx] = decode_code<E5>(code) * ep.out_scale;
            }
        }
    }
}

// ---- M = 1 decode GEMV, the common case ---------------------------------------------------------
// One activation row whose elements come in aligned groups of 4, power-of-two activation and output
// scales (so x / s is x * (1/s) exactly) -- the fused Cast -> MatMul -> Cast of decoding.  Same
// arithmetic as fp8_gemv_kernel, with everything the general kernel decides at run time fixed at
// compile time: the activation load is issued first (an L2 hit, so its wait does not also wait for
// the weight stream issued right after), encoding is the hardware converter with the reference's
// saturation fix-up, and the output type is a template parameter.
template <int ADT>
__device__ __forceinline__ void load_act_group(const void* __restrict__ a, int64_t k, int g, uint32_t (&raw)[4],
                                               bool& live) {
    live = (int64_t)g * 4 < k;
    const int64_t e = live ? (int64_t)g * 4 : 0;
    if constexpr (ADT == 0) {
        raw[0] = *(reinterpret_cast<const uint32_t*>(a) + e / 4);
    } else if constexpr (ADT == 1) {
        const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a) + e);
        raw[0] = v.x << 16;
        raw[1] = v.x & 0xffff0000u;
        raw[2] = v.y << 16;
        raw[3] = v.y & 0xffff0000u;
    } else {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const float*>(a) + e);
        raw[0] = v.x;
        raw[1] = v.y;
        raw[2] = v.z;
        raw[3] = v.w;
    }
}

template <bool E5, int ADT>
__device__ __forceinline__ uint32_t encode_act_group(const uint32_t (&raw)[4], float a_inv, bool live) {
    if (!live) return 0u;
    if constexpr (ADT == 0) return raw[0];
    float q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = fhip::bits_f32(raw[i]) * a_inv;
    return encode4<E5>(q);
}

// Activations of one 16-element chunk as four groups of raw words: VEC (k % 16 == 0) with 16-byte loads of
// the chunk (a chunk lies wholly inside the row or wholly past it), else per-group loads.  Loads are
// unconditional (clamped addresses); groups past k are flagged dead.
template <int ADT, bool VEC>
__device__ __forceinline__ void load_act_chunk(const void* __restrict__ a, int64_t k, int c, uint32_t (&raw)[4][4],
                                               bool (&live)[4]) {
    if constexpr (VEC) {
        constexpr int esz = ADT == 0 ? 1 : (ADT == 1 ? 2 : 4);
        const bool in = (int64_t)c * 16 < k;
        const uint8_t* p = static_cast<const uint8_t*>(a) + (in ? (int64_t)c * 16 * esz : 0);
        uint32_t wd[4 * esz];
#pragma unroll
        for (int j = 0; j < esz; ++j) {
            const uint4 v = *reinterpret_cast<const uint4*>(p + 16 * j);
            wd[4 * j] = v.x;
            wd[4 * j + 1] = v.y;
            wd[4 * j + 2] = v.z;
            wd[4 * j + 3] = v.w;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            live[g] = in;
            if constexpr (ADT == 0) {
                raw[g][0] = wd[g];
            } else if constexpr (ADT == 1) {
                raw[g][0] = wd[2 * g] << 16;
                raw[g][1] = wd[2 * g] & 0xffff0000u;
                raw[g][2] = wd[2 * g + 1] << 16;
                raw[g][3] = wd[2 * g + 1] & 0xffff0000u;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) raw[g][i] = wd[4 * g + i];
            }
        }
    } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) load_act_group<ADT>(a, k, 4 * c + g, raw[g], live[g]);
    }
}

template <bool E5, int ADT, int OUT_BYTES, int R, bool VEC, bool SINGLE>
__global__ __launch_bounds__(kGemvThreads) void fp8_gemv1_kernel(const void* __restrict__ a, float a_inv, int64_t k,
                                                                  const uint8_t* __restrict__ w, int64_t kp, int64_t n,
                                                                  Fp8Epilogue ep) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row0 = ((int64_t)blockIdx.x * (kGemvThreads / 64) + wave) * R;
    const int chunks = (int)(kp / 16);
    // Lane l owns the 16-element chunks l, l+64, ... of every row of its wave.  It loads and encodes the
    // activations of its own chunk in registers: no LDS staging and no barrier, which measured 0.4 us
    // per launch on the C2 shape.  The activation loads (L2 hits after the first wave) are issued before
    // the weight loads, so waiting for them leaves the weight stream in flight.  Encoding keeps the
    // hardware codes in the hot path; a lane that meets a value past the largest finite code (or
    // Inf/NaN) redoes its chunk with the reference's saturated / special codes.
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    // SINGLE (kp <= 1024, the decode shapes): one chunk per lane, no loop, so the loads issue right
    // after the kernel arguments arrive; lanes past the padded row read chunk 0 and contribute zero.
    for (int c = lane; SINGLE ? c == lane : c < chunks; c += 64) {
        const bool lane_live = !SINGLE || c < chunks;
        const int cc = SINGLE && !lane_live ? 0 : c;
        uint32_t raw[4][4];
        bool live[4];
        load_act_chunk<ADT, VEC>(a, k, cc, raw, live);
        uint4 wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r) wv[r] = load_stream16(w + (row0 + r) * kp + cc * 16);
#pragma unroll
        for (int g = 0; g < 4; ++g) live[g] = live[g] && lane_live;
        if (SINGLE && !lane_live) {  // a NaN weight code in chunk 0 must not meet the zero activation
#pragma unroll
            for (int r = 0; r < R; ++r) wv[r] = make_uint4(0, 0, 0, 0);
        }
        uint32_t xc[4];
        if constexpr (ADT == 0) {
#pragma unroll
            for (int g = 0; g < 4; ++g) xc[g] = live[g] ? raw[g][0] : 0u;
        } else {
            uint32_t flag = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                float q[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) q[i] = fhip::bits_f32(raw[g][i]) * a_inv;
                const uint32_t code = encode4_flag<E5>(q, flag);
                xc[g] = live[g] ? code : 0u;
            }
            if (__builtin_expect((flag & 0x80808080u) != 0, 0)) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float q[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) q[i] = fhip::bits_f32(raw[g][i]) * a_inv;
                    xc[g] = live[g] ? encode4<E5>(q) : 0u;
                }
            }
        }
        float xf[16];
        decode4<E5>(xc[0], xf);
        decode4<E5>(xc[1], xf + 4);
        decode4<E5>(xc[2], xf + 8);
        decode4<E5>(xc[3], xf + 12);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float wf[16];
            decode4<E5>(wv[r].x, wf);
            decode4<E5>(wv[r].y, wf + 4);
            decode4<E5>(wv[r].z, wf + 8);
            decode4<E5>(wv[r].w, wf + 12);
            float s = acc[r];
#pragma unroll
            for (int i = 0; i < 16; ++i) s += wf[i] * xf[i];
            acc[r] = s;
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = fhip::wave_sum(acc[r]);
    float mine = acc[0];
#pragma unroll
    for (int r = 1; r < R; ++r) mine = lane == r ? acc[r] : mine;
    const int64_t col = row0 + lane;
    if (lane < R && col < n) {
        // the general epilogue's order: acc*ab_scale, *alpha, [+ beta*bias], then * (1/out_scale)
        float y = mine * ep.ab_scale;
        y *= ep.alpha;
        if (ep.bias_kind != FHIP_BIAS_NONE) {
            const uint8_t bc = ep.bias[col];  // vector bias (a matrix bias has one row here)
            y += ep.beta * (fhip::fp8_decode(bc, E5) * ep.bias_scale);
        }
        const uint32_t code = encode1<E5>(y * ep.out_inv);
        if constexpr (OUT_BYTES == 1) {
            static_cast<uint8_t*>(ep.out)[col] = (uint8_t)code;
        } else if constexpr (OUT_BYTES == 2) {
            static_cast<uint16_t*>(ep.out)[col] = fhip::bf16_encode(decode_code<E5>(code) * ep.out_scale);
        } else {
            static_cast<float*>(ep.out)[col] = decode_code<E5>(code) * ep.out_scale;
        }
    }
}

// ---- GEMM operand staging: FP8 codes [m][k64], k64 = k rounded up to 64, zero padded; BF16/FP32
// activations are encoded with the preceding Cast node's rule Enc(x / a_scale).
__global__ void stage_gemm_a_kernel(const void* __restrict__ a, int a_dtype, float a_scale, float a_inv, int64_t m,
                                    int64_t k, int64_t k64, uint8_t* __restrict__ dst, bool e5) {
    const int64_t total = m * k64;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / k64, kk = i - r * k64;
        uint8_t code = 0;
        if (kk < k) {
            const int64_t e = r * k + kk;
            if (a_dtype == FHIP_BF16) {
                const float x = fhip::bf16_decode(static_cast<const uint16_t*>(a)[e]);
                code = fhip::fp8_encode(a_inv != 0.0f ? x * a_inv : x / a_scale, e5);
            } else if (a_dtype == FHIP_FP32) {
                const float x = static_cast<const float*>(a)[e];
                code = fhip::fp8_encode(a_inv != 0.0f ? x * a_inv : x / a_scale, e5);
            } else {
                code = static_cast<const uint8_t*>(a)[e];
            }
        }
        dst[i] = code;
    }
}

// ---- Cast ------------------------------------------------------------------------------------
// Cast decodes in software: the reference decodes every NaN code to +qNaN, while the hardware
// converter keeps the code's sign, which a following BF16/FP16 encode would preserve.
__device__ __forceinline__ float cast_read(const void* src, int dtype, int64_t i, float scale) {
    switch (dtype) {
        case FHIP_FP32: return static_cast<const float*>(src)[i];
        case FHIP_BF16: return fhip::bf16_decode(static_cast<const uint16_t*>(src)[i]);
        case FHIP_FP16: return fhip::fp16_decode(static_cast<const uint16_t*>(src)[i]);
        case FHIP_FP8E4M3: return fhip::fp8_decode(static_cast<const uint8_t*>(src)[i], false) * scale;
        default: return fhip::fp8_decode(static_cast<const uint8_t*>(src)[i], true) * scale;
    }
}

__global__ void cast_kernel(const void* __restrict__ src, int src_dtype, float src_scale, int64_t count, void* dst,
                            int dst_dtype, float dst_scale) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const float v = cast_read(src, src_dtype, i, src_scale);
        switch (dst_dtype) {
            case FHIP_FP32: static_cast<float*>(dst)[i] = v; break;
            case FHIP_BF16: static_cast<uint16_t*>(dst)[i] = fhip::bf16_encode(v); break;
            case FHIP_FP16: static_cast<uint16_t*>(dst)[i] = fhip::fp16_encode_cast(v); break;  // FloatToHalf
            case FHIP_FP8E4M3: static_cast<uint8_t*>(dst)[i] = fhip::fp8_encode(v / dst_scale, false); break;
            default: static_cast<uint8_t*>(dst)[i] = fhip::fp8_encode(v / dst_scale, true); break;
        }
    }
}

bool is_fp8(int d) { return d == FHIP_FP8E4M3 || d == FHIP_FP8E5M2; }
bool is_castable(int d) { return d == FHIP_FP32 || d == FHIP_BF16 || d == FHIP_FP16 || is_fp8(d); }

unsigned grid_for(int64_t count, int threads) {
    int64_t blocks = (count + threads - 1) / threads;
    if (blocks > 65536) blocks = 65536;
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

template <bool E5, int ADT>
int launch_gemv_t(fhip_context ctx, const void* a, float a_scale, int64_t m, const fhip_weight_s* w,
                  const Fp8Epilogue& ep) {
    const int64_t kp = ((w->k + 127) / 128) * 128;
    const uint8_t* wd = static_cast<const uint8_t*>(w->data);
    const int a_vec = (w->k % 4 == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0) ? 1 : 0;
    const float a_inv = pow2_inverse(a_scale);
    if (m == 1 && a_vec && a_inv != 0.0f && ep.out_inv != 0.0f) {
        constexpr int R = FHIP_GEMV_R1;
        const unsigned grid = (unsigned)((w->n + 4 * R - 1) / (4 * R));
#define FHIP_GEMV1_LAUNCH1(OB, V, S)                                                                              \
    fp8_gemv1_kernel<E5, ADT, OB, R, V, S><<<grid, kGemvThreads, 0, ctx->stream>>>(a, a_inv, w->k, wd, kp, w->n, ep)
#define FHIP_GEMV1_LAUNCH(OB, V)                                                                                  \
    do {                                                                                                          \
        if (kp <= 1024) FHIP_GEMV1_LAUNCH1(OB, V, true); else FHIP_GEMV1_LAUNCH1(OB, V, false);                  \
    } while (0)
        const bool vec = w->k % 16 == 0;
        if (ep.out_dtype == FHIP_BF16) {
            if (vec) FHIP_GEMV1_LAUNCH(2, true); else FHIP_GEMV1_LAUNCH(2, false);
        } else if (ep.out_dtype == FHIP_FP32) {
            if (vec) FHIP_GEMV1_LAUNCH(4, true); else FHIP_GEMV1_LAUNCH(4, false);
        } else {
            if (vec) FHIP_GEMV1_LAUNCH(1, true); else FHIP_GEMV1_LAUNCH(1, false);
        }
#undef FHIP_GEMV1_LAUNCH
#undef FHIP_GEMV1_LAUNCH1
        ctx->last_backend = "fp8_gemv_m1";
        FHIP_CHECK_LAUNCH(ctx, "fp8_gemv1_kernel");
        return FHIP_OK;
    }
    constexpr int kVecElems = ADT == 0 ? 16 : (ADT == 1 ? 8 : 4);
    // 2 <= m <= 16 with aligned activation rows: the register kernel; otherwise the LDS-staged kernel
    if (m > 1 && m <= 16 && a_vec && w->k % kVecElems == 0) {
        const unsigned grid = (unsigned)((w->n + 15) / 16);
        // 8 waves split K (one 128-deep step each per batch at K <= 1024), so each lane encodes 32 activations
        // per step of its own and two waves per SIMD cover each other's encode latency
#define FHIP_REG_LAUNCH(U, P2, OB)                                                                                \
    fp8_gemv_mfma_reg_kernel<E5, ADT, U, P2, 8, OB><<<grid, 8 * 64, 0, ctx->stream>>>(a, a_scale, a_inv, m, w->k, wd, \
                                                                                      kp, w->n, ep)
#define FHIP_REG_LAUNCH_OB(U)                                                                                     \
    do {                                                                                                          \
        if (ob == 1) FHIP_REG_LAUNCH(U, true, 1);                                                                 \
        else if (ob == 2) FHIP_REG_LAUNCH(U, true, 2);                                                            \
        else if (ob == 4) FHIP_REG_LAUNCH(U, true, 4);                                                            \
        else FHIP_REG_LAUNCH(U, true, 0);                                                                         \
    } while (0)
        const bool p2 = a_inv != 0.0f;
        // power-of-two activation and output scales (decode): the specialized output tail
        const int ob = ep.out_inv == 0.0f ? 0 : (ep.out_dtype == FHIP_BF16 ? 2 : (ep.out_dtype == FHIP_FP32 ? 4 : 1));
        if (kp / 128 <= 8) {
            if (p2) FHIP_REG_LAUNCH_OB(1);
            else FHIP_REG_LAUNCH(1, false, 0);
        } else {
            if (p2) FHIP_REG_LAUNCH_OB(2);
            else FHIP_REG_LAUNCH(2, false, 0);
        }
#undef FHIP_REG_LAUNCH_OB
#undef FHIP_REG_LAUNCH
        ctx->last_backend = "fp8_gemv_mfma";
        FHIP_CHECK_LAUNCH(ctx, "fp8_gemv_mfma_reg_kernel");
        return FHIP_OK;
    }
    if (m <= 16) {
        const unsigned grid = (unsigned)((w->n + 15) / 16);
        const size_t lds = (size_t)m * kp;
        if (m <= 4)
            fp8_gemv_mfma_kernel<E5, ADT, 4><<<grid, kGemvThreads, lds, ctx->stream>>>(a, a_vec, a_scale, a_inv, m, w->k,
                                                                                      wd, kp, w->n, ep);
        else
            fp8_gemv_mfma_kernel<E5, ADT, 16><<<grid, kGemvThreads, lds, ctx->stream>>>(a, a_vec, a_scale, a_inv, m, w->k,
                                                                                       wd, kp, w->n, ep);
        ctx->last_backend = "fp8_gemv_mfma";
        FHIP_CHECK_LAUNCH(ctx, "fp8_gemv_mfma_kernel");
        return FHIP_OK;
    }
    return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "gemv: m > 16");
}

template <bool E5>
int launch_gemv(fhip_context ctx, const void* a, int a_dtype, float a_scale, int64_t m, const fhip_weight_s* w,
                const Fp8Epilogue& ep) {
    if (a_dtype == FHIP_BF16) return launch_gemv_t<E5, 1>(ctx, a, a_scale, m, w, ep);
    if (a_dtype == FHIP_FP32) return launch_gemv_t<E5, 2>(ctx, a, a_scale, m, w, ep);
    return launch_gemv_t<E5, 0>(ctx, a, a_scale, m, w, ep);
}

}  // namespace

float fhip::pow2_inverse(float s) {
    int e = 0;
    const float f = std::frexp(s, &e);
    if (f != 0.5f) return 0.0f;
    const float inv = std::ldexp(1.0f, 1 - e);
    return std::isfinite(inv) && inv * s == 1.0f ? inv : 0.0f;
}

extern "C" {

int fhip_cast(fhip_context ctx, int src_dtype, const void* src, float src_scale, int64_t count, int dst_dtype,
              void* dst, float dst_scale) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (count == 0) return FHIP_OK;  // empty tensor: nothing to convert
    if (!src || !dst || count < 0 || !is_castable(src_dtype) || !is_castable(dst_dtype))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "cast: bad arguments");
    if ((is_fp8(src_dtype) && !fhip::valid_scale(src_scale)) || (is_fp8(dst_dtype) && !fhip::valid_scale(dst_scale)))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "cast: FP8 scale must be finite and positive");
    if (count == 0) return FHIP_OK;
    cast_kernel<<<grid_for(count, 256), 256, 0, ctx->stream>>>(src, src_dtype, src_scale, count, dst, dst_dtype,
                                                                dst_scale);
    ctx->last_backend = "cast";
    FHIP_CHECK_LAUNCH(ctx, "cast_kernel");
    return FHIP_OK;
}

int fhip_fp8_linear(fhip_context ctx, int a_dtype, const void* a, float a_scale, int64_t m, fhip_weight w,
                    float w_scale, const uint8_t* bias, float bias_scale, int bias_kind, float alpha, float beta,
                    int out_dtype, void* out, float out_scale) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (m == 0) return FHIP_OK;  // no activation rows: the reference's loops run zero times
    if (!w || !a || !out || m < 0 || w->kind != kLinearWeight || !is_fp8(w->dtype))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "fp8_linear: bad arguments");
    if (a_dtype != w->dtype && a_dtype != FHIP_BF16 && a_dtype != FHIP_FP32)
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8_linear: activation dtype must match the weight");
    if (out_dtype != w->dtype && out_dtype != FHIP_BF16 && out_dtype != FHIP_FP32)
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8_linear: output dtype");
    if (!fhip::valid_scale(a_scale) || !fhip::valid_scale(w_scale) || !fhip::valid_scale(out_scale) ||
        (bias_kind != FHIP_BIAS_NONE && (!bias || !fhip::valid_scale(bias_scale))) ||
        bias_kind < FHIP_BIAS_NONE || bias_kind > FHIP_BIAS_MATRIX)
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "fp8_linear: scales must be finite and positive");
    const bool e5 = w->dtype == FHIP_FP8E5M2;
    Fp8Epilogue ep{a_scale * w_scale, alpha, beta, bias, bias_scale, bias_kind, out_scale, pow2_inverse(out_scale),
                   out_dtype, out, w->n, e5};
    const int64_t kp = ((w->k + 127) / 128) * 128;
    if (m <= 16 && (size_t)(16 * kp) <= (size_t)kGemvMaxLds) {
        return e5 ? launch_gemv<true>(ctx, a, a_dtype, a_scale, m, w, ep)
                  : launch_gemv<false>(ctx, a, a_dtype, a_scale, m, w, ep);
    }
    // MFMA path: A must be FP8 codes with K a multiple of 64 and 16-byte aligned rows.
    const uint8_t* codes = static_cast<const uint8_t*>(a);
    const int64_t k64 = (w->k + 63) / 64 * 64;
    if (a_dtype != w->dtype || k64 != w->k || (reinterpret_cast<uintptr_t>(a) & 15) != 0) {
        void* ws = nullptr;
        int rc = fhip::acquire_workspace(ctx, (size_t)(m * k64), &ws);
        if (rc != FHIP_OK) return rc;
        stage_gemm_a_kernel<<<grid_for(m * k64, 256), 256, 0, ctx->stream>>>(a, a_dtype, a_scale, pow2_inverse(a_scale),
                                                                              m, w->k, k64, static_cast<uint8_t*>(ws), e5);
        FHIP_CHECK_LAUNCH(ctx, "stage_gemm_a_kernel");
        codes = static_cast<const uint8_t*>(ws);
    }
    return fhip::launch_fp8_gemm(ctx, codes, m, k64, w, ep);
}

}  // extern "C"
