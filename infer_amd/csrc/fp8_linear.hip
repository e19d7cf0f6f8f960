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
//   * fp8_gemv_kernel   -- decode rows (m <= 16): bandwidth-bound.  Weight rows stream from HBM
//                          with 16-byte loads, activations are staged once per block in LDS as FP8
//                          codes, products accumulate on the VALU, a cross-lane butterfly reduces.
//   * fp8_mfma_gemm_kernel -- prefill (m > 16): v_mfma_scale_f32_16x16x128_f8f6f4 with unit
//                          block scales, fp32 accumulation.
// Weights come prepared as [Np][Kp] (K contiguous, zero padded; runtime.hip).
#include "fhip_internal.h"
#include "codec.h"

namespace {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Decodes four FP8 codes packed little-endian in `w` with the hardware OCP converters.
template <bool E5>
__device__ __forceinline__ void decode4(uint32_t w, float* out) {
    v2f lo, hi;
    if constexpr (E5) {
        lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, false);
        hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, true);
    } else {
        lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
        hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    }
    out[0] = lo.x;
    out[1] = lo.y;
    out[2] = hi.x;
    out[3] = hi.y;
}

struct Fp8Epilogue {
    float ab_scale;      // a_scale * w_scale
    float alpha, beta;
    const uint8_t* bias;
    float bias_scale;
    int bias_kind;
    float out_scale;
    int out_dtype;       // FP8 (code), BF16 or FP32 (decoded through the FP8 code)
    void* out;
    int64_t n;           // row stride of out
    bool e5;

    __device__ __forceinline__ void store(float acc, int64_t row, int64_t col) const {
        float y = acc * ab_scale;
        if (bias_kind != FHIP_BIAS_NONE) {
            y *= alpha;
            const uint8_t bc = bias[bias_kind == FHIP_BIAS_VECTOR ? col : row * n + col];
            y += beta * (fhip::fp8_decode(bc, e5) * bias_scale);
        } else {
            y *= alpha;
        }
        const uint8_t code = fhip::fp8_encode(y / out_scale, e5);
        const int64_t idx = row * n + col;
        if (out_dtype == FHIP_BF16) {
            static_cast<uint16_t*>(out)[idx] = fhip::bf16_encode(fhip::fp8_decode(code, e5) * out_scale);
        } else if (out_dtype == FHIP_FP32) {
            static_cast<float*>(out)[idx] = fhip::fp8_decode(code, e5) * out_scale;
        } else {
            static_cast<uint8_t*>(out)[idx] = code;
        }
    }
};

// Loads activation element i of row r as an FP8 code: FP8 input is copied, BF16/FP32 input is
// encoded with the preceding Cast node's rule Enc(x / a_scale).
template <bool E5>
__device__ __forceinline__ uint8_t activation_code(const void* a, int a_dtype, int64_t idx, float a_scale) {
    if (a_dtype == FHIP_BF16) return fhip::fp8_encode(fhip::bf16_decode(static_cast<const uint16_t*>(a)[idx]) / a_scale, E5);
    if (a_dtype == FHIP_FP32) return fhip::fp8_encode(static_cast<const float*>(a)[idx] / a_scale, E5);
    return static_cast<const uint8_t*>(a)[idx];
}

constexpr int kGemvThreads = 256;
constexpr int kGemvRowsPerWave = 2;
constexpr int kGemvMaxLds = 64 * 1024;

// grid.x = ceil(n / (4 waves * R rows)); one wave owns R weight rows, lane l owns the 16-byte
// chunks l, l+64, ... of each row.
template <bool E5, int MT>
__global__ __launch_bounds__(kGemvThreads) void fp8_gemv_kernel(const void* __restrict__ a, int a_dtype, float a_scale,
                                                                 int64_t m, int64_t k, const uint8_t* __restrict__ w,
                                                                 int64_t kp, int64_t n, Fp8Epilogue ep) {
    extern __shared__ __align__(16) uint8_t xs[];  // [MT][kp] FP8 codes
    const int tid = threadIdx.x;
    for (int64_t idx = tid; idx < MT * kp; idx += kGemvThreads) {
        const int64_t r = idx / kp, kk = idx - r * kp;
        xs[idx] = (r < m && kk < k) ? activation_code<E5>(a, a_dtype, r * k + kk, a_scale) : (uint8_t)0;
    }
    __syncthreads();

    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row0 = ((int64_t)blockIdx.x * (kGemvThreads / 64) + wave) * kGemvRowsPerWave;
    float acc[kGemvRowsPerWave][MT];
#pragma unroll
    for (int r = 0; r < kGemvRowsPerWave; ++r)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[r][j] = 0.0f;

    const int64_t chunks = kp / 16;
    for (int64_t c = lane; c < chunks; c += 64) {
        uint4 wv[kGemvRowsPerWave];
#pragma unroll
        for (int r = 0; r < kGemvRowsPerWave; ++r) {
            const int64_t row = row0 + r < n ? row0 + r : n - 1;  // clamp: duplicate work, never stored
            wv[r] = *reinterpret_cast<const uint4*>(w + row * kp + c * 16);
        }
        float wf[kGemvRowsPerWave][16];
#pragma unroll
        for (int r = 0; r < kGemvRowsPerWave; ++r) {
            decode4<E5>(wv[r].x, wf[r]);
            decode4<E5>(wv[r].y, wf[r] + 4);
            decode4<E5>(wv[r].z, wf[r] + 8);
            decode4<E5>(wv[r].w, wf[r] + 12);
        }
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            const uint4 xv = *reinterpret_cast<const uint4*>(xs + j * kp + c * 16);
            float xf[16];
            decode4<E5>(xv.x, xf);
            decode4<E5>(xv.y, xf + 4);
            decode4<E5>(xv.z, xf + 8);
            decode4<E5>(xv.w, xf + 12);
#pragma unroll
            for (int r = 0; r < kGemvRowsPerWave; ++r) {
                float s = acc[r][j];
#pragma unroll
                for (int i = 0; i < 16; ++i) s += wf[r][i] * xf[i];
                acc[r][j] = s;
            }
        }
    }
    // Butterfly over the 64 lanes: every lane ends with the full sums.
#pragma unroll
    for (int r = 0; r < kGemvRowsPerWave; ++r)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            float v = acc[r][j];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
            acc[r][j] = v;
        }
#pragma unroll
    for (int r = 0; r < kGemvRowsPerWave; ++r)
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            if (lane == r * MT + j && j < m && row0 + r < n) ep.store(acc[r][j], j, row0 + r);
        }
}

// ---- MFMA GEMM (first version: operands straight from global/L2 into registers) -------------
// Block: 4 waves in a 2 x 2 arrangement, wave tile (16*WM) x (16*WN), block tile (32*WM) x (32*WN).
// A: [m][k] FP8 codes (row-major), B: prepared [Np][Kp].  k step 128 (one MFMA depth).
// Operand fragment of lane l: row/col l%16, bytes [32*(l/16), 32*(l/16)+32) of the 128-deep
// slice, for A and B alike, so both index the same k for every MFMA slot.
template <bool E5, int WM, int WN>
__global__ __launch_bounds__(256) void fp8_mfma_gemm_kernel(const uint8_t* __restrict__ a, int64_t m, int64_t k,
                                                            const uint8_t* __restrict__ b, int64_t kp,
                                                            Fp8Epilogue ep) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t row_base = (int64_t)blockIdx.y * (32 * WM) + (wave >> 1) * (16 * WM);
    const int64_t col_base = (int64_t)blockIdx.x * (32 * WN) + (wave & 1) * (16 * WN);
    const int frag_row = lane & 15;
    const int frag_k = (lane >> 4) * 32;
    constexpr int fmt = E5 ? 1 : 0;

    v4f acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int64_t k0 = 0; k0 < k; k0 += 128) {
        v8i af[WM], bf[WN];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int64_t row = row_base + i * 16 + frag_row;
            const int64_t kk = k0 + frag_k;
            uint4 lo = make_uint4(0, 0, 0, 0), hi = make_uint4(0, 0, 0, 0);
            if (row < m) {
                const uint8_t* p = a + row * k + kk;
                if (kk < k) lo = *reinterpret_cast<const uint4*>(p);
                if (kk + 16 < k) hi = *reinterpret_cast<const uint4*>(p + 16);
            }
            af[i] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const uint8_t* p = b + (col_base + j * 16 + frag_row) * kp + k0 + frag_k;
            const uint4 lo = *reinterpret_cast<const uint4*>(p);
            const uint4 hi = *reinterpret_cast<const uint4*>(p + 16);
            bf[j] = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[i], bf[j], acc[i][j], fmt, fmt, 0, 127,
                                                                             0, 127);
    }
    // C fragment of lane l: column l%16, rows 4*(l/16) .. +3.
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int64_t col = col_base + j * 16 + (lane & 15);
            if (col >= ep.n) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = row_base + i * 16 + (lane >> 4) * 4 + r;
                if (row < m) ep.store(acc[i][j][r], row, col);
            }
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
            case FHIP_FP16: static_cast<uint16_t*>(dst)[i] = fhip::fp16_encode(v); break;
            case FHIP_FP8E4M3: static_cast<uint8_t*>(dst)[i] = fhip::fp8_encode(v / dst_scale, false); break;
            default: static_cast<uint8_t*>(dst)[i] = fhip::fp8_encode(v / dst_scale, true); break;
        }
    }
}

bool is_fp8(int d) { return d == FHIP_FP8E4M3 || d == FHIP_FP8E5M2; }
bool is_castable(int d) { return d == FHIP_FP32 || d == FHIP_BF16 || d == FHIP_FP16 || is_fp8(d); }
size_t dtype_bytes(int d) { return d == FHIP_FP32 ? 4 : (d == FHIP_BF16 || d == FHIP_FP16 ? 2 : 1); }

unsigned grid_for(int64_t count, int threads) {
    int64_t blocks = (count + threads - 1) / threads;
    if (blocks > 65536) blocks = 65536;
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

template <bool E5>
int launch_gemv(fhip_context ctx, const void* a, int a_dtype, float a_scale, int64_t m, const fhip_weight_s* w,
                const Fp8Epilogue& ep) {
    const int64_t kp = ((w->k + 127) / 128) * 128;
    const unsigned grid = (unsigned)((w->n + 4 * kGemvRowsPerWave - 1) / (4 * kGemvRowsPerWave));
    const uint8_t* wd = static_cast<const uint8_t*>(w->data);
#define FHIP_GEMV_CASE(MT)                                                                                      \
    if (m <= MT) {                                                                                              \
        const size_t lds = (size_t)MT * kp;                                                                     \
        fp8_gemv_kernel<E5, MT><<<grid, kGemvThreads, lds, ctx->stream>>>(a, a_dtype, a_scale, m, w->k, wd, kp, \
                                                                          w->n, ep);                            \
        ctx->last_backend = "fp8_gemv_m" #MT;                                                                  \
        FHIP_CHECK_LAUNCH(ctx, "fp8_gemv_kernel");                                                              \
        return FHIP_OK;                                                                                         \
    }
    FHIP_GEMV_CASE(1)
    FHIP_GEMV_CASE(2)
    FHIP_GEMV_CASE(4)
    FHIP_GEMV_CASE(8)
    FHIP_GEMV_CASE(16)
#undef FHIP_GEMV_CASE
    return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "gemv: m > 16");
}

template <bool E5>
int launch_gemm(fhip_context ctx, const uint8_t* a, int64_t m, const fhip_weight_s* w, const Fp8Epilogue& ep) {
    const int64_t kp = ((w->k + 127) / 128) * 128;
    constexpr int WM = 4, WN = 4;
    dim3 grid((unsigned)((w->n + 32 * WN - 1) / (32 * WN)), (unsigned)((m + 32 * WM - 1) / (32 * WM)));
    fp8_mfma_gemm_kernel<E5, WM, WN><<<grid, 256, 0, ctx->stream>>>(a, m, w->k, static_cast<const uint8_t*>(w->data),
                                                                    kp, ep);
    ctx->last_backend = "fp8_mfma_gemm_128x128";
    FHIP_CHECK_LAUNCH(ctx, "fp8_mfma_gemm_kernel");
    return FHIP_OK;
}

}  // namespace

extern "C" {

int fhip_cast(fhip_context ctx, int src_dtype, const void* src, float src_scale, int64_t count, int dst_dtype,
              void* dst, float dst_scale) {
    if (!ctx) return FHIP_ERR_INVALID;
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
    if (!w || !a || !out || m <= 0 || w->kind != kLinearWeight || !is_fp8(w->dtype))
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
    Fp8Epilogue ep{a_scale * w_scale, alpha, beta, bias, bias_scale, bias_kind, out_scale, out_dtype, out, w->n, e5};
    const int64_t kp = ((w->k + 127) / 128) * 128;
    if (m <= 16 && (size_t)(16 * kp) <= (size_t)kGemvMaxLds) {
        return e5 ? launch_gemv<true>(ctx, a, a_dtype, a_scale, m, w, ep)
                  : launch_gemv<false>(ctx, a, a_dtype, a_scale, m, w, ep);
    }
    if (w->k % 16 != 0)
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8_linear: MFMA path needs K % 16 == 0");
    const uint8_t* codes = static_cast<const uint8_t*>(a);
    if (a_dtype != w->dtype) {
        void* ws = nullptr;
        int rc = fhip::acquire_workspace(ctx, (size_t)(m * w->k), &ws);
        if (rc != FHIP_OK) return rc;
        rc = fhip_cast(ctx, a_dtype, a, 1.0f, m * w->k, w->dtype, ws, a_scale);
        if (rc != FHIP_OK) return rc;
        codes = static_cast<const uint8_t*>(ws);
    }
    return e5 ? launch_gemm<true>(ctx, codes, m, w, ep) : launch_gemm<false>(ctx, codes, m, w, ep);
}

}  // extern "C"
