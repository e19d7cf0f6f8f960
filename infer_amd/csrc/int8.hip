// int8.hip -- INT8 per-channel-requantized linear (MatMul/FC/Gemm), INT8 Conv2D as an implicit GEMM,
// QuantizeLinear and DequantizeLinear on gfx950.
//
// Accumulation: v_mfma_i32_16x16x64_i8, int32.  The activation zero point is folded out exactly:
//     sum_k (a - zp_a) * w  =  sum_k a * w  -  zp_a * sum_k w
// with sum_k w per output channel computed when the weight is prepared (weights must be symmetric,
// zp_w = 0, the static quantizer's choice: src/quant/static_quantizer.cc:211-287).  Conv padding
// taps are filled with zp_in so they contribute zero, as the reference skips them.
// The host bounds |every partial sum| below 2^31 before launching, so the int32 results equal the
// reference's int64 running sums exactly (src/kernel/common/gemm.cc:170-181).
//
// Requantization is the reference's, in fp64 with no contraction
// (src/kernel/common/int8_kernel_utils.h:155-179, include/quant/quantization.h:94-99):
//     real = acc * (double(s_in) * double(s_w[c]))                (MatMul, FC: acc includes bias)
//     real = (double(alpha)*dot + double(beta)*bias) * scale      (Gemm)
//     q    = clamp(round_half_away(real / double(s_out) + zp_out), -128, 127)
#include "fhip_internal.h"
#include "codec.h"
#include "i8_common.h"

#include <algorithm>
#include <cmath>

namespace {

using fhip::I8Epilogue;
using fhip::clamp_round_i8;
using fhip::requant_i8;
using fhip::requant_i8_fast;
using fhip::requant_i8_split;

typedef int v4i __attribute__((ext_vector_type(4)));

#pragma clang fp contract(off)

// ---- INT8 GEMM: A [m][k] int8 row-major, B prepared [Np][Kp] ---------------------------------
// Block tile (16*FM) x (16*FN).  The NW waves split K: wave w takes the 64-deep steps w, w+NW, ...,
// issues the loads of UNR steps before their MFMAs (one memory round trip per UNR*NW steps), and the
// NW partial tiles are summed through LDS; integer sums are exact in any order.
// MFMA depth 64: lane l supplies row/col l%16 and bytes [16*(l/16), 16*(l/16)+16) of the step.
constexpr int kI8Unroll = 4;
// fhip_i8_linear runs the tile GEMM (i8_gemm_tile.hip) from kI8TileMinRows activation rows on, and from
// kI8TileMinRowsLarge rows when the product holds at least kI8TileMinMacs multiply-adds (measured crossovers:
// the K-split kernel wins below ~384 rows at 1024 x 1024, below ~150 at 4096 x 4096, above 64 nowhere at
// 3584 x 18944).
constexpr int64_t kI8TileMinRows = 384;
constexpr int64_t kI8TileMinRowsLarge = 64;
constexpr double kI8TileMinMacs = 2.5e9;

template <int FM, int FN, int NW = 4, int UNR = kI8Unroll>
__global__ __launch_bounds__(NW * 64) void i8_gemm_kernel(const int8_t* __restrict__ a, int64_t m, int64_t k,
                                                      const int8_t* __restrict__ b, int64_t kp, int64_t n,
                                                      I8Epilogue ep) {
    constexpr int TM = 16 * FM, TN = 16 * FN;
    constexpr int NT = NW * 64;
    __shared__ int32_t red[NW][TM][TN + 1];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t row_base = (int64_t)blockIdx.y * TM;
    const int64_t col_base = (int64_t)blockIdx.x * TN;
    const int fr = lane & 15;
    const int fk = (lane >> 4) * 16;
    const int8_t* arow[FM];
    bool arow_ok[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int64_t row = row_base + i * 16 + fr;
        arow_ok[i] = row < m;
        arow[i] = a + (arow_ok[i] ? row : 0) * k + fk;
    }
    const int8_t* bcol[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) bcol[j] = b + (col_base + j * 16 + fr) * kp + fk;  // rows padded to 256
    // Every output element this thread finishes lies in column col_base + tid % TN (NT % TN == 0), so its
    // channel parameters are loaded here, overlapping the main loop, instead of once per element.
    static_assert(NT % TN == 0, "epilogue column per thread");
    const int64_t my_col = col_base + (threadIdx.x % TN);
    const I8Epilogue::Col my_params = ep.col_params(my_col < n ? my_col : n - 1);
    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    const int64_t steps = (k + 63) / 64;
    for (int64_t s0 = wave; s0 < steps; s0 += NW * UNR) {
        v4i af[UNR][FM], bf[UNR][FN];
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
            const int64_t s = s0 + NW * u;
            const int64_t k0 = s * 64;
            const bool live = s < steps;
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                uint4 v = make_uint4(0, 0, 0, 0);
                if (live && arow_ok[i] && k0 + fk < k) v = *reinterpret_cast<const uint4*>(arow[i] + k0);
                af[u][i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                uint4 v = make_uint4(0, 0, 0, 0);
                if (live) v = *reinterpret_cast<const uint4*>(bcol[j] + k0);  // zero-padded past k
                bf[u][j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
        }
#pragma unroll
        for (int u = 0; u < UNR; ++u)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[u][i], bf[u][j], acc[i][j], 0, 0, 0);
    }
    // C fragment of lane l: column l%16, rows 4*(l/16) .. +3.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][i * 16 + (lane >> 4) * 4 + r][j * 16 + fr] = acc[i][j][r];
    __syncthreads();
    for (int e = threadIdx.x; e < TM * TN; e += NT) {
        const int rr = e / TN, cc = e % TN;
        const int64_t row = row_base + rr, col = col_base + cc;
        if (row >= m || col >= n) continue;
        int32_t raw = red[0][rr][cc];
#pragma unroll
        for (int q = 1; q < NW; ++q) raw += red[q][rr][cc];
        ep.store(raw, row, col, my_params);
    }
}

// ---- INT8 Conv2D implicit GEMM ------------------------------------------------------------------
// GEMM view per group g: rows = output pixels (b, oy, ox), cols = output channels of the group,
// K = icg*kh*kw in the weight's own (ci, ky, kx) order.  A fragments are gathered from the image.
struct ConvGeom {
    int64_t n, c, h, w, oh, ow, icg, kh, kw, ocg, k, kp;
    int32_t sh, sw, ph, pw, dh, dw;
    int layout;
    int8_t zp_in;
};

// One output pixel's input geometry, computed once per lane and fragment row (the host keeps n*oh*ow, h*w and
// the padded K below 2^31, so the splits are 32-bit).
struct ConvPix {
    bool live;
    int iy0, ix0;   // input coordinates of tap (0, 0)
    int64_t base;   // element offset of (b, first channel of the group, 0, 0)
};

__device__ __forceinline__ ConvPix conv_pix(const ConvGeom& g, int64_t pix, int group) {
    ConvPix p{false, 0, 0, 0};
    const int ohw = (int)(g.oh * g.ow);
    if (pix >= (int64_t)g.n * ohw) return p;
    const int q = (int)pix;
    const int b = q / ohw, rem = q - b * ohw;
    const int oy = rem / (int)g.ow, ox = rem - oy * (int)g.ow;
    p.live = true;
    p.iy0 = oy * g.sh - g.ph;
    p.ix0 = ox * g.sw - g.pw;
    const int64_t c0 = (int64_t)group * g.icg;
    p.base = g.layout == FHIP_NCHW ? ((int64_t)b * g.c + c0) * g.h * g.w : (int64_t)b * g.h * g.w * g.c + c0;
    return p;
}

// 16 consecutive K elements (weight order ci, ky, kx) of one pixel's implicit-GEMM row, from kk0.
__device__ __forceinline__ void conv_gather16(const int8_t* __restrict__ in, const ConvGeom& g, const ConvPix& p,
                                              int kk0, uint32_t* out4) {
    uint8_t bytes[16];
    const int kw = (int)g.kw, kh = (int)g.kh, khw = kh * kw, w = (int)g.w, h = (int)g.h, k = (int)g.k;
    int ci = kk0 / khw;
    const int r2 = kk0 - ci * khw;
    int ky = r2 / kw, kx = r2 - ky * kw;
    const int64_t plane = (int64_t)h * w;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        uint8_t v = 0;
        if (p.live && kk0 + i < k) {
            const int iy = p.iy0 + ky * (int)g.dh;
            const int ix = p.ix0 + kx * (int)g.dw;
            v = (uint8_t)g.zp_in;
            if (iy >= 0 && iy < h && ix >= 0 && ix < w) {
                const int64_t off = g.layout == FHIP_NCHW ? p.base + ci * plane + (int64_t)(iy * w + ix)
                                                          : p.base + (int64_t)(iy * w + ix) * g.c + ci;
                v = (uint8_t)in[off];
            }
        }
        bytes[i] = v;
        if (++kx == kw) {
            kx = 0;
            if (++ky == kh) {
                ky = 0;
                ++ci;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        out4[i] = (uint32_t)bytes[4 * i] | ((uint32_t)bytes[4 * i + 1] << 8) | ((uint32_t)bytes[4 * i + 2] << 16) |
                  ((uint32_t)bytes[4 * i + 3] << 24);
}

template <int WM, int WN>
__global__ __launch_bounds__(256) void i8_conv_kernel(const int8_t* __restrict__ in, ConvGeom g,
                                                      const int8_t* __restrict__ wt, const int32_t* __restrict__ bias,
                                                      I8Epilogue ep) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int group = blockIdx.z;
    const int64_t np = g.n * g.oh * g.ow;
    const int64_t oc_base = (int64_t)blockIdx.x * (32 * WN) + (wave & 1) * (16 * WN);  // within the group
    const int fr = lane & 15;
    const int fk = (lane >> 4) * 16;
    // pixel tiles of 32*WM rows, grid-strided over y (the grid's y extent is capped at 65535)
    const int64_t tiles_y = (np + 32 * WM - 1) / (32 * WM);
    for (int64_t ty = blockIdx.y; ty < tiles_y; ty += gridDim.y) {
        const int64_t pix_base = ty * (32 * WM) + (wave >> 1) * (16 * WM);
        v4i acc[WM][WN];
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j) acc[i][j] = v4i{0, 0, 0, 0};
        ConvPix px[WM];
#pragma unroll
        for (int i = 0; i < WM; ++i) px[i] = conv_pix(g, pix_base + i * 16 + fr, group);
        for (int k0 = 0; k0 < (int)g.k; k0 += 64) {
            v4i af[WM], bf[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                uint32_t v[4];
                conv_gather16(in, g, px[i], k0 + fk, v);
                af[i] = v4i{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                int64_t oc = oc_base + j * 16 + fr;
                oc = oc < g.ocg ? group * g.ocg + oc : 0;  // rows past the group read channel 0, never stored
                const uint4 v = *reinterpret_cast<const uint4*>(wt + oc * g.kp + k0 + fk);
                bf[j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int64_t ocl = oc_base + j * 16 + fr;
                if (ocl >= g.ocg) continue;
                const int64_t oc = group * g.ocg + ocl;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t pix = pix_base + i * 16 + (lane >> 4) * 4 + r;
                    if (pix >= np) continue;
                    const int ohw = (int)(g.oh * g.ow), q = (int)pix;  // np < 2^31 (host-checked)
                    const int64_t b = q / ohw;
                    const int rem = q - (int)b * ohw;
                    const int64_t oy = rem / (int)g.ow, ox = rem - (int)oy * (int)g.ow;
                    const int32_t dot = acc[i][j][r] - (int32_t)g.zp_in * ep.wsum[oc];
                    const int32_t total = dot + (bias ? bias[oc] : 0);
                    const double real = (double)total * ((double)ep.s_a * (double)ep.w_scales[oc]);
                    const int64_t off = g.layout == FHIP_NCHW ? ((b * (g.ocg * gridDim.z) + oc) * g.oh + oy) * g.ow + ox
                                                              : ((b * g.oh + oy) * g.ow + ox) * (g.ocg * gridDim.z) + oc;
                    ep.out[off] = requant_i8(real, ep.inv_out_den, ep.recip_out, ep.zp_out);
                }
            }
    }
}

// ---- INT8 Conv2D with one input channel per group (depthwise, channel multiplier ocg) -------------------
// Direct: a thread per output element sums its kh*kw taps in int32 over the in-image positions (padding taps
// are skipped, as the reference skips them: src/kernel/common/conv2d.cc:482-581), adds the bias and
// requantizes like the other kernels.  Consecutive threads take consecutive output x (NCHW) or channels
// (NHWC), so the output is written coalesced; the few input bytes per output come through the caches.
// The host keeps the output element count below 2^31 (32-bit index splits).
__global__ __launch_bounds__(256) void i8_conv_dw_kernel(const int8_t* __restrict__ in, ConvGeom g,
                                                         const int8_t* __restrict__ wt,
                                                         const int32_t* __restrict__ bias, I8Epilogue ep,
                                                         int oc_total) {
    const int ow = (int)g.ow, oh = (int)g.oh, w = (int)g.w, h = (int)g.h, kw = (int)g.kw, kh = (int)g.kh;
    const int ocg = (int)g.ocg;
    const int total = (int)g.n * oc_total * oh * ow;
    for (int e = blockIdx.x * 256 + threadIdx.x; e < total; e += gridDim.x * 256) {
        int b, oc, oy, ox, t;
        if (g.layout == FHIP_NCHW) {
            ox = e % ow;
            t = e / ow;
            oy = t % oh;
            t /= oh;
            oc = t % oc_total;
            b = t / oc_total;
        } else {
            oc = e % oc_total;
            t = e / oc_total;
            ox = t % ow;
            t /= ow;
            oy = t % oh;
            b = t / oh;
        }
        const int ci = oc / ocg;  // the group's one input channel
        const int8_t* wrow = wt + (int64_t)oc * g.kp;
        const int iy0 = oy * g.sh - g.ph, ix0 = ox * g.sw - g.pw;
        int32_t acc = 0;
        for (int ky = 0; ky < kh; ++ky) {
            const int iy = iy0 + ky * g.dh;
            if (iy < 0 || iy >= h) continue;
            for (int kx = 0; kx < kw; ++kx) {
                const int ix = ix0 + kx * g.dw;
                if (ix < 0 || ix >= w) continue;
                const int64_t off = g.layout == FHIP_NCHW ? (((int64_t)b * g.c + ci) * h + iy) * w + ix
                                                          : (((int64_t)b * h + iy) * w + ix) * g.c + ci;
                acc += ((int32_t)in[off] - (int32_t)g.zp_in) * (int32_t)wrow[ky * kw + kx];
            }
        }
        const int32_t sum = acc + (bias ? bias[oc] : 0);
        const double real = (double)sum * ((double)ep.s_a * (double)ep.w_scales[oc]);
        ep.out[e] = requant_i8(real, ep.inv_out_den, ep.recip_out, ep.zp_out);
    }
}

// ---- INT8 Conv2D, LDS-window implicit GEMM (group 1, IC a multiple of 64) -----------------------
// A block owns kConvTox consecutive output x positions of one output row (b, oy) and 64*WNF output
// channels per wave.  For each 64-channel chunk it stages the input window the row segment needs --
// KH rows x WX columns x 64 channels, channel-last, out-of-image taps filled with zp_in -- into LDS.
// Every A fragment (16 pixels x 16 channels of one tap) is then a single ds_read_b128; the weight is
// the tap-major copy [OC][KH*KW][IC], so a B fragment is one 16-byte load.  K runs over
// (chunk, ky, kx, 64 channels) with v_mfma_i32_16x16x64_i8; integer accumulation is exact, so the
// order differs from the reference's (ci, ky, kx) order without changing any sum.
constexpr int kConvTox = 32;
constexpr int kConvFrags = kConvTox / 16;  // 16-pixel A fragments per block
constexpr int kConvPitch = 80;  // 64 channels + 16 bytes: stride-2 fragment reads spread over banks
// NCHW fast staging: a thread covers kWinCols window columns of 4 channels, kWinSpan aligned dwords per
// channel (the columns plus up to 3 bytes of alignment shift); windows up to 4 * kWinCols = 80 columns.
constexpr int kWinCols = 20;
constexpr int kWinSpan = kWinCols / 4 + 1;
// NCHW 16-byte staging: the window is widened to whole aligned 16-byte chunks of each input row (at most
// kWinChunks), so a thread loads 4 channels x one chunk with four 16-byte loads; rows a multiple of 16 bytes
// make every chunk either wholly inside the row or wholly padding.
constexpr int kWinChunks = 5;
__host__ __device__ constexpr int conv_chunks(int wx) { return (wx + 15 + 15) / 16; }

// STG = 1: compiled for the 16-byte NCHW staging path only (the host checks its conditions).  A launch
// is latency-bound and starts with a cold instruction cache, so code the shape never runs still costs:
// on C4 the 16-byte-only kernel spans 5.1 us in-kernel against 5.6 us for the general one.
template <int WNF, int TAPS, int STG = 0>
__global__ __launch_bounds__(256) void i8_conv_window_kernel(const int8_t* __restrict__ in, ConvGeom g,
                                                             const int8_t* __restrict__ wt,
                                                             const int32_t* __restrict__ bias, I8Epilogue ep,
                                                             int64_t oc_total) {
    extern __shared__ __align__(16) uint8_t win[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t ox0 = (int64_t)blockIdx.x * kConvTox;
    // 32-bit: the grid's y extent is n * oh < 2^31 (a 64-bit division is a long scalar sequence)
    const int64_t b = (int)blockIdx.y / (int)g.oh, oy = (int)blockIdx.y % (int)g.oh;
    const int64_t oc_base = (int64_t)blockIdx.z * (4 * WNF * 16) + wave * (WNF * 16);
    const int wx = (kConvTox - 1) * g.sw + (int)((g.kw - 1) * g.dw) + 1;
    const int64_t taps = g.kh * g.kw;
    const int kq = (lane >> 4) * 16;  // channel quarter of this lane's fragment
    v4i acc[kConvFrags][WNF];
#pragma unroll
    for (int f = 0; f < kConvFrags; ++f)
#pragma unroll
        for (int j = 0; j < WNF; ++j) acc[f][j] = v4i{0, 0, 0, 0};

    auto load_b = [&](int64_t tap, int64_t c0, v4i (&bf)[WNF]) {
#pragma unroll
        for (int j = 0; j < WNF; ++j) {
            int64_t oc = oc_base + j * 16 + (lane & 15);
            oc = oc < oc_total ? oc : oc_total - 1;  // clamped rows are computed, never stored
            const uint4 v = *reinterpret_cast<const uint4*>(wt + (oc * taps + tap) * g.c + c0 + kq);
            bf[j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        }
    };
    // Epilogue parameters (per-channel scale, weight sum, bias) are requested before anything else.
    float e_scale[WNF];
    int32_t e_wsum[WNF], e_bias[WNF];
#pragma unroll
    for (int j = 0; j < WNF; ++j) {
        int64_t oc = oc_base + j * 16 + (lane & 15);
        oc = oc < oc_total ? oc : oc_total - 1;
        e_scale[j] = ep.w_scales[oc];
        e_wsum[j] = ep.wsum[oc];
        e_bias[j] = bias ? bias[oc] : 0;
    }
    const int ix0 = (int)(ox0 * g.sw - g.pw);
    const uint8_t zp = (uint8_t)g.zp_in;
    // NCHW 16-byte path: rows a multiple of 16 bytes, 16-byte aligned input, kh * 16 * chunks threads.
    const int chunks = conv_chunks(wx);
    const bool vec_rows = STG == 1 || (g.layout == FHIP_NCHW && (g.w & 15) == 0 &&
                                       (reinterpret_cast<uintptr_t>(in) & 15) == 0 && chunks <= kWinChunks &&
                                       g.kh * 16 * chunks <= 256);
    // window row length in LDS and the column of the first window byte in it
    const int wrow = vec_rows ? 16 * chunks : wx;
    const int a0 = ix0 >= 0 ? ix0 & ~15 : -((-ix0 + 15) & ~15);  // floor to a multiple of 16
    const int xsh = vec_rows ? ix0 - a0 : 0;
    // NCHW dword path: rows 4-byte aligned, at most 4 tap rows, a window of at most 80 columns.
    const bool dword_rows = STG != 1 && !vec_rows && g.layout == FHIP_NCHW && (g.w & 3) == 0 &&
                            (reinterpret_cast<uintptr_t>(in) & 3) == 0 && wx <= 4 * kWinCols && g.kh * 64 <= 256;
    for (int64_t c0 = 0; c0 < g.c; c0 += 64) {
        // 1. issue this thread's window loads (fast path), then every tap's weight fragments; nothing
        //    waits until the LDS writes below, so all of them are in flight together
        // thread t: tap row ky = t / 64, channels 4*cq .. 4*cq+3 with cq = (t / 4) % 16, window columns
        // [20*xq, 20*xq + 20) with xq = t % 4; per channel the columns come as kWinSpan aligned dwords
        uint32_t d[4][kWinSpan];
        uint4 q16[4];
        int sh = 0;
        // 16-byte path: thread t = (ky * 16 + cq) * chunks + xq loads chunk xq (columns a0 + 16 xq ..) of
        // channels 4 cq .. 4 cq + 3 of tap row ky; consecutive lanes read consecutive chunks of a row
        if (vec_rows && tid < g.kh * 16 * chunks) {
            const int xq = tid % chunks, cq = (tid / chunks) & 15, ky = tid / (16 * chunks);
            const int iy = (int)(oy * g.sh - g.ph) + ky * (int)g.dh;
            const int gx = a0 + 16 * xq;
            const bool live = iy >= 0 && iy < (int)g.h && gx >= 0 && gx < (int)g.w;
            const uint32_t z = (uint32_t)zp * 0x01010101u;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int8_t* src = in + ((b * g.c + c0 + 4 * cq + c) * g.h + (live ? iy : 0)) * g.w + (live ? gx : 0);
                q16[c] = live ? *reinterpret_cast<const uint4*>(src) : make_uint4(z, z, z, z);
            }
        }
        if (dword_rows) {
            const int ky = tid >> 6, cq = (tid >> 2) & 15, xq = tid & 3;
            const int iy = (int)(oy * g.sh - g.ph) + ky * (int)g.dh;
            const bool row_live = tid < g.kh * 64 && iy >= 0 && iy < (int)g.h;
            const int gx = ix0 + xq * kWinCols;       // first input column of this thread
            const int a0 = gx & ~3;                   // floor to a multiple of 4 (two's complement)
            sh = gx - a0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint8_t* row = reinterpret_cast<const uint8_t*>(in) +
                                     ((b * g.c + c0 + (row_live ? 4 * cq + c : 0)) * g.h + (row_live ? iy : 0)) * g.w;
#pragma unroll
                for (int i = 0; i < kWinSpan; ++i) {
                    const int off = a0 + 4 * i;
                    // a dword is either inside the row or entirely padding (rows are 4-byte aligned);
                    // padding dwords read the row's first dword and are replaced below
                    const bool in_row = off >= 0 && off < (int)g.w;
                    d[c][i] = *reinterpret_cast<const uint32_t*>(row + (in_row ? off : 0));
                    if (!(in_row && row_live)) d[c][i] = (uint32_t)zp * 0x01010101u;
                }
            }
        }
        v4i bpre[TAPS > 0 ? TAPS : 1][WNF];
        if constexpr (TAPS > 0) {
#pragma unroll
            for (int t = 0; t < TAPS; ++t) load_b(t, c0, bpre[t]);
        }
        // 2. the previous chunk's taps must be done with the window before it is overwritten
        if (c0 > 0) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
        }
        // 3. stage the window (channel-last in LDS)
        if (vec_rows) {
            if (tid < g.kh * 16 * chunks) {
                const int xq = tid % chunks, cq = (tid / chunks) & 15, ky = tid / (16 * chunks);
                uint8_t* dst = win + (ky * wrow + 16 * xq) * kConvPitch + 4 * cq;
                const uint32_t w4[4][4] = {{q16[0].x, q16[0].y, q16[0].z, q16[0].w},
                                           {q16[1].x, q16[1].y, q16[1].z, q16[1].w},
                                           {q16[2].x, q16[2].y, q16[2].z, q16[2].w},
                                           {q16[3].x, q16[3].y, q16[3].z, q16[3].w}};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // w4[c][i] holds columns 4i .. 4i+3 of channel c: transpose to one dword (4 channels) per column
                    const uint32_t lo01 = __builtin_amdgcn_perm(w4[1][i], w4[0][i], 0x05010400u);
                    const uint32_t hi01 = __builtin_amdgcn_perm(w4[1][i], w4[0][i], 0x07030602u);
                    const uint32_t lo23 = __builtin_amdgcn_perm(w4[3][i], w4[2][i], 0x05010400u);
                    const uint32_t hi23 = __builtin_amdgcn_perm(w4[3][i], w4[2][i], 0x07030602u);
                    const uint32_t col[4] = {__builtin_amdgcn_perm(lo23, lo01, 0x05040100u),
                                             __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                                             __builtin_amdgcn_perm(hi23, hi01, 0x05040100u),
                                             __builtin_amdgcn_perm(hi23, hi01, 0x07060302u)};
#pragma unroll
                    for (int u = 0; u < 4; ++u) *reinterpret_cast<uint32_t*>(dst + (4 * i + u) * kConvPitch) = col[u];
                }
            }
        } else if (dword_rows) {
            if (tid < g.kh * 64) {
                const int ky = tid >> 6, cq = (tid >> 2) & 15, x0 = (tid & 3) * kWinCols;
                uint8_t* dst = win + (ky * wx + x0) * kConvPitch + 4 * cq;
#pragma unroll
                for (int i = 0; i < kWinCols / 4; ++i) {
                    // e[c] holds columns x0+4i .. +3 of channel c; a 4x4 byte transpose gives, per column,
                    // the four channels as one dword (v_perm_b32: bytes 0-3 = second operand)
                    uint32_t e[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) e[c] = __builtin_amdgcn_alignbyte(d[c][i + 1], d[c][i], (uint32_t)sh);
                    const uint32_t lo01 = __builtin_amdgcn_perm(e[1], e[0], 0x05010400u);
                    const uint32_t hi01 = __builtin_amdgcn_perm(e[1], e[0], 0x07030602u);
                    const uint32_t lo23 = __builtin_amdgcn_perm(e[3], e[2], 0x05010400u);
                    const uint32_t hi23 = __builtin_amdgcn_perm(e[3], e[2], 0x07030602u);
                    const uint32_t col[4] = {__builtin_amdgcn_perm(lo23, lo01, 0x05040100u),
                                             __builtin_amdgcn_perm(lo23, lo01, 0x07060302u),
                                             __builtin_amdgcn_perm(hi23, hi01, 0x05040100u),
                                             __builtin_amdgcn_perm(hi23, hi01, 0x07060302u)};
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (x0 + 4 * i + u < wx) *reinterpret_cast<uint32_t*>(dst + (4 * i + u) * kConvPitch) = col[u];
                }
            }
        } else if (g.layout == FHIP_NCHW) {
            // byte path: thread (ky, ci) copies one input row segment, transposed to channel-last
            const bool interior = ix0 >= 0 && ix0 + wx <= (int)g.w;  // block-uniform
            for (int r = tid; r < (int)g.kh * 64; r += 256) {
                const int ci = r & 63, ky = r >> 6;
                const int iy = (int)(oy * g.sh - g.ph) + ky * (int)g.dh;
                uint8_t* dst = win + ky * wx * kConvPitch + ci;
                if (iy < 0 || iy >= (int)g.h) {
                    for (int x = 0; x < wx; ++x) dst[x * kConvPitch] = zp;
                    continue;
                }
                const uint8_t* row = reinterpret_cast<const uint8_t*>(in) + ((b * g.c + c0 + ci) * g.h + iy) * g.w;
                if (interior) {
                    const uint8_t* src = row + ix0;
                    int x = 0;
                    for (; x + 8 <= wx; x += 8) {
                        uint8_t v[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) v[u] = src[x + u];
#pragma unroll
                        for (int u = 0; u < 8; ++u) dst[(x + u) * kConvPitch] = v[u];
                    }
                    for (; x < wx; ++x) dst[x * kConvPitch] = src[x];
                } else {
                    const int wlast = (int)g.w - 1;
                    int x = 0;
                    for (; x + 8 <= wx; x += 8) {
                        uint8_t v[8];
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            const int ix = ix0 + x + u;
                            const uint8_t t = row[ix < 0 ? 0 : (ix > wlast ? wlast : ix)];
                            v[u] = (ix >= 0 && ix <= wlast) ? t : zp;
                        }
#pragma unroll
                        for (int u = 0; u < 8; ++u) dst[(x + u) * kConvPitch] = v[u];
                    }
                    for (; x < wx; ++x) {
                        const int ix = ix0 + x;
                        dst[x * kConvPitch] = (ix >= 0 && ix <= wlast) ? row[ix] : zp;
                    }
                }
            }
        } else {
            const int total = (int)g.kh * wx * 4;  // 16-byte quarters
            for (int idx = tid; idx < total; idx += 256) {
                const int q = idx & 3, t = idx >> 2;
                const int x = t % wx, ky = t / wx;
                const int64_t iy = oy * g.sh - g.ph + ky * g.dh;
                const int64_t ix = ox0 * g.sw - g.pw + x;
                uint4 v;
                const uint32_t z = (uint32_t)(uint8_t)g.zp_in * 0x01010101u;
                if (iy >= 0 && iy < g.h && ix >= 0 && ix < g.w)
                    v = *reinterpret_cast<const uint4*>(in + ((b * g.h + iy) * g.w + ix) * g.c + c0 + q * 16);
                else
                    v = make_uint4(z, z, z, z);
                *reinterpret_cast<uint4*>(win + (ky * wx + x) * kConvPitch + q * 16) = v;
            }
        }
        __syncthreads();
        auto tap_step = [&](int64_t ky, int64_t kx, const v4i (&bf)[WNF]) {
            v4i af[kConvFrags];
#pragma unroll
            for (int f = 0; f < kConvFrags; ++f) {
                const int p = f * 16 + (lane & 15);
                const int x = p * g.sw + (int)(kx * g.dw);
                const uint4 v = *reinterpret_cast<const uint4*>(win + (ky * wrow + x + xsh) * kConvPitch + kq);
                af[f] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
#pragma unroll
            for (int f = 0; f < kConvFrags; ++f)
#pragma unroll
                for (int j = 0; j < WNF; ++j)
                    acc[f][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[f], bf[j], acc[f][j], 0, 0, 0);
        };
        if constexpr (TAPS > 0) {
            // tap t = ky * kw + kx, stepped incrementally (kw is a kernel argument: no division per tap)
            int ky = 0, kx = 0;
            const int kw = (int)g.kw;
#pragma unroll
            for (int t = 0; t < TAPS; ++t) {
                tap_step(ky, kx, bpre[t]);
                if (++kx == kw) {
                    kx = 0;
                    ++ky;
                }
            }
        } else {
            for (int64_t ky = 0; ky < g.kh; ++ky)
                for (int64_t kx = 0; kx < g.kw; ++kx) {
                    v4i bf[WNF];
                    load_b(ky * g.kw + kx, c0, bf);
                    tap_step(ky, kx, bf);
                }
        }
    }
    // C fragment of lane l: channel l%16, pixels 4*(l/16) .. +3 (consecutive output x).
    // Requantize every value on the integer path (requant_i8_split: acc + shift is the exact int32 sum,
    // K = s_in * s_w / s_out a float pair per channel); values it cannot decide (x.5 points) are redone
    // with the reference's fp64 division in one cold branch, so the hot tail holds no per-value branch.
    int8_t qv[kConvFrags][WNF][4];
    uint32_t ties = 0;
    float kh[WNF], kl[WNF];
    int32_t shift[WNF];
#pragma unroll
    for (int j = 0; j < WNF; ++j) {
        ep.split_scale(e_scale[j], kh[j], kl[j]);
        shift[j] = e_bias[j] - (int32_t)g.zp_in * e_wsum[j];
    }
    const int32_t zp_out_i = (int32_t)ep.zp_out;
#pragma unroll
    for (int f = 0; f < kConvFrags; ++f)
#pragma unroll
        for (int j = 0; j < WNF; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                bool tie;
                qv[f][j][r] = requant_i8_split(acc[f][j][r] + shift[j], kh[j], kl[j], zp_out_i, tie);
                ties |= (uint32_t)tie << ((f * WNF + j) * 4 + r);
            }
        }
    if (__builtin_expect(ties != 0, 0)) {
#pragma unroll
        for (int f = 0; f < kConvFrags; ++f)
#pragma unroll
            for (int j = 0; j < WNF; ++j) {
                const double scale = (double)ep.s_a * (double)e_scale[j];
                const int32_t shift = e_bias[j] - (int32_t)g.zp_in * e_wsum[j];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if ((ties >> ((f * WNF + j) * 4 + r)) & 1u)
                        qv[f][j][r] = clamp_round_i8((double)(acc[f][j][r] + shift) * scale / ep.inv_out_den + ep.zp_out);
            }
    }
#pragma unroll
    for (int f = 0; f < kConvFrags; ++f)
#pragma unroll
        for (int j = 0; j < WNF; ++j) {
            const int64_t oc = oc_base + j * 16 + (lane & 15);
            if (oc >= oc_total) continue;
            const int8_t (&q)[4] = qv[f][j];
            const uint32_t packed = (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) |
                                    ((uint32_t)(uint8_t)q[2] << 16) | ((uint32_t)(uint8_t)q[3] << 24);
            const int64_t ox = ox0 + f * 16 + (lane >> 4) * 4;
            if (STG == 1 || g.layout == FHIP_NCHW) {
                int8_t* dst = ep.out + ((b * oc_total + oc) * g.oh + oy) * g.ow + ox;
                if (ox + 3 < g.ow && ((reinterpret_cast<uintptr_t>(dst) & 3) == 0)) {
                    *reinterpret_cast<uint32_t*>(dst) = packed;
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (ox + r < g.ow) dst[r] = q[r];
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (ox + r < g.ow) ep.out[((b * g.oh + oy) * g.ow + ox + r) * oc_total + oc] = q[r];
            }
        }
}

// ---- QuantizeLinear / DequantizeLinear ---------------------------------------------------------
constexpr int kInlineChannels = 128;
struct QParams {
    float scale[kInlineChannels];
    int32_t zp[kInlineChannels];
};

__device__ __forceinline__ float read_float(const void* src, int dtype, int64_t i) {
    if (dtype == FHIP_FP32) return static_cast<const float*>(src)[i];
    if (dtype == FHIP_BF16) return fhip::bf16_decode(static_cast<const uint16_t*>(src)[i]);
    return fhip::fp16_decode(static_cast<const uint16_t*>(src)[i]);
}

// Parameters either inline (channels <= kInlineChannels) or from device arrays.
__global__ void quantize_kernel(const void* __restrict__ src, int src_dtype, int64_t count, int64_t channels,
                                int64_t inner, QParams inline_params, const float* __restrict__ scales,
                                const int32_t* __restrict__ zps, int per_channel_zp, int8_t* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t p = channels == 1 ? 0 : (i / inner) % channels;
        const int64_t pz = per_channel_zp ? p : 0;
        const float s = scales ? scales[p] : inline_params.scale[p];
        const int32_t z = zps ? zps[pz] : inline_params.zp[pz];
        const double t = (double)read_float(src, src_dtype, i) / (double)s + (double)z;
        out[i] = clamp_round_i8(t);
    }
}

// Per-tensor QuantizeLinear (one scale, one zero point; the C1 activation): the source type is a template
// parameter and the division x / s becomes requant_i8's multiply by 1/s with the exact division near an x.5
// point, which yields the same clamp(round_away(double(x) / double(s) + zp)) -- also for NaN and Inf, whose
// t is NaN and so takes the division.  No per-channel index arithmetic is compiled in.
template <int SRC>
__global__ void quantize_tensor_kernel(const void* __restrict__ src, int64_t count, float scale, int32_t zp,
                                       int8_t* __restrict__ out) {
    const double s = scale, r = 1.0 / s, z = zp;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = requant_i8((double)read_float(src, SRC, i), s, r, z);
}

__global__ void dequantize_kernel(const int8_t* __restrict__ src, int64_t count, int64_t channels, int64_t inner,
                                  QParams inline_params, const float* __restrict__ scales,
                                  const int32_t* __restrict__ zps, int per_channel_zp, int dst_dtype, void* out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t p = channels == 1 ? 0 : (i / inner) % channels;
        const int64_t pz = per_channel_zp ? p : 0;
        const float s = scales ? scales[p] : inline_params.scale[p];
        const int32_t z = zps ? zps[pz] : inline_params.zp[pz];
        const float v = (float)((int32_t)src[i] - z) * s;
        if (dst_dtype == FHIP_FP32) static_cast<float*>(out)[i] = v;
        else if (dst_dtype == FHIP_FP16) static_cast<uint16_t*>(out)[i] = fhip::fp16_encode(v);
        else static_cast<uint16_t*>(out)[i] = fhip::bf16_encode_plain(v);
    }
}

unsigned grid_for(int64_t count, int threads) {
    int64_t blocks = (count + threads - 1) / threads;
    if (blocks > 65536) blocks = 65536;
    return (unsigned)(blocks < 1 ? 1 : blocks);
}

// Host bound: every partial sum of (a - zp_a)*(w - zp_w) and of the device-side terms stays
// within int32, and the requantized value is finite.
bool int32_safe(int64_t k, int32_t zp_a, int32_t max_abs_w, int64_t bias_abs) {
    const double amax = 128.0 + (zp_a < 0 ? -zp_a : zp_a);
    const double bound = (double)k * amax * (double)max_abs_w + (double)bias_abs;
    return bound < 2147483647.0;
}

int upload_params(fhip_context ctx, int64_t channels, const float* scales, const int32_t* zps, int64_t n_zp,
                  QParams* inline_params, const float** dscales, const int32_t** dzps) {
    *dscales = nullptr;
    *dzps = nullptr;
    if (channels <= kInlineChannels) {
        for (int64_t i = 0; i < channels; ++i) inline_params->scale[i] = scales[i];
        for (int64_t i = 0; i < n_zp; ++i) inline_params->zp[i] = zps[i];
        return FHIP_OK;
    }
    if (ctx->capturing)
        return fhip::set_error(ctx, FHIP_ERR_STATE, "per-channel parameters beyond 128 channels cannot be captured");
    void* ws = nullptr;
    int rc = fhip::acquire_workspace(ctx, (size_t)(channels * 4 + n_zp * 4), &ws);
    if (rc != FHIP_OK) return rc;
    rc = fhip::check_hip(ctx, hipStreamSynchronize(ctx->stream), "sync before parameter upload");
    if (rc == FHIP_OK) rc = fhip::check_hip(ctx, hipMemcpy(ws, scales, channels * 4, hipMemcpyHostToDevice), "upload scales");
    if (rc == FHIP_OK)
        rc = fhip::check_hip(ctx, hipMemcpy(static_cast<char*>(ws) + channels * 4, zps, n_zp * 4, hipMemcpyHostToDevice),
                             "upload zero points");
    *dscales = static_cast<const float*>(ws);
    *dzps = reinterpret_cast<const int32_t*>(static_cast<char*>(ws) + channels * 4);
    return rc;
}

int validate_qparams(fhip_context ctx, int64_t channels, const float* scales, const int32_t* zps, int64_t n_zp) {
    if (channels <= 0 || !scales || !zps || (n_zp != 1 && n_zp != channels))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "quantization parameters do not match the channel count");
    for (int64_t i = 0; i < channels; ++i)
        if (!fhip::valid_scale(scales[i])) return fhip::set_error(ctx, FHIP_ERR_INVALID, "invalid quantization scale");
    for (int64_t i = 0; i < n_zp; ++i)
        if (zps[i] < -128 || zps[i] > 127) return fhip::set_error(ctx, FHIP_ERR_INVALID, "zero point outside [-128, 127]");
    return FHIP_OK;
}

}  // namespace

extern "C" {

int fhip_i8_linear(fhip_context ctx, int kind, const int8_t* a, float s_a, int32_t zp_a, int64_t m, fhip_weight w,
                   const int32_t* bias, int bias_kind, int32_t bias_abs_max, float alpha, float beta, int8_t* out,
                   float s_out, int32_t zp_out) {
    return fhip_i8_linear_ex(ctx, kind, a, s_a, zp_a, m, w, bias, bias_kind, bias_abs_max, alpha, beta, FHIP_INT8, out,
                             s_out, zp_out, 1.0f, 0);
}

int fhip_i8_linear_ex(fhip_context ctx, int kind, const int8_t* a, float s_a, int32_t zp_a, int64_t m, fhip_weight w,
                      const int32_t* bias, int bias_kind, int32_t bias_abs_max, float alpha, float beta, int out_dtype,
                      void* out, float s_out, int32_t zp_out, float dq_scale, int32_t dq_zp) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (out_dtype != FHIP_INT8 && out_dtype != FHIP_FP32 && out_dtype != FHIP_FP16 && out_dtype != FHIP_BF16)
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_linear: out_dtype must be INT8, FP32, FP16 or BF16");
    if (out_dtype != FHIP_INT8 && (!fhip::valid_scale(dq_scale) || dq_zp < -128 || dq_zp > 127))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_linear: invalid DequantizeLinear parameters");
    if (m == 0) return FHIP_OK;  // no activation rows: the reference's loops run zero times
    if (!a || !w || !out || m < 0 || w->kind != kLinearWeight || w->dtype != FHIP_INT8 || kind < FHIP_I8_MATMUL ||
        kind > FHIP_I8_GEMM || bias_kind < FHIP_BIAS_NONE || bias_kind > FHIP_BIAS_MATRIX ||
        (bias_kind != FHIP_BIAS_NONE && !bias))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_linear: bad arguments");
    if (!fhip::valid_scale(s_a) || !fhip::valid_scale(s_out) || zp_a < -128 || zp_a > 127 || zp_out < -128 ||
        zp_out > 127 || (kind == FHIP_I8_GEMM && (!std::isfinite(alpha) || !std::isfinite(beta))))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_linear: invalid quantization parameters");
    if (kind == FHIP_I8_MATMUL) bias_kind = FHIP_BIAS_NONE;
    if (w->any_zp) return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_linear: weight zero points must be 0");
    if (w->k % 16 != 0) return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_linear: K % 16 != 0");
    const int64_t babs = bias_kind == FHIP_BIAS_NONE ? 0 : (bias_abs_max < 0 ? -(int64_t)bias_abs_max : bias_abs_max);
    if (!int32_safe(w->k, zp_a, w->max_abs_w, kind == FHIP_I8_FC ? babs : 0))
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_linear: int32 accumulator could overflow");
    const double real_bound = (std::fabs((double)alpha) + std::fabs((double)beta) + 1.0) * 4294967296.0 *
                              (double)s_a * (double)w->max_scale / (double)s_out;
    if (!(real_bound < 1e300)) return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_linear: scales too large");
    I8Epilogue ep{kind, w->scales, w->wsum, bias, bias_kind, zp_a, s_a, (double)alpha, (double)beta, (double)s_out,
                  (double)zp_out, 1.0 / (double)s_out, static_cast<int8_t*>(out), w->n};
    ep.out_dtype = out_dtype;
    ep.dq_scale = dq_scale;
    ep.dq_zp = dq_zp;
    ep.out_any = out;
    ep.int_path = kind != FHIP_I8_GEMM ||
                  (alpha == 1.0f && beta == 1.0f && int32_safe(w->k, zp_a, w->max_abs_w, babs));
    // Large M: the LDS-staged MFMA tile GEMM (operand reuse across a 128x128 or 256x256 tile).
    const bool tile_rows =
        m >= kI8TileMinRows || (m >= kI8TileMinRowsLarge && (double)m * (double)w->n * (double)w->k >= kI8TileMinMacs);
    // (its buffer resources address the activations and the prepared weight with 32-bit offsets)
    const int64_t tile_wbytes = ((w->n + 255) / 256 * 256) * ((w->k + 127) / 128 * 128);
    if (tile_rows && w->k % 64 == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0 &&
        m * w->k < (int64_t(1) << 31) && tile_wbytes < (int64_t(1) << 31))
        return fhip::launch_i8_gemm_tile(ctx, a, m, w, ep);
    const int64_t kp = ((w->k + 127) / 128) * 128;
    // largest tile that still puts about two blocks on every CU
    const int64_t blocks32 = ((w->n + 31) / 32) * ((m + 31) / 32);
    const int8_t* bw = static_cast<const int8_t*>(w->data);
    if (blocks32 >= 512) {
        dim3 grid((unsigned)((w->n + 31) / 32), (unsigned)((m + 31) / 32));
        i8_gemm_kernel<2, 2><<<grid, 256, 0, ctx->stream>>>(a, m, w->k, bw, kp, w->n, ep);
        ctx->last_backend = "i8_mfma_gemm_32x32_ksplit4";
    } else {
        dim3 grid((unsigned)((w->n + 31) / 32), (unsigned)((m + 15) / 16));
        i8_gemm_kernel<1, 2, 8, 2><<<grid, 512, 0, ctx->stream>>>(a, m, w->k, bw, kp, w->n, ep);
        ctx->last_backend = "i8_mfma_gemm_16x32_ksplit4";
    }
    FHIP_CHECK_LAUNCH(ctx, "i8_gemm_kernel");
    return FHIP_OK;
}

int fhip_i8_conv2d(fhip_context ctx, const int8_t* in, int64_t n, int64_t c, int64_t h, int64_t w, int layout,
                   float s_in, int32_t zp_in, fhip_weight wt, const int32_t* bias, int32_t bias_abs_max,
                   int32_t stride_h, int32_t stride_w, int32_t pad_h, int32_t pad_w, int32_t dil_h, int32_t dil_w,
                   int8_t* out, int64_t oh, int64_t ow, float s_out, int32_t zp_out) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (n == 0) return FHIP_OK;  // empty batch
    if (!in || !wt || !out || wt->kind != kConvWeight || n < 0 || c <= 0 || h <= 0 || w <= 0 || stride_h <= 0 ||
        stride_w <= 0 || dil_h <= 0 || dil_w <= 0 || pad_h < 0 || pad_w < 0 || (layout != FHIP_NCHW && layout != FHIP_NHWC))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_conv2d: bad arguments");
    if (c != wt->icg * wt->group) return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_conv2d: channels do not match");
    const int64_t eh = (h + 2 * pad_h - dil_h * (wt->kh - 1) - 1) / stride_h + 1;
    const int64_t ew = (w + 2 * pad_w - dil_w * (wt->kw - 1) - 1) / stride_w + 1;
    if (eh <= 0 || ew <= 0 || eh != oh || ew != ow) return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_conv2d: output shape");
    if (!fhip::valid_scale(s_in) || !fhip::valid_scale(s_out) || zp_in < -128 || zp_in > 127 || zp_out < -128 ||
        zp_out > 127)
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "i8_conv2d: invalid quantization parameters");
    if (wt->any_zp) return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_conv2d: weight zero points must be 0");
    const int64_t babs = bias ? (bias_abs_max < 0 ? -(int64_t)bias_abs_max : bias_abs_max) : 0;
    if (!int32_safe(wt->k, zp_in, wt->max_abs_w, babs))
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_conv2d: int32 accumulator could overflow");
    const double real_bound = 4294967296.0 * (double)s_in * (double)wt->max_scale / (double)s_out;
    if (!(real_bound < 1e300)) return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_conv2d: scales too large");
    ConvGeom g{n, c, h, w, oh, ow, wt->icg, wt->kh, wt->kw, wt->n / wt->group, wt->k, ((wt->k + 127) / 128) * 128,
               stride_h, stride_w, pad_h, pad_w, dil_h, dil_w, layout, (int8_t)zp_in};
    I8Epilogue ep{FHIP_I8_FC, wt->scales, wt->wsum, nullptr, FHIP_BIAS_NONE, zp_in, s_in, 1.0, 1.0, (double)s_out,
                  (double)zp_out, 1.0 / (double)s_out, out, 0};
    if (wt->tap_major && c % 64 == 0 && wt->group == 1 &&
        (layout == FHIP_NCHW || (reinterpret_cast<uintptr_t>(in) & 15) == 0)) {
        // 128 output channels per block (8 wave fragments) share each staged window across more channels,
        // 64 per block give twice the blocks: measured on C4 (240 blocks at 128 channels), 64 per block
        // runs 7.0 us against 7.7 us, so 128 is used only where its grid already holds two blocks per CU.
        const int64_t x_blocks = (ow + kConvTox - 1) / kConvTox;
        const int wnf = wt->n >= 128 && x_blocks * n * oh * ((wt->n + 127) / 128) >= 2 * (int64_t)ctx->cus ? 2 : 1;
        const int wx = (kConvTox - 1) * stride_w + (int)((wt->kw - 1) * dil_w) + 1;
        // room for the 16-byte path's widened window (the kernel picks the path; either fits)
        const size_t lds = (size_t)wt->kh * std::max(wx, 16 * conv_chunks(wx)) * kConvPitch;
        if (lds <= 64 * 1024) {
            const int64_t oc = wt->n;
            dim3 grid((unsigned)x_blocks, (unsigned)(n * oh),
                      (unsigned)((oc + 4 * wnf * 16 - 1) / (4 * wnf * 16)));
            const int8_t* tm = static_cast<const int8_t*>(wt->tap_major);
            const bool t9 = wt->kh * wt->kw == 9;
            // the kernel's 16-byte staging conditions (vec_rows), decided here to pick the specialized build
            const bool vec = layout == FHIP_NCHW && (w & 15) == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 &&
                             conv_chunks(wx) <= kWinChunks && wt->kh * 16 * conv_chunks(wx) <= 256;
            if (vec && wnf == 2 && t9) i8_conv_window_kernel<2, 9, 1><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            else if (vec && wnf == 2) i8_conv_window_kernel<2, 0, 1><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            else if (vec && t9) i8_conv_window_kernel<1, 9, 1><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            else if (vec) i8_conv_window_kernel<1, 0, 1><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            else if (wnf == 2 && t9) i8_conv_window_kernel<2, 9><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            else if (wnf == 2) i8_conv_window_kernel<2, 0><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            else if (t9) i8_conv_window_kernel<1, 9><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            else i8_conv_window_kernel<1, 0><<<grid, 256, lds, ctx->stream>>>(in, g, tm, bias, ep, oc);
            ctx->last_backend = "i8_mfma_conv_window";
            FHIP_CHECK_LAUNCH(ctx, "i8_conv_window_kernel");
            return FHIP_OK;
        }
    }
    if (wt->icg == 1 && n * wt->n * oh * ow < (int64_t(1) << 31) && h * w < (int64_t(1) << 31)) {
        const int64_t total = n * wt->n * oh * ow;
        const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
        i8_conv_dw_kernel<<<grid, 256, 0, ctx->stream>>>(in, g, static_cast<const int8_t*>(wt->data), bias, ep,
                                                         (int)wt->n);
        ctx->last_backend = "i8_conv_depthwise";
        FHIP_CHECK_LAUNCH(ctx, "i8_conv_dw_kernel");
        return FHIP_OK;
    }
    constexpr int WM = 2, WN = 2;
    const int64_t np = n * oh * ow;
    if (np >= (int64_t(1) << 31) || h * w >= (int64_t(1) << 31) || wt->group > 65535)
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "i8_conv2d: image too large for the gathered conv kernel");
    dim3 grid((unsigned)((g.ocg + 32 * WN - 1) / (32 * WN)),
              (unsigned)std::min<int64_t>((np + 32 * WM - 1) / (32 * WM), 65535), (unsigned)wt->group);
    i8_conv_kernel<WM, WN><<<grid, 256, 0, ctx->stream>>>(in, g, static_cast<const int8_t*>(wt->data), bias, ep);
    ctx->last_backend = "i8_mfma_conv_64x64";
    FHIP_CHECK_LAUNCH(ctx, "i8_conv_kernel");
    return FHIP_OK;
}

int fhip_quantize_linear(fhip_context ctx, int src_dtype, const void* src, int64_t count, int64_t channels,
                         int64_t inner, const float* scales, const int32_t* zero_points, int64_t n_zp, int8_t* out) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (count == 0) return FHIP_OK;  // empty tensor
    if (!src || !out || count < 0 || inner <= 0 ||
        (src_dtype != FHIP_FP32 && src_dtype != FHIP_BF16 && src_dtype != FHIP_FP16))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "quantize_linear: bad arguments");
    int rc = validate_qparams(ctx, channels, scales, zero_points, n_zp);
    if (rc != FHIP_OK) return rc;
    QParams qp{};
    const float* ds;
    const int32_t* dz;
    if ((rc = upload_params(ctx, channels, scales, zero_points, n_zp, &qp, &ds, &dz)) != FHIP_OK) return rc;
    if (channels == 1 && !ds) {  // per tensor, parameters inline
        const float sc = qp.scale[0];
        const int32_t z = qp.zp[0];
        if (src_dtype == FHIP_FP32)
            quantize_tensor_kernel<FHIP_FP32><<<grid_for(count, 256), 256, 0, ctx->stream>>>(src, count, sc, z, out);
        else if (src_dtype == FHIP_BF16)
            quantize_tensor_kernel<FHIP_BF16><<<grid_for(count, 256), 256, 0, ctx->stream>>>(src, count, sc, z, out);
        else
            quantize_tensor_kernel<FHIP_FP16><<<grid_for(count, 256), 256, 0, ctx->stream>>>(src, count, sc, z, out);
    } else {
        quantize_kernel<<<grid_for(count, 256), 256, 0, ctx->stream>>>(src, src_dtype, count, channels, inner, qp, ds,
                                                                        dz, n_zp > 1 ? 1 : 0, out);
    }
    ctx->last_backend = "quantize_linear";
    FHIP_CHECK_LAUNCH(ctx, "quantize_kernel");
    return FHIP_OK;
}

int fhip_dequantize_linear(fhip_context ctx, const int8_t* src, int64_t count, int64_t channels, int64_t inner,
                           const float* scales, const int32_t* zero_points, int64_t n_zp, int dst_dtype, void* out) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (count == 0) return FHIP_OK;  // empty tensor
    if (!src || !out || count < 0 || inner <= 0 ||
        (dst_dtype != FHIP_FP32 && dst_dtype != FHIP_BF16 && dst_dtype != FHIP_FP16))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "dequantize_linear: bad arguments");
    int rc = validate_qparams(ctx, channels, scales, zero_points, n_zp);
    if (rc != FHIP_OK) return rc;
    QParams qp{};
    const float* ds;
    const int32_t* dz;
    if ((rc = upload_params(ctx, channels, scales, zero_points, n_zp, &qp, &ds, &dz)) != FHIP_OK) return rc;
    dequantize_kernel<<<grid_for(count, 256), 256, 0, ctx->stream>>>(src, count, channels, inner, qp, ds, dz,
                                                                      n_zp > 1 ? 1 : 0, dst_dtype, out);
    ctx->last_backend = "dequantize_linear";
    FHIP_CHECK_LAUNCH(ctx, "dequantize_kernel");
    return FHIP_OK;
}

}  // extern "C"
