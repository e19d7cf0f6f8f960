// fp8_gemm_impl.h -- FP8 (e4m3 / e5m2) prefill GEMM on gfx950 MFMA: the kernel and its launcher.
//
// Included by the fp8_gemm_<fmt>_<out>.hip translation units, each of which instantiates the launcher
// for one (FP8 format, output width) pair, so the kernel's many specialisations compile in parallel.
// The dispatcher over those pairs is fp8_gemm.hip.
//
// out[m, n] = epilogue( sum_k Dec(A[m,k]) * Dec(B[n,k]) )   (Fp8Epilogue: scales, alpha/beta/bias,
// FP8 output code, optional decode to BF16/FP32 -- src/kernel/common/gemm.cc:62-100).
//
// Tiling:
//   * block tile BM x BN, 8 waves (512 threads) arranged WAVES_M x WAVES_N; K advances BK (64 or 128) per
//     stage; v_mfma_scale_f32_32x32x64_f8f6f4 (block scale 1, or a folded power-of-two output factor), fp32
//     accumulators; lane l supplies row/column l%32 and the 32-byte K slice (l/32) of each 64-deep step,
//     for A and B alike, so both index the same K in every MFMA slot;
//   * A (activations, [m][k]) and B (prepared weight, [Np][Kp]) stages move global -> LDS with
//     buffer_load ... lds (no VGPR round trip) through buffer resources based at the tile's first row;
//     16-byte chunks are XOR-swizzled per row so every ds_read_b128 group of 16 lanes hits 16 distinct
//     bank groups; a ring of STAGES buffers keeps the next stages' loads in flight;
//   * with 128-deep stages the two 64-deep steps are software-pipelined: the fragment reads of the next
//     step are in flight while the current step's MFMAs run;
//   * tile order is XCD-aware: consecutive workgroups land on different XCDs (round-robin dispatch),
//     so the tile index is re-derived to give each XCD a rectangle of tiles whose shared operand rows
//     fit in that XCD's L2 (XcdMap);
//   * epilogue: accumulators -> output bits -> LDS tile -> coalesced 16-byte global stores.
//
// The same kernel in its INT8 mode (template flag I8; i8_gemm_tile.hip): int8 operands, two
// v_mfma_i32_32x32x32_i8 per 64-deep step, int32 accumulators, and I8Epilogue's requantization (i8_common.h)
// in a rolled loop over accumulators staged through LDS.
#ifndef FHIP_FP8_GEMM_IMPL_H
#define FHIP_FP8_GEMM_IMPL_H
#include "fp8_common.h"
#include "i8_common.h"

#include <cmath>
#include <utility>

namespace {

using namespace fhip;

// The FP8 instantiations take this empty stand-in, so their kernel arguments stay as small as before.
struct NoI8Epilogue {};

typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef int v4i_t __attribute__((ext_vector_type(4)));


// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N).  Used where the accumulator
// registers are indexed, so no index is ever a runtime value (which would demote them to scratch).
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS stage: A rows [BM][BK bytes], then B rows [BNP][BK] (BNP = BN rounded up so every wave issues
// the same number of 16-byte loads).  Rows are unpadded; the 16-byte chunk c of row r sits at position
// c ^ swz(r): BK = 64 (4 chunks): swz(r) = (r >> 2) & 3; BK = 128 (8 chunks): swz(r) = (r >> 1) & 7.  Both
// keep the 16 lanes of every ds_read_b128 group (16 consecutive rows, one chunk) on 16 distinct 16-byte
// bank groups.
template <int BM, int BN, int NT, int BK>
struct Stage {
    static constexpr int kChunks = BK / 16;             // 16-byte chunks per row
    static constexpr int kRowsPerPass = NT / kChunks;   // one pass of 16-byte loads covers these rows
    static constexpr int BNP = (BN + kRowsPerPass - 1) / kRowsPerPass * kRowsPerPass;
    static constexpr int kA = BM * BK;
    static constexpr int kBytes = (BM + BNP) * BK;
    static constexpr int kLoadsA = BM * kChunks / NT;   // 16-byte loads per thread per stage
    static constexpr int kLoadsB = BNP * kChunks / NT;
    static constexpr int kLoads = kLoadsA + kLoadsB;
    static_assert(kLoadsA * NT == BM * kChunks, "BM must be a multiple of NT/kChunks");
};

// Dynamic LDS of the tile kernel: the operand stage ring, reused for the output tile in the epilogue;
// in the INT8 mode followed by the tile's per-column requantization parameters (wsum, vector bias, weight
// scale: three [BN] arrays of 4-byte values).
template <int BM, int BN, int NT, int OUT_BYTES, int BK, int STAGES, bool I8 = false>
constexpr size_t lds_bytes() {
    constexpr size_t ops = (size_t)STAGES * Stage<BM, BN, NT, BK>::kBytes;
    constexpr size_t epi = (size_t)BM * (BN * OUT_BYTES + 16);
    return (ops > epi ? ops : epi) + (I8 ? (size_t)((BN + 63) / 64 * 64) * 12 : 0);
}

template <int BK>
__device__ __forceinline__ int swz(int r) { return BK == 64 ? (r >> 2) & 3 : (r >> 1) & 7; }

typedef __attribute__((address_space(3))) void* lds_ptr;

// Buffer resource word 3 for raw (unstructured) byte-addressed buffers on gfx9-family parts.
constexpr int kBufferRsrcWord3 = 0x00020000;

// LDS fragment read issued as inline asm.  The compiler's wait-count pass treats every LDS read as
// possibly aliasing the in-flight LDS-DMA stage loads and would put a vmcnt(0) in front of it, draining
// the whole load pipeline each stage; the explicit vmcnt(N) + s_barrier above each stage already
// orders these reads.  The matching lgkmcnt wait is lds_fence() below.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
template <int OFF>
__device__ __forceinline__ u32x4_t lds_read16(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds_read offset field is 16 bits");
    u32x4_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}

template <int FM, int FN>
__device__ __forceinline__ void lds_fence(u32x4_t (&fa)[FM][2], u32x4_t (&fb)[FN][2]) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < FM; ++i) asm volatile("" : "+v"(fa[i][0]), "+v"(fa[i][1]));
#pragma unroll
    for (int j = 0; j < FN; ++j) asm volatile("" : "+v"(fb[j][0]), "+v"(fb[j][1]));
}

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}

// Output bits for one accumulator, branch-free.  The hardware converter encodes finite in-range values
// (round to nearest even; checked against the reference codec on every such input by the GPU test
// suite); values beyond the largest finite code are replaced with the reference's saturated / special
// codes by selects: finite overflow -> max finite, Inf -> 0x7e (e4m3) / 0x7c (e5m2), NaN -> 0x7f / 0x7d,
// each with the value's sign (include/util/fp8.h:66-211).
// Scale modes of the epilogue (host-selected):
//   kScaleGeneral: any out_scale; the reference's order and its division (gemm.cc:87-98);
//   kScalePow2:    out_scale a power of two; without a bias acc*ab_scale*alpha/out_scale is one multiply
//                  by the precombined factor `mul`; with a bias the reference's order, then * 1/out_scale;
//   kScaleFolded:  no bias and `mul` = 2^e with |e| <= 64: the factor rides on the MFMA's block-scale
//                  operand, so the accumulators already hold y / out_scale.  Scaling by 2^e is exact for
//                  every product and partial sum of FP8 values in that range (|e| <= 64 keeps them normal
//                  and finite in fp32), so the result equals acc * mul.
constexpr int kScaleGeneral = 0, kScalePow2 = 1, kScaleFolded = 2;

template <bool E5, int SM, bool BIAS>
__device__ __forceinline__ float scaled(const Fp8Epilogue& ep, float mul, float acc, int64_t row, int64_t col) {
    if constexpr (SM == kScaleFolded) {
        return acc;
    } else if constexpr (!BIAS) {
        if constexpr (SM == kScalePow2) return acc * mul;
        return (acc * ep.ab_scale * ep.alpha) / ep.out_scale;
    } else {
        float y = acc * ep.ab_scale * ep.alpha;
        // the tile epilogue evaluates positions past n (and past m: the caller clamps the row) that are never
        // stored; their bias index is clamped into the bias, which holds exactly n (vector) or m * n values
        const int64_t bcol = col < ep.n ? col : ep.n - 1;
        const uint8_t bc = ep.bias[ep.bias_kind == FHIP_BIAS_VECTOR ? bcol : row * ep.n + bcol];
        y += ep.beta * (fhip::fp8_decode(bc, E5) * ep.bias_scale);
        return SM == kScalePow2 ? y * ep.out_inv : y / ep.out_scale;
    }
}


// Output bits of four consecutive columns (col..col+3) of one row, packed little-endian: four FP8 codes
// in one dword (OUT_BYTES 1), four BF16 in two dwords (2) or four FP32 (4).  The hardware converter
// encodes finite in-range values (round to nearest even; checked against the reference codec on every
// such input by the GPU test suite); beyond the largest finite code the reference's saturated and
// special codes are selected instead: finite overflow -> max finite, Inf -> 0x7e (e4m3) / 0x7c (e5m2),
// NaN -> 0x7f / 0x7d, each with the value's sign (include/util/fp8.h:66-211).
// FIX = false: hardware codes only, with `flag` marking special codes (encode4_flag; the caller then
// redoes the tile with FIX = true, so the patch-up code stays out of the hot path).
template <bool E5, int SM, bool BIAS, int OUT_BYTES, bool FIX>
__device__ __forceinline__ void fast_value4(const Fp8Epilogue& ep, float mul, const float (&acc)[4], int64_t row,
                                            int64_t col, uint32_t (&out)[OUT_BYTES], uint32_t& flag) {
    float q[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) q[t] = scaled<E5, SM, BIAS>(ep, mul, acc[t], row, col + t);
    const uint32_t packed = FIX ? encode4<E5>(q) : encode4_flag<E5>(q, flag);
    if constexpr (OUT_BYTES == 1) {
        out[0] = packed;
    } else if constexpr (SM != kScaleGeneral) {
        // out_scale is a power of two in [2^-100, 2^100] (host-checked): Dec(code) * out_scale is exact and
        // normal in fp32, so its BF16 form is the upper half of its bits (no rounding happens).  The
        // reference decodes every NaN code to +qNaN; the hardware keeps the sign, so NaN is replaced.
        const v2f lo = E5 ? __builtin_amdgcn_cvt_pk_f32_bf8((int)packed, false) : __builtin_amdgcn_cvt_pk_f32_fp8((int)packed, false);
        const v2f hi = E5 ? __builtin_amdgcn_cvt_pk_f32_bf8((int)packed, true) : __builtin_amdgcn_cvt_pk_f32_fp8((int)packed, true);
        const float d[4] = {lo.x, lo.y, hi.x, hi.y};
        uint32_t bits[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const float v = d[t] * ep.out_scale;
            bits[t] = v != v ? 0x7fc00000u : __float_as_uint(v);
        }
        if constexpr (OUT_BYTES == 2) {
            out[0] = __builtin_amdgcn_perm(bits[1], bits[0], 0x07060302u);  // high halves: bf16 of v0, v1
            out[1] = __builtin_amdgcn_perm(bits[3], bits[2], 0x07060302u);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) out[t] = bits[t];
        }
    } else {
        float v[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) v[t] = decode_code<E5>((packed >> (8 * t)) & 0xffu) * ep.out_scale;
        if constexpr (OUT_BYTES == 2) {
            out[0] = (uint32_t)fhip::bf16_encode(v[0]) | ((uint32_t)fhip::bf16_encode(v[1]) << 16);
            out[1] = (uint32_t)fhip::bf16_encode(v[2]) | ((uint32_t)fhip::bf16_encode(v[3]) << 16);
        } else {
#pragma unroll
            for (int t = 0; t < 4; ++t) out[t] = __float_as_uint(v[t]);
        }
    }
}

// Tile -> XCD assignment.  Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2.  When the tile grid splits into 8 equal rectangles (gm x gn rectangles of rm x rn tiles), XCD x
// takes rectangle x, chosen so that the A rows and B columns its tiles share (rm*BM + rn*BN rows of
// K bytes) are as few as possible; otherwise consecutive tile indices go to the same XCD.
struct XcdMap {
    int gn, rm, rn;  // rm == 0: no rectangle split
};

// WTN1 > 0 (WAVES_N == 2): the two wave columns are unequal, BN - WTN1 and WTN1 wide.  Waves w and
// w + WAVES_M (one of each width) then share a SIMD (a block's waves are spread over the 4 SIMDs
// round-robin), so every SIMD carries the same MFMA work; this lets BN be 224 = 128 + 96.
// I8 = true: the INT8 GEMM on the same tiles -- A and B are int8, each 64-deep step is two
// v_mfma_i32_32x32x32_i8 (the two 16-byte halves of every lane's 32-byte K slice, for A and B alike, so
// both still index the same K in every MFMA slot; integer sums are exact in any order), int32 accumulators,
// and the epilogue is I8Epilogue's requantization (OUT_BYTES 1: INT8 codes, 4: fused DequantizeLinear to
// FP32).  E5, SM and the Fp8Epilogue are unused then.
template <bool E5, int BM, int BN, int WAVES_M, int WAVES_N, int OUT_BYTES, int SM, int BK, int STAGES, int WTN1,
          bool I8 = false>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void fp8_gemm_kernel(const uint8_t* __restrict__ a, int64_t m, int64_t k,
                                                       const uint8_t* __restrict__ b, int64_t kp, int64_t np,
                                                       int tiles_n, int tiles_total, XcdMap xm, int mfma_scale, Fp8Epilogue ep,
                                                       std::conditional_t<I8, I8Epilogue, NoI8Epilogue> iep) {
    constexpr int NT = 64 * WAVES_M * WAVES_N;
    using S = Stage<BM, BN, NT, BK>;
    constexpr int kSub = BK / 64;  // 64-deep MFMA steps per stage
    static_assert(BK == 64 || BK == 128, "stage depth is 64 or 128");
    static_assert(WTN1 == 0 || (WAVES_N == 2 && WAVES_M == 4 && WTN1 < BN), "unequal wave columns: 4 x 2 waves");
    constexpr int WTM = BM / WAVES_M;
    constexpr int WTN0 = WTN1 == 0 ? BN / WAVES_N : BN - WTN1;  // width of wave column 0 (all columns if equal)
    constexpr int FM = WTM / 32, FN0 = WTN0 / 32, FN1 = WTN1 / 32;
    static_assert(FM * 32 == WTM && FN0 * 32 == WTN0 && FN1 * 32 == WTN1, "wave tile must be a multiple of 32");
    static_assert(WTN1 != 0 || WTN0 * WAVES_N == BN, "equal wave columns must cover BN");
    constexpr int fmt = E5 ? 1 : 0;
    extern __shared__ __align__(16) uint8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = WTN1 == 0 ? wave / WAVES_N : wave % WAVES_M;
    const int wn = WTN1 == 0 ? wave % WAVES_N : wave / WAVES_M;
    const int wcol = wn * WTN0;  // first tile column of this wave

    int tile = blockIdx.x;
    if (xm.rm > 0) {
        // workgroup b runs on XCD b % 8; XCD x takes the x-th rm x rn rectangle of tiles
        const int x = tile & 7, l = tile >> 3;
        tile = ((x / xm.gn) * xm.rm + l / xm.rn) * tiles_n + (x % xm.gn) * xm.rn + l % xm.rn;
    } else if ((gridDim.x & 7) == 0) {
        tile = (tile & 7) * (gridDim.x >> 3) + (tile >> 3);
    }
    if (tile >= tiles_total) return;
    const int64_t m0 = (int64_t)(tile / tiles_n) * BM;
    const int64_t n0 = (int64_t)(tile % tiles_n) * BN;

    const int nk = (int)(k / BK);  // host guarantees k % BK == 0
    // Stage loads go through buffer resources based at this tile's first row: one 32-bit offset register
    // per 16-byte load instead of a 64-bit pointer.  A rows past m are out of the resource's range and
    // read as zero (those rows are computed, never stored); the prepared weight is padded to np rows.
    // The host keeps m*k and np*kp below 2^31.
    const __amdgpu_buffer_rsrc_t rsrc_a =
        __builtin_amdgcn_make_buffer_rsrc((void*)(a + m0 * k), 0, (int)((m - m0) * k), kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rsrc_b =
        __builtin_amdgcn_make_buffer_rsrc((void*)(b + n0 * kp), 0, (int)((np - n0) * kp), kBufferRsrcWord3);
    // Slot i of a thread's loads covers row r0 + i * kRowsPerPass, same chunk (the swizzle repeats every 16
    // rows), so one base offset per operand plus a uniform per-slot, per-stage term addresses every load.
    static_assert(S::kRowsPerPass % 16 == 0, "slot rows must keep the swizzle phase");
    const int r0 = tid / S::kChunks;
    const int c0s = (tid % S::kChunks) ^ swz<BK>(r0);
    const uint32_t voff_a = (uint32_t)(r0 * k + c0s * 16);
    const uint32_t voff_b = (uint32_t)(r0 * kp + c0s * 16);
    auto issue = [&](int kt) {
        uint8_t* st = smem + (kt % STAGES) * S::kBytes;
#pragma unroll
        for (int i = 0; i < S::kLoads; ++i) {
            const bool is_a = i < S::kLoadsA;
            const int slot = is_a ? i : i - S::kLoadsA;
            uint8_t* dst = st + (is_a ? 0 : S::kA) + (slot * NT + wave * 64) * 16;
            // the uniform term varies with kt, so the per-slot sums are not hoisted into live registers
            const uint32_t u = (uint32_t)(slot * S::kRowsPerPass * (is_a ? k : kp) + (int64_t)kt * BK);
            // a stage past the last is out of the resource's range (operands are below 2^31 bytes), and so
            // are the B rows of the last pass beyond BN (BNP > BN when BN = 224), which no fragment reads
            const bool live = kt < nk && (is_a || S::BNP == BN || r0 + slot * S::kRowsPerPass < BN);
            const uint32_t off = live ? (is_a ? voff_a : voff_b) + u : 0x80000000u;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(is_a ? rsrc_a : rsrc_b, (lds_ptr)dst, 16, off, 0, 0, 0);
        }
    };

    constexpr int kOutPitch = BN * OUT_BYTES + 16;  // epilogue: output tile staged in LDS
    uint8_t* const so = smem;
    // INT8: the tile's per-column requantization parameters move to LDS (past the ring and the output tile)
    // with 4-byte buffer_load ... lds, issued before any stage load: every later vmcnt wait of the main
    // loop covers them.  Columns past n read as zero and are never stored.
    constexpr size_t kColOff = lds_bytes<BM, BN, NT, OUT_BYTES, BK, STAGES, false>();
    // column arrays of the INT8 mode: BN rounded up to 64 entries (whole 64-lane DMA loads; BN = 224 tiles)
    constexpr int BNR = (BN + 63) / 64 * 64;
    if constexpr (I8) {
        constexpr int kParts = BNR / 64;
        const int cols = (int)(iep.ldo - n0 < BN ? iep.ldo - n0 : BN);
        for (int q = wave; q < 3 * kParts; q += NT / 64) {
            const int arr = q / kParts, part = q % kParts;
            const void* src = arr == 0 ? (const void*)iep.wsum
                              : arr == 1 ? (const void*)iep.bias : (const void*)iep.w_scales;
            const int bytes = arr == 1 && iep.bias_kind != FHIP_BIAS_VECTOR ? 0 : cols * 4;
            const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(static_cast<const uint8_t*>(src) + (bytes ? n0 * 4 : 0)), 0, bytes, kBufferRsrcWord3);
            uint8_t* dst = smem + kColOff + (size_t)arr * BNR * 4 + part * 256;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)dst, 4, (uint32_t)(part * 256 + lane * 4), 0, 0, 0);
        }
    }
  // The rest runs with this wave's fragment-column count FN as a compile-time constant.
  auto body = [&](auto fn_tag) {
    constexpr int FN = decltype(fn_tag)::value;
    using AccT = std::conditional_t<I8, v16i_t, v16f>;
    AccT acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;

    const int frag_row = lane & 31;
    const int frag_c = (lane >> 5) * 2;
    // Fragment reads of 64-deep step u of the stage at byte offset `st` into fa/fb.  The swizzle of a
    // fragment row depends only on frag_row (wave and fragment row offsets are multiples of 32), so every
    // read is one of four per-thread column offsets plus a per-thread row base, a uniform stage offset
    // and a compile-time immediate; no per-fragment address registers stay live across the loop.
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr)smem;
    const uint32_t row_a = lds0 + (uint32_t)((wm * WTM + frag_row) * BK);
    const uint32_t row_b = lds0 + (uint32_t)(S::kA + (wcol + frag_row) * BK);
    const uint32_t col0 = (uint32_t)((frag_c ^ swz<BK>(frag_row)) << 4);
    const uint32_t col1 = (uint32_t)(((frag_c + 1) ^ swz<BK>(frag_row)) << 4);
    auto read_frags = [&](uint32_t st, int u, u32x4_t (&fa)[FM][2], u32x4_t (&fb)[FN][2]) {
        const uint32_t cu = (uint32_t)u * 64u;  // chunk index + 4u: frag_c + 1 < 4, so XOR with 4 adds 4u
        const uint32_t a0 = row_a + st + (col0 ^ cu), a1 = row_a + st + (col1 ^ cu);
        const uint32_t b0 = row_b + st + (col0 ^ cu), b1 = row_b + st + (col1 ^ cu);
        static_for<FM>([&](auto ii) {
            constexpr int i = decltype(ii)::value;
            fa[i][0] = lds_read16<i * 32 * BK>(a0);
            fa[i][1] = lds_read16<i * 32 * BK>(a1);
        });
        static_for<FN>([&](auto jj) {
            constexpr int j = decltype(jj)::value;
            fb[j][0] = lds_read16<j * 32 * BK>(b0);
            fb[j][1] = lds_read16<j * 32 * BK>(b1);
        });
    };
    // The block scale lives in one VGPR for the whole kernel.  Left to the compiler, the kernel-argument
    // SGPR is copied into a VGPR inside the loop, and that copy gets an lgkmcnt(0) wait in front of it,
    // which stalls the MFMAs behind the fragment reads issued just before them.
    int scale_v;
    asm volatile("v_mov_b32 %0, %1" : "=v"(scale_v) : "s"(mfma_scale));
    auto mfmas = [&](const u32x4_t (&fa)[FM][2], const u32x4_t (&fb)[FN][2]) {
        if constexpr (I8) {
            // Two MFMAs per 64-deep step, one per 16-byte half of each lane's K slice.  The half is the outer
            // loop so consecutive MFMAs write different accumulators (no back-to-back dependency).  Weight
            // fragment as the row operand: each 32x32 block is computed transposed.
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        const v4i_t av = v4i_t{(int)fa[i][h].x, (int)fa[i][h].y, (int)fa[i][h].z, (int)fa[i][h].w};
                        const v4i_t bv = v4i_t{(int)fb[j][h].x, (int)fb[j][h].y, (int)fb[j][h].z, (int)fb[j][h].w};
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv, av, acc[i][j], 0, 0, 0);
                    }
        } else {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const v8i av = v8i{(int)fa[i][0].x, (int)fa[i][0].y, (int)fa[i][0].z, (int)fa[i][0].w,
                                       (int)fa[i][1].x, (int)fa[i][1].y, (int)fa[i][1].z, (int)fa[i][1].w};
                    const v8i bv = v8i{(int)fb[j][0].x, (int)fb[j][0].y, (int)fb[j][0].z, (int)fb[j][0].w,
                                       (int)fb[j][1].x, (int)fb[j][1].y, (int)fb[j][1].z, (int)fb[j][1].w};
                    // weight fragment as the row operand: each 32x32 block is computed transposed
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, acc[i][j], fmt, fmt, 0, scale_v, 0, 127);
                }
        }
        // Pin the MFMAs here: they are pure operations, which IR-level code motion may sink below the
        // following lgkmcnt fence (sched_barrier binds only the machine scheduler).  Volatile asm keeps
        // its order with the fence.
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) asm volatile("" : "+v"(acc[i][j]));
    };
    // Wait until at most min(STAGES - 2, nk - 1 - kt) stages issued after stage kt are still in flight.
    auto wait_stage = [&](int kt) {
        const int ahead = nk - 1 - kt;
        if (STAGES >= 4 && ahead >= 2) wait_vmcnt<2 * S::kLoads>();
        else if (STAGES >= 3 && ahead >= 1) wait_vmcnt<S::kLoads>();
        else wait_vmcnt<0>();
    };

    if constexpr (kSub == 2) {
        // Software pipeline over the two 64-deep steps of each stage: the fragment reads of the next step
        // (of this stage, or the first step of the next stage, after its barrier) are in flight while the
        // MFMAs of the current step run.  A stage's buffer is refilled only after the barrier that follows
        // every wave's last read of it.
        // The loop body has no branch (a branch lets the compiler sink the first step's MFMAs below it,
        // keeping two copies of the f0 fragments alive): stages past the last are issued as out-of-range
        // loads, which move nothing from memory and write zeros into a buffer nobody reads again, so
        // exactly STAGES - 2 stages are in flight behind the one waited for.
        u32x4_t f0a[FM][2], f0b[FN][2], f1a[FM][2], f1b[FN][2];
        for (int s0 = 0; s0 < STAGES - 1; ++s0) issue(s0);
        wait_vmcnt<(STAGES - 2) * S::kLoads>();
        __builtin_amdgcn_s_barrier();
        issue(STAGES - 1);
        read_frags(0u, 0, f0a, f0b);
        lds_fence<FM, FN>(f0a, f0b);
        for (int kt = 0; kt < nk - 1; ++kt) {
            read_frags((uint32_t)((kt % STAGES) * S::kBytes), 1, f1a, f1b);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(f0a, f0b);
            __builtin_amdgcn_sched_barrier(0);
            lds_fence<FM, FN>(f1a, f1b);
            wait_vmcnt<(STAGES - 2) * S::kLoads>();
            __builtin_amdgcn_s_barrier();
            issue(kt + STAGES);
            read_frags((uint32_t)(((kt + 1) % STAGES) * S::kBytes), 0, f0a, f0b);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(f1a, f1b);
            __builtin_amdgcn_sched_barrier(0);
            lds_fence<FM, FN>(f0a, f0b);
        }
        read_frags((uint32_t)(((nk - 1) % STAGES) * S::kBytes), 1, f1a, f1b);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(f0a, f0b);
        __builtin_amdgcn_sched_barrier(0);
        lds_fence<FM, FN>(f1a, f1b);
        mfmas(f1a, f1b);
        wait_vmcnt<0>();  // the trailing out-of-range loads still write LDS, which the epilogue reuses
    } else {
#pragma unroll
        for (int s0 = 0; s0 < STAGES - 1; ++s0)
            if (s0 < nk) issue(s0);
        for (int kt = 0; kt < nk; ++kt) {
            wait_stage(kt);
            // Plain s_barrier: the explicit vmcnt wait above already covers this wave's stage loads, and a
            // __syncthreads() fence would also wait for the loads of the stages still in flight.
            __builtin_amdgcn_s_barrier();
            if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1);
            u32x4_t fa[FM][2], fb[FN][2];
            read_frags((uint32_t)((kt % STAGES) * S::kBytes), 0, fa, fb);
            // Wait for the fragment reads; every fragment register is an operand, so no MFMA that uses
            // one can be scheduled above the wait.
            lds_fence<FM, FN>(fa, fb);
            mfmas(fa, fb);
        }
    }
    if constexpr (I8) {
        // Integer path: each column's parameters become (dot + bias correction, kl, kh) in place: shift =
        // vector bias - zp_a * wsum, and K = s_a * s_w / s_out split into a float pair.  The staged values
        // are visible here (every wave waited for its loads and passed a barrier since).
        if (iep.int_path) {
            int32_t* cw = reinterpret_cast<int32_t*>(smem + kColOff);
            for (int c = tid; c < BN; c += NT) {
                float kh, kl;
                iep.split_scale(reinterpret_cast<const float*>(cw + 2 * BNR)[c], kh, kl);
                cw[c] = (iep.bias_kind == FHIP_BIAS_VECTOR ? cw[BNR + c] : 0) - iep.zp_a * cw[c];
                reinterpret_cast<float*>(cw + BNR)[c] = kl;
                reinterpret_cast<float*>(cw + 2 * BNR)[c] = kh;
            }
        }
    }
    __syncthreads();

    // ---- epilogue.  The MFMA computed each 32x32 block transposed (weight fragment as the row operand),
    // so lane l holds output row m = l%32 of the block and, for e = 4g..4g+3, the four consecutive
    // output columns 8g + 4*(l/32) .. +3: one packed dword (FP8) per group, staged in an LDS tile and
    // written out with coalesced 16-byte stores.
    const int row_in = lane & 31;
    const int col_q = (lane >> 5) * 4;
    const float mul = ep.ab_scale * ep.alpha * ep.out_inv;
    auto stage_tile = [&](auto bias_tag, auto fix_tag) __attribute__((always_inline)) {
        constexpr bool BIAS = decltype(bias_tag)::value, FIX = decltype(fix_tag)::value;
        uint32_t flag = 0;
        static_for<FM * FN>([&](auto ij) {
            constexpr int i = decltype(ij)::value / FN, j = decltype(ij)::value % FN;
            static_for<4>([&](auto gg) {
                constexpr int g = decltype(gg)::value;
                const int r = wm * WTM + i * 32 + row_in;
                const int c = wcol + j * 32 + g * 8 + col_q;
                const float v4[4] = {acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                uint32_t packed[OUT_BYTES];
                // rows past m are computed, never stored: their bias row is clamped to the last one
                const int64_t brow = m0 + r < m ? m0 + r : m - 1;
                fast_value4<E5, SM, BIAS, OUT_BYTES, FIX>(ep, mul, v4, brow, n0 + c, packed, flag);
                uint8_t* dst = so + r * kOutPitch + c * OUT_BYTES;
                if constexpr (OUT_BYTES == 1) *reinterpret_cast<uint32_t*>(dst) = packed[0];
                else if constexpr (OUT_BYTES == 2) *reinterpret_cast<uint2*>(dst) = make_uint2(packed[0], packed[1]);
                else *reinterpret_cast<uint4*>(dst) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            });
        });
        return (flag & 0x80808080u) != 0;
    };
    // Hot pass with the hardware codes; a lane that met a value beyond the largest finite code (or
    // Inf/NaN) rewrites its whole share with the reference's codes in a separate, cold pass.
    auto epilogue = [&](auto bias_tag) {
        if (__builtin_expect(stage_tile(bias_tag, std::false_type{}), 0)) {
            // opaque to the optimiser, so the hot pass's intermediate values are not kept alive for reuse here
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) asm volatile("" : "+v"(acc[i][j]));
            stage_tile(bias_tag, std::true_type{});
        }
    };
    if constexpr (I8) {
        // INT8: the int32 accumulators go through LDS one fragment row at a time (a slab of WAVES_M x 32 rows
        // by BN columns), and a rolled loop requantizes four consecutive values per thread (I8Epilogue:
        // zero-point correction, bias, alpha/beta, scales) and stores their codes (OUT_BYTES 1) or their
        // DequantizeLinear values (2: FP16/BF16, 4: FP32) straight to the output.  Unrolled over the 64 to
        // 128 accumulators of a lane, the same work held the whole accumulator set live through a long
        // branchy tail and spilled.  The integer path decides each code with requant_i8_split; values it
        // cannot decide (x.5 points) take the reference's fp64 arithmetic in place.
        constexpr int kSlabRows = WAVES_M * 32;
        constexpr int kChunksRow = BNR / 4;  // 16-byte chunks of int32 per staged row (past BN: never read)
        static_assert((size_t)kSlabRows * BNR * 4 <= kColOff, "INT8 slab must not reach the column parameters");
        int32_t* const slab = reinterpret_cast<int32_t*>(smem);
        // chunk swizzle: the 32 rows of one ds_write_b128 group land on distinct 16-byte bank groups
        auto slab_at = [&](int srow, int chunk) __attribute__((always_inline)) {
            return slab + srow * BNR + ((chunk ^ ((srow & (kChunksRow / 2 - 1)) << 1)) << 2);
        };
        const int rows_in = (int)(m - m0 < BM ? m - m0 : BM);
        const int cols_in = (int)(iep.ldo - n0 < BN ? iep.ldo - n0 : BN);
        const int32_t zp_out_i = (int32_t)iep.zp_out;
        const float zp_half = (float)zp_out_i + 0.5f;
        const int32_t* colp = reinterpret_cast<const int32_t*>(smem + kColOff);
        // NT is a multiple of the chunks per row, so a thread's chunk (its four columns) is the same in every
        // pass and slab: their parameters are read once
        static_assert(NT % kChunksRow == 0, "one chunk per thread");
        const int chunk = tid % kChunksRow, c = chunk * 4;
        const int64_t col = n0 + c;
        const int nv = cols_in - c < 4 ? cols_in - c : 4;
        const int4 p0 = *reinterpret_cast<const int4*>(colp + c);
        const int4 p1 = *reinterpret_cast<const int4*>(colp + BNR + c);
        const int4 p2 = *reinterpret_cast<const int4*>(colp + 2 * BNR + c);
        const int a0[4] = {p0.x, p0.y, p0.z, p0.w}, a1[4] = {p1.x, p1.y, p1.z, p1.w};
        const int a2[4] = {p2.x, p2.y, p2.z, p2.w};
        static_for<FM>([&](auto ii) {
            constexpr int i = decltype(ii)::value;
            if (i > 0) __syncthreads();  // the previous slab has been read
            static_for<FN>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                static_for<4>([&](auto gg) {
                    constexpr int g = decltype(gg)::value;
                    const int c = wcol + j * 32 + g * 8 + col_q;
                    *reinterpret_cast<int4*>(slab_at(wm * 32 + row_in, c >> 2)) =
                        make_int4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
                });
            });
            __syncthreads();
            for (int srow = tid / kChunksRow; srow < kSlabRows && c < cols_in; srow += NT / kChunksRow) {
                const int r = (srow >> 5) * WTM + i * 32 + (srow & 31);
                if (r >= rows_in) continue;
                const int4 raw4 = *reinterpret_cast<const int4*>(slab_at(srow, chunk));
                const int raw[4] = {raw4.x, raw4.y, raw4.z, raw4.w};
                const int64_t row = m0 + r;
                int8_t qv[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    bool unsafe;
                    if (iep.int_path) {
                        // a0 = shift (bias - zp_a * wsum), a1 = kl bits, a2 = kh bits; the cheap screen
                        // first, the float-pair form where it cannot decide (about 2^-10 of the values)
                        int32_t v = raw[t] + a0[t];
                        if (iep.bias_kind == FHIP_BIAS_MATRIX) v += iep.bias[row * iep.ldo + col + (t < nv ? t : 0)];
                        qv[t] = requant_i8_screen(v, __int_as_float(a2[t]), zp_half, unsafe);
                        if (__builtin_expect(unsafe, 0))
                            qv[t] = requant_i8_split(v, __int_as_float(a2[t]), __int_as_float(a1[t]), zp_out_i, unsafe);
                    } else {
                        const I8Epilogue::Col cpt{a0[t], a1[t], __int_as_float(a2[t])};
                        const int64_t ct = col + (t < nv ? t : 0);
                        qv[t] = requant_i8_fast(iep.real(raw[t], row, ct, cpt), iep.recip_out, iep.zp_out, unsafe);
                    }
                    if (__builtin_expect(unsafe && t < nv, 0))
                        qv[t] = iep.code(raw[t], row, col + t, iep.col_params(col + t));
                }
                const int64_t idx = row * iep.ldo + col;
                if constexpr (OUT_BYTES == 1) {
                    int8_t* dst = static_cast<int8_t*>(iep.out_any) + idx;
                    if (nv == 4 && (reinterpret_cast<uintptr_t>(dst) & 3) == 0) {
                        *reinterpret_cast<uint32_t*>(dst) = (uint32_t)(uint8_t)qv[0] | (uint32_t)(uint8_t)qv[1] << 8 |
                                                            (uint32_t)(uint8_t)qv[2] << 16 |
                                                            (uint32_t)(uint8_t)qv[3] << 24;
                    } else {
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            if (t < nv) dst[t] = qv[t];
                    }
                } else if constexpr (OUT_BYTES == 2) {
                    uint16_t h[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const float v = iep.dequant(qv[t]);
                        h[t] = iep.out_dtype == FHIP_FP16 ? fhip::fp16_encode(v) : fhip::bf16_encode_plain(v);
                    }
                    uint16_t* dst = static_cast<uint16_t*>(iep.out_any) + idx;
                    if (nv == 4 && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
                        *reinterpret_cast<uint2*>(dst) = make_uint2((uint32_t)h[0] | (uint32_t)h[1] << 16,
                                                                    (uint32_t)h[2] | (uint32_t)h[3] << 16);
                    } else {
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            if (t < nv) dst[t] = h[t];
                    }
                } else {
                    float* dst = static_cast<float*>(iep.out_any) + idx;
                    const float4 v = make_float4(iep.dequant(qv[0]), iep.dequant(qv[1]), iep.dequant(qv[2]),
                                                 iep.dequant(qv[3]));
                    if (nv == 4 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
                        *reinterpret_cast<float4*>(dst) = v;
                    } else {
                        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int t = 0; t < 4; ++t)
                            if (t < nv) dst[t] = vv[t];
                    }
                }
            }
        });
    } else {
        if (ep.bias_kind != FHIP_BIAS_NONE) epilogue(std::true_type{});
        else epilogue(std::false_type{});
    }
  };
    // wave-uniform branch; both bodies run the same sequence of barriers
    if (WTN1 == 0 || wn == 0) body(std::integral_constant<int, FN0>{});
    else body(std::integral_constant<int, (FN1 > 0 ? FN1 : 1)>{});
    if constexpr (I8) return;  // the INT8 epilogue stored its values itself
    __syncthreads();
    constexpr int kChunks = BN * OUT_BYTES / 16;
    const int64_t n_bytes = ep.n * OUT_BYTES;
    uint8_t* out = static_cast<uint8_t*>(ep.out);
    const bool vec = (n_bytes & 15) == 0;
    for (int q = tid; q < BM * kChunks; q += NT) {
        const int r = q / kChunks, c = q % kChunks;
        const int64_t row = m0 + r;
        const int64_t colb = n0 * OUT_BYTES + c * 16;
        if (row >= m || colb >= n_bytes) continue;
        const uint8_t* s2 = so + r * kOutPitch + c * 16;
        uint8_t* dst = out + row * n_bytes + colb;
        if (vec) {
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(s2);
        } else {
            for (int i = 0; i < 16 && colb + i < n_bytes; ++i) dst[i] = s2[i];
        }
    }
}


template <bool E5, int OB, int BM, int BN, int WAVES_M, int WAVES_N, int BK = 64, int STAGES = 4, int WTN1 = 0,
          bool I8 = false>
int launch_tile(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w,
                const Fp8Epilogue& ep, const char* name, const I8Epilogue* iep = nullptr) {
    const int64_t kp = ((w->k + 127) / 128) * 128;
    const int64_t np = ((w->n + 255) / 256) * 256;
    const int tiles_m = (int)((m + BM - 1) / BM), tiles_n = (int)((w->n + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int grid = tiles;  // the kernel remaps tiles XCD-wise
    if (m * k64 >= (int64_t(1) << 31) || np * kp >= (int64_t(1) << 31))
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8 gemm: a prepared weight of 2 GiB or more");
    XcdMap xm{1, 0, 1};
    {
        const int splits[4][2] = {{8, 1}, {4, 2}, {2, 4}, {1, 8}};
        int64_t best = -1;
        for (const auto& sp : splits) {
            if (tiles_m % sp[0] != 0 || tiles_n % sp[1] != 0) continue;
            const int rm = tiles_m / sp[0], rn = tiles_n / sp[1];
            const int64_t rows = (int64_t)rm * BM + (int64_t)rn * BN;
            if (best < 0 || rows < best) {
                best = rows;
                xm = XcdMap{sp[1], rm, rn};
            }
        }
    }
    const uint8_t* wd = static_cast<const uint8_t*>(w->data);
    // power-of-two output scale in a range where decoded outputs stay exact normal fp32 values
    const bool pow2 = ep.out_inv != 0.0f && ep.out_scale >= 0x1p-100f && ep.out_scale <= 0x1p100f;
    int sm = pow2 ? kScalePow2 : kScaleGeneral;
    int mfma_scale = 127;  // E8M0 block scale 2^(s - 127)
    if (pow2 && ep.bias_kind == FHIP_BIAS_NONE) {
        const float mul = ep.ab_scale * ep.alpha * ep.out_inv;
        int e = 0;
        if (std::isfinite(mul) && std::frexp(mul, &e) == 0.5f && e - 1 >= -64 && e - 1 <= 64) {
            sm = kScaleFolded;
            mfma_scale = 127 + (e - 1);
        }
    }
    std::conditional_t<I8, I8Epilogue, NoI8Epilogue> i8_arg{};
    if constexpr (I8) i8_arg = *iep;
#define FHIP_GEMM_LAUNCH(OB, SMV)                                                                                   \
    fp8_gemm_kernel<E5, BM, BN, WAVES_M, WAVES_N, OB, SMV, BK, STAGES, WTN1, I8><<<grid, 64 * WAVES_M * WAVES_N,                       \
                                                          lds_bytes<BM, BN, 64 * WAVES_M * WAVES_N, OB, BK, STAGES, I8>(), ctx->stream>>>( \
        a, m, k64, wd, kp, np, tiles_n, tiles, xm, mfma_scale, ep, i8_arg)
#define FHIP_GEMM_LAUNCH_SM(OB)                                                                                     \
    do {                                                                                                            \
        if (sm == kScaleFolded) FHIP_GEMM_LAUNCH(OB, kScaleFolded);                                                 \
        else if (sm == kScalePow2) FHIP_GEMM_LAUNCH(OB, kScalePow2);                                                \
        else FHIP_GEMM_LAUNCH(OB, kScaleGeneral);                                                                   \
    } while (0)
    if constexpr (lds_bytes<BM, BN, 64 * WAVES_M * WAVES_N, OB, BK, STAGES, I8>() > 160 * 1024) {
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8 gemm: output tile too large for LDS");
    } else if constexpr (I8) {
        FHIP_GEMM_LAUNCH(OB, kScaleGeneral);
    } else {
        FHIP_GEMM_LAUNCH_SM(OB);
    }
#undef FHIP_GEMM_LAUNCH_SM
#undef FHIP_GEMM_LAUNCH
    ctx->last_backend = name;
    FHIP_CHECK_LAUNCH(ctx, "fp8_gemm_kernel");
    return FHIP_OK;
}

template <bool E5, int OB>
int launch(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k64, const fhip_weight_s* w, const Fp8Epilogue& ep) {
    const int64_t n = w->n;
    // Tile choice: fill the 256 CUs with whole tiles where the shape allows it; 128-deep stages (half the
    // barriers per MFMA) when K allows them.
    const bool big = ((m + 255) / 256) * ((n + 255) / 256) >= 192 && OB != 4;
    if (k64 % 128 == 0) {
        // N a multiple of 224 (Qwen's 3584 = 16 x 224): 256x224 tiles, so the tile count is a multiple of 16
        // instead of 14 (C3 up-projection: 256 tiles for 256 CUs instead of 224); measured ~2% faster
        if (big && n % 224 == 0)
            return launch_tile<E5, OB, 256, 224, 4, 2, 128, 2, 96>(ctx, a, m, k64, w, ep, "fp8_mfma_gemm_256x224_bk128_w8");
        if (big) return launch_tile<E5, OB, 256, 256, 4, 2, 128, 2>(ctx, a, m, k64, w, ep, "fp8_mfma_gemm_256x256_bk128_w8");
        return launch_tile<E5, OB, 128, 128, 2, 4, 128, 4>(ctx, a, m, k64, w, ep, "fp8_mfma_gemm_128x128_bk128_w8");
    }
    if (big) return launch_tile<E5, OB, 256, 256, 4, 2>(ctx, a, m, k64, w, ep, "fp8_mfma_gemm_256x256_w8");
    return launch_tile<E5, OB, 128, 128, 2, 4>(ctx, a, m, k64, w, ep, "fp8_mfma_gemm_128x128_w8");
}

}  // namespace

#endif  // FHIP_FP8_GEMM_IMPL_H
