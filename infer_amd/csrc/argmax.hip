// argmax.hip -- decode LM-head GEMV with fused greedy selection (QwenGemmArgmax) on gfx950.
//
// Semantics (src/kernel/common/qwen_gemm_argmax.cc:28-49, x86/linear.cc:603-648): per vocabulary row
// v, s_v = fp32 dot(a, w_v); the value compared is BF16(s_v) (RNE, NaN quieted); NaN values are
// skipped; the first strict maximum wins, so equal values -- including +0 and -0 -- keep the lowest
// index; when every value is NaN the token is 0.
// FP8 head (x86/linear_fp8.cc:757-788; the exported Gemm -> Cast(bf16) pair): the value compared is
// BF16(Dec(Enc(s_v / out_scale)) * out_scale).
//
// Selection is a max over 64-bit keys  (order(bf16) << 32) | (0xffffffff - v):  `order` maps BF16
// bits to an unsigned key monotone in the value with +0/-0 merged, NaN never enters, and a larger
// low word means a lower index.  Key 0 means "no candidate".
//
// Layout of the work: the weight [V][K] streams once from HBM with 16-byte loads; each wave owns a
// strip of rows and keeps R rows in flight; the activation rows (m <= 16) stay in registers as raw
// BF16/FP8 bits.  Each block publishes one key per activation row to a partials array, and the
// last block to finish (atomic ticket) reduces the partials, writes the int64 tokens and re-arms
// the ticket, so the kernel is replay-safe with no memset.
#include "fhip_internal.h"
#include "codec.h"

#include <algorithm>
#include <mutex>
#include <utility>

namespace {

typedef float v2f __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint4 load_stream16(const uint8_t* p) {
    const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(x.x, x.y, x.z, x.w);
}

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRows = 4;  // weight rows per wave and unit of the m = 1 kernel's C5-shaped case (grid sizing)

// Compile-time loop: f(std::integral_constant<int, I>) for I in [0, N), so register arrays are only ever
// indexed by constants.
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ unsigned long long make_key(uint16_t bf, int64_t idx) {
    if ((bf & 0x7f80u) == 0x7f80u && (bf & 0x7fu) != 0u) return 0ull;  // NaN: never selected
    uint32_t u = bf;
    if ((u & 0x7fffu) == 0u) u = 0u;                                    // -0 == +0
    const uint32_t order = (u & 0x8000u) ? (~u & 0xffffu) : (u | 0x8000u);
    return ((unsigned long long)order << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ int64_t key_index(unsigned long long key) {
    return key == 0ull ? 0 : (int64_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
}

__device__ __forceinline__ unsigned long long wave_max(unsigned long long v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// Element type of the head: BF16 (2 B) or FP8 (1 B).  One 16-byte load = 8 BF16 or 16 FP8 values.
template <int KIND>  // 0 = BF16, 1 = FP8 e4m3, 2 = FP8 e5m2
struct Head {
    static constexpr int kPer16 = KIND == 0 ? 8 : 16;
    __device__ static __forceinline__ void decode(const uint4& v, float* f) {
        if constexpr (KIND == 0) {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[2 * i] = __uint_as_float(w[i] << 16);
                f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v2f lo, hi;
                if constexpr (KIND == 2) {
                    lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w[i], false);
                    hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w[i], true);
                } else {
                    lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
                    hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
                }
                f[4 * i] = lo.x;
                f[4 * i + 1] = lo.y;
                f[4 * i + 2] = hi.x;
                f[4 * i + 3] = hi.y;
            }
        }
    }
};

struct HeadParams {
    float ab_scale;   // FP8: a_scale * w_scale
    float out_scale;  // FP8: output scale
    float* logits;    // optional [m][v]
};

// Cross-block hand-off.  Each block stores its per-row keys as agent-scope atomic stores, then takes a
// ticket; the block that takes the last ticket reads every block's keys with agent-scope atomic loads
// and writes the tokens.  Two orderings are compiled:
//   kRelease = true (the m = 1 kernel): the ticket is a release RMW, the last block of each ticket
//     group acquires the group (acquire fence) and passes it on with an acq_rel RMW on the top counter,
//     so the final block has acquired every block's key stores through the counters' release
//     sequences -- HIP's scoped C++ memory model at agent scope, with no reliance on the hardware.  On
//     gfx950 each release is `buffer_wbl2 sc1; s_waitcnt vmcnt(0)` before the RMW and each acquire a
//     `buffer_inv sc1` after it; on the C5 head (256 blocks) it costs nothing measurable
//     (54.0 us per call either way).
//   kRelease = false (the MFMA kernel, 2 blocks per CU): the same RMWs relaxed, after
//     `s_waitcnt vmcnt(0)` -- the completion half of LLVM's agent-scope release sequence for gfx942/gfx950
//     without the L2 write-back (`buffer_wbl2`).  The write-back exists for non-atomic stores that may
//     sit dirty in one XCD's L2; the keys are agent-scope atomic stores, which the same memory model
//     keeps coherent across the agent's L2s, and the wait makes each one complete before its block's
//     ticket is counted; the final block's agent-scope atomic loads are issued after it has seen the
//     last ticket.  Here the write-back is not free: the release form measured 80.6 us per C5 M=8 call
//     against 61.8 us.
__device__ __forceinline__ void publish_key(unsigned long long* slot, unsigned long long key) {
    __hip_atomic_store(slot, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every block after it published its per-row keys to partials[block * stride + j].  The
// last block to take a ticket reduces all blocks' keys, writes the tokens and re-arms the tickets,
// so the kernel is replay-safe with no memset.
template <int STRIDE, bool kRelease>
__device__ __forceinline__ void ticket_and_finish(const unsigned long long* partials, int64_t m,
                                                  ArgmaxScratch* scratch, int64_t* tokens) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    __shared__ bool last;
    __syncthreads();
    if (threadIdx.x == 0) {
        // block b counts in group b % G; the group's last block counts in `done`
        const unsigned int groups = gridDim.x < (unsigned)kTicketGroups ? gridDim.x : (unsigned)kTicketGroups;
        const unsigned int g = blockIdx.x % groups;
        const unsigned int members = (gridDim.x - g + groups - 1) / groups;
        // the barrier above orders every thread's key store before the ticket
        bool top = false;
        unsigned int t;
        if constexpr (kRelease) {
            t = __hip_atomic_fetch_add(&scratch->group_done[g][0], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            __builtin_amdgcn_s_waitcnt(0);  // this block's key stores (threads < 16, same wave) are complete
            t = __hip_atomic_fetch_add(&scratch->group_done[g][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (t == members - 1) {
            // every member has counted: re-arm the group and count the group in `done`
            if constexpr (kRelease) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __hip_atomic_store(&scratch->group_done[g][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            top = __hip_atomic_fetch_add(&scratch->done, 1u, kRelease ? __ATOMIC_ACQ_REL : __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT) == groups - 1;
        }
        last = top;
    }
    __syncthreads();
    if (!last) return;
    __shared__ unsigned long long fin[kWaves][STRIDE];
    for (int j = 0; j < STRIDE && j < m; ++j) {
        unsigned long long b = 0ull;
        for (int64_t q = threadIdx.x; q < gridDim.x; q += kThreads) {
            const unsigned long long p = __hip_atomic_load(&partials[q * STRIDE + j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            b = p > b ? p : b;
        }
        b = wave_max(b);
        if (lane == 0) fin[wave][j] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int j = 0; j < STRIDE && j < m; ++j) {
            unsigned long long b = fin[0][j];
            for (int q = 1; q < kWaves; ++q) b = fin[q][j] > b ? fin[q][j] : b;
            tokens[j] = key_index(b);
        }
        __hip_atomic_store(&scratch->done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // re-arm
    }
}

// Transposing butterfly over the wave: v[0..V) holds V partial sums per lane (V a power of two
// <= 64).  Each exchange step halves the values a lane keeps (the lane keeps the half selected by
// its lane bit and adds its partner's copy of that half), so after log2(V) steps lane l owns the
// wave-wide sum of value index  l >> (6 - log2 V), and the remaining steps are plain
// butterflies.  V-1 + (6 - log2 V) shuffles in total instead of 6*V.
template <int V>
__device__ __forceinline__ float transpose_reduce(float (&v)[V], int lane) {
    int cnt = V;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        if (cnt > 1) {
            const int half = cnt / 2;
            const bool upper = (lane & off) != 0;
#pragma unroll
            for (int i = 0; i < V / 2; ++i) {
                if (i < half) {
                    const float send = upper ? v[i] : v[i + half];
                    const float keep = upper ? v[i + half] : v[i];
                    v[i] = keep + __shfl_xor(send, off, 64);
                }
            }
            cnt = half;
        } else {
            v[0] += __shfl_xor(v[0], off, 64);
        }
    }
    return v[0];
}

template <int V>
struct Log2 {
    static constexpr int value = V <= 1 ? 0 : 1 + Log2<V / 2>::value;
};

// ---- m = 1: LDS-ring kernel ------------------------------------------------------------------------
// Each wave streams units of the weight -- ROWS rows x SEGS 1 KiB segments, one 16-byte load per lane
// per row segment, 8 loads in all -- into its own two-slot LDS ring with buffer_load ... lds (no VGPR
// round trip), and computes unit u while unit u+1 is in flight.  A wave walks row groups g = gw,
// gw + GW, ... (gw its global wave index, GW the wave count), each group being nsb consecutive units
// over the row's segments; the per-lane partial sums of the group's ROWS rows carry across its units
// and are reduced (transposing butterfly) after the last one.
// Measured against the register double buffer this replaces (C5 head, 311 MB): ~4 us less per call.
// One strip in flight per wave (two slots) is the fastest depth: more slots put more of the head in
// flight than the HBM system serves best (three or four slots measured slower).
// The activation stays in registers when one unit covers the whole row (WHOLE), and otherwise sits in
// LDS behind the rings, zero-padded to whole units, so any K with K * esize <= kArgmaxMaxRowBytes works.
// Lanes past the row's end and rows past v load out of the buffer resource's range, which writes zeros
// into the ring without touching memory.
typedef __attribute__((address_space(3))) void* lds_ptr;
constexpr int kRingSlots = 2;
constexpr int kUnitLoads = 8;                      // 1 KiB wave loads per unit
constexpr int kUnitBytes = kUnitLoads * 1024;
constexpr int kRingBytes = kWaves * kRingSlots * kUnitBytes;  // 64 KiB
constexpr int kBufferRsrcWord3 = 0x00020000;       // raw byte-addressed buffer
constexpr int kCachePolicyNT = 2;                  // non-temporal: the head streams once

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    // gfx9 s_waitcnt: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[15:14]
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | (((N >> 4) & 3) << 14));
}

// LDS read as inline asm: the compiler's wait-count pass would otherwise treat it as aliasing the
// in-flight LDS-DMA loads and drain them all (vmcnt(0)) in front of it.  The caller orders it with
// wait_vmcnt and waits for it with lgkmcnt(0).
template <int OFF>
__device__ __forceinline__ u32x4 lds_read16(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}

__device__ __forceinline__ uint4 to_uint4(const u32x4& v) { return make_uint4(v.x, v.y, v.z, v.w); }

template <int KIND, int ROWS, int SEGS, bool WHOLE>
__global__ __launch_bounds__(kThreads) void gemv_argmax_kernel(const uint8_t* __restrict__ a, int64_t k,
                                                               const uint8_t* __restrict__ w, int64_t v,
                                                               HeadParams hp, unsigned long long* __restrict__ partials,
                                                               ArgmaxScratch* __restrict__ scratch,
                                                               int64_t* __restrict__ tokens) {
    static_assert(ROWS * SEGS == kUnitLoads, "a unit is kUnitLoads row segments");
    using H = Head<KIND>;
    constexpr int esize = KIND == 0 ? 2 : 1;
    constexpr int kShift = 6 - Log2<ROWS>::value;
    extern __shared__ __align__(16) uint8_t smem[];  // [kWaves][kRingSlots][kUnitBytes] rings, then the activation
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row_bytes = k * esize;
    const int nsb = WHOLE ? 1 : (int)((row_bytes + SEGS * 1024 - 1) / (SEGS * 1024));  // units per row group
    uint8_t* const ring = smem + wave * (kRingSlots * kUnitBytes);
    const uint32_t ring_addr = (uint32_t)(uintptr_t)(lds_ptr)ring + (uint32_t)lane * 16u;
    uint8_t* const xl = smem + kRingBytes;
    const uint32_t x_addr = (uint32_t)(uintptr_t)(lds_ptr)xl + (uint32_t)lane * 16u;

    float xf[WHOLE ? SEGS : 1][H::kPer16];
    if constexpr (WHOLE) {
#pragma unroll
        for (int j = 0; j < SEGS; ++j) {
            const int64_t col = (int64_t)j * 1024 + lane * 16;
            const uint4 c = col < row_bytes ? *reinterpret_cast<const uint4*>(a + col) : make_uint4(0, 0, 0, 0);
            H::decode(c, xf[j]);
        }
    } else {
        const int64_t padded = (int64_t)nsb * SEGS * 1024;
        for (int64_t c = (int64_t)threadIdx.x * 16; c < padded; c += kThreads * 16)
            *reinterpret_cast<uint4*>(xl + c) = c < row_bytes ? *reinterpret_cast<const uint4*>(a + c) : make_uint4(0, 0, 0, 0);
        __syncthreads();
    }

    const int64_t gw = (int64_t)blockIdx.x * kWaves + wave;
    const int64_t group_stride = (int64_t)gridDim.x * kWaves * ROWS;
    // Issue side: the unit (i_row, i_b) goes to slot i_slot; one unit ahead of the compute side.
    int64_t i_row = gw * ROWS;
    int i_b = 0, i_slot = 0;
    auto issue = [&]() {
        const bool live = i_row < v;
        const int64_t rem = live ? (v - i_row) * row_bytes : 0;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(w + (live ? i_row : 0) * row_bytes), 0, (int)(rem < 0x7fffffff ? rem : 0x7fffffff), kBufferRsrcWord3);
        uint8_t* const dst = ring + i_slot * kUnitBytes;
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int j = 0; j < SEGS; ++j) {
                const int64_t col = (int64_t)(i_b * SEGS + j) * 1024 + lane * 16;
                const uint32_t off = col < row_bytes ? (uint32_t)(r * row_bytes + col) : 0x80000000u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(dst + (r * SEGS + j) * 1024), 16, off, 0, 0,
                                                         kCachePolicyNT);
            }
        i_slot ^= 1;
        if (++i_b == nsb) {
            i_b = 0;
            i_row += group_stride;
        }
    };

    unsigned long long best = 0ull;
    float acc[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
    int64_t c_row = gw * ROWS;
    int c_b = 0, c_slot = 0;
    issue();
    while (c_row < v) {
        wait_vmcnt<0>();  // this unit has landed; nothing else is in flight
        issue();          // the next unit goes to the other slot, whose reads completed last iteration
        const uint32_t sa = ring_addr + (uint32_t)(c_slot * kUnitBytes);
        u32x4 wv[ROWS][SEGS];
        static_for<ROWS * SEGS>([&](auto ii) {
            constexpr int i = decltype(ii)::value;
            wv[i / SEGS][i % SEGS] = lds_read16<i * 1024>(sa);
        });
        u32x4 xv[WHOLE ? 1 : SEGS];
        if constexpr (!WHOLE) {
            const uint32_t xa = x_addr + (uint32_t)(c_b * SEGS * 1024);
            static_for<SEGS>([&](auto jj) {
                constexpr int j = decltype(jj)::value;
                xv[j] = lds_read16<j * 1024>(xa);
            });
        }
        // Wait for the reads, and tie every fragment register to the wait so no use of one is scheduled above it.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int j = 0; j < SEGS; ++j) asm volatile("" : "+v"(wv[r][j]));
        if constexpr (!WHOLE) {
#pragma unroll
            for (int j = 0; j < SEGS; ++j) asm volatile("" : "+v"(xv[j]));
        }
#pragma unroll
        for (int j = 0; j < SEGS; ++j) {
            float xs[H::kPer16];
            if constexpr (WHOLE) {
#pragma unroll
                for (int i = 0; i < H::kPer16; ++i) xs[i] = xf[j][i];
            } else {
                H::decode(to_uint4(xv[j]), xs);
            }
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                float wf[H::kPer16];
                H::decode(to_uint4(wv[r][j]), wf);
                float s = acc[r];
#pragma unroll
                for (int i = 0; i < H::kPer16; ++i) s += xs[i] * wf[i];
                acc[r] = s;
            }
        }
        c_slot ^= 1;
        if (++c_b == nsb) {
            c_b = 0;
            float s = transpose_reduce<ROWS>(acc, lane);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = 0.0f;
            const int64_t row = c_row + (lane >> kShift);
            if (row < v) {
                uint16_t bf;
                if constexpr (KIND == 0) {
                    bf = fhip::bf16_encode(s);
                } else {
                    const uint8_t code = fhip::fp8_encode(s * hp.ab_scale / hp.out_scale, KIND == 2);
                    s = fhip::fp8_decode(code, KIND == 2) * hp.out_scale;
                    bf = fhip::bf16_encode(s);
                }
                const unsigned long long key = make_key(bf, row);
                best = key > best ? key : best;
                if (hp.logits != nullptr && (lane & ((1 << kShift) - 1)) == 0) hp.logits[row] = s;
            }
            c_row += group_stride;
        }
    }
    wait_vmcnt<0>();  // the trailing unit (past the end: zeros, no memory traffic) lands before the wave exits

    // Block reduction -> partials[block]
    __shared__ unsigned long long red[kWaves];
    best = wave_max(best);
    if (lane == 0) red[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = red[0];
#pragma unroll
        for (int q = 1; q < kWaves; ++q) b = red[q] > b ? red[q] : b;
        publish_key(&partials[blockIdx.x], b);
    }
    ticket_and_finish<1, true>(partials, 1, scratch, tokens);
}

// ---- m >= 2: MFMA kernel --------------------------------------------------------------------------
// A block walks vocabulary tiles of 16 rows (grid-stride).  Its 4 waves split K: wave w owns the
// SPW consecutive steps starting at w*SPW, a step being 32 BF16 (v_mfma_f32_16x16x32_bf16) or 128 FP8
// (v_mfma_scale_f32_16x16x128_f8f6f4, unit scales) values of K.  The activation rows are the A operand
// and stay in registers for the whole kernel; each tile's weight rows are the B operand.  Each wave
// streams its own K quarter of the tile (16 rows x SPW steps) into a private two-slot LDS ring with
// 1 KiB buffer_load ... lds loads and computes one tile while the next is in flight, so the ring needs
// no barrier (measured on the C5 head, M = 8: 54.4 us against 62.3 us for the same kernel loading B
// into registers with a register double buffer).  The lanes of a DMA load are permuted so that LDS
// holds each row's chunks XOR-swizzled by the row index, and the fragment reads of 16 rows x one
// chunk hit 16 distinct bank groups.  Lane l supplies row l%16 (activation row / vocabulary row) and
// the l/16-th 16-byte (BF16) or 32-byte (FP8) slice of the step, for A and B alike.  The four partial
// 16x16 tiles meet in LDS (double buffered: one barrier per tile) and thread t finishes activation
// row t/16 of vocabulary row t%16.

// Dynamic LDS of the MFMA kernel: each wave's two-slot ring of its K quarter of a 16-row tile.
template <int KIND, int SPW>
constexpr size_t mfma_ring_bytes() {
    return (size_t)kWaves * 2 * 16 * SPW * 4 * (KIND == 0 ? 16 : 32);
}

template <int KIND, int SPW>
__global__ __launch_bounds__(kThreads) void gemv_argmax_mfma_kernel(const uint8_t* __restrict__ a, int64_t m,
                                                                         int64_t k, const uint8_t* __restrict__ w,
                                                                         int64_t v, HeadParams hp,
                                                                         unsigned long long* __restrict__ partials,
                                                                         ArgmaxScratch* __restrict__ scratch,
                                                                         int64_t* __restrict__ tokens) {
    constexpr int esize = KIND == 0 ? 2 : 1;
    constexpr int SB = KIND == 0 ? 16 : 32;   // bytes per lane per step
    constexpr int NV = SB / 16;               // 16-byte fragment reads per lane per step
    constexpr int QB = SPW * 4 * SB;          // bytes of each row in one wave's K quarter
    constexpr int CPR = QB / 16;              // 16-byte chunks per row of a quarter
    constexpr int SWM = (CPR < 16 ? CPR : 16) - 1;
    constexpr int QBYTES = 16 * QB;           // one wave's quarter of a 16-row tile
    constexpr int LOADS = QBYTES / 1024;      // 1 KiB DMA loads per wave per tile
    static_assert(QBYTES % 1024 == 0, "a quarter is whole 1 KiB loads");
    static_assert(LOADS <= 32, "vmcnt range");
    extern __shared__ __align__(16) uint8_t smem[];  // [kWaves][2 slots][QBYTES]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int fr = lane & 15;
    const int64_t row_bytes = k * esize;
    const int64_t qoff = (int64_t)wave * QB;  // this wave's quarter within a row
    uint8_t* const ring = smem + wave * 2 * QBYTES;
    // activation fragments (A operand), masked past the row end and past m
    uint4 xa[SPW][NV];
    {
        const bool arow = fr < m;
        const uint8_t* ar = a + (arow ? fr : 0) * row_bytes;
#pragma unroll
        for (int s = 0; s < SPW; ++s)
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                const int64_t o = qoff + s * 4 * SB + (lane >> 4) * SB + 16 * q;
                const bool live = arow && o < row_bytes;
                const uint4 x = *reinterpret_cast<const uint4*>(ar + (live ? o : 0));
                const uint32_t msk = live ? 0xffffffffu : 0u;
                xa[s][q] = make_uint4(x.x & msk, x.y & msk, x.z & msk, x.w & msk);
            }
    }
    // DMA lane map: load i, lane p fills LDS chunk f = i*64 + p of the quarter ([row][CPR] chunks), which
    // holds chunk (f % CPR) ^ swz(row) of that row, so the fragment reads of 16 rows x one chunk hit 16
    // distinct bank groups.
    uint32_t voff[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int f = i * 64 + lane;
        const int row = f / CPR;
        const int c = (f % CPR) ^ (row & SWM);
        const int64_t col = qoff + c * 16;
        voff[i] = col < row_bytes ? (uint32_t)(row * row_bytes + col) : 0x80000000u;
    }
    const int64_t ntiles = (v + 15) / 16;
    auto issue = [&](int64_t t_issue, int s_issue) {
        const bool live = t_issue < ntiles;
        const int64_t row0 = live ? t_issue * 16 : 0;
        const int64_t rem = live ? (v - row0) * row_bytes : 0;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(w + row0 * row_bytes), 0, (int)(rem < 0x7fffffff ? rem : 0x7fffffff), kBufferRsrcWord3);
        uint8_t* const dst = ring + s_issue * QBYTES;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const uint32_t off = voff[i];
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(dst + i * 1024), 16, off, 0, 0, kCachePolicyNT);
        }
    };
    // fragment read addresses: row fr, chunk s*(4*SB/16) + (lane>>4)*NV + q
    const uint32_t rbase = (uint32_t)(uintptr_t)(lds_ptr)ring + (uint32_t)(fr * CPR * 16);
    uint32_t rcol[SPW][NV];
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
        for (int q = 0; q < NV; ++q) rcol[s][q] = (uint32_t)((((s * 4 * SB) / 16 + (lane >> 4) * NV + q) ^ (fr & SWM)) * 16);
    __shared__ float red[2][kWaves][16][17];
    const int my_m = threadIdx.x >> 4, my_c = threadIdx.x & 15;
    unsigned long long best = 0ull;
    int buf = 0, slot = 0;
    int64_t tile = blockIdx.x;
    issue(tile, 0);
    for (; tile < ntiles; tile += gridDim.x) {
        wait_vmcnt<0>();
        issue(tile + gridDim.x, slot ^ 1);
        const uint32_t sb = rbase + (uint32_t)(slot * QBYTES);
        u32x4 bw[SPW][NV];
#pragma unroll
        for (int s = 0; s < SPW; ++s)
#pragma unroll
            for (int q = 0; q < NV; ++q) {
                u32x4 t;
                asm volatile("ds_read_b128 %0, %1" : "=v"(t) : "v"(sb + rcol[s][q]));
                bw[s][q] = t;
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int s = 0; s < SPW; ++s)
#pragma unroll
            for (int q = 0; q < NV; ++q) asm volatile("" : "+v"(bw[s][q]));
        v4f acc = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < SPW; ++s) {
            if constexpr (KIND == 0) {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, xa[s][0]),
                                                              __builtin_bit_cast(v8bf, bw[s][0]), acc, 0, 0, 0);
            } else {
                const v8i av = v8i{(int)xa[s][0].x, (int)xa[s][0].y, (int)xa[s][0].z, (int)xa[s][0].w,
                                   (int)xa[s][NV - 1].x, (int)xa[s][NV - 1].y, (int)xa[s][NV - 1].z, (int)xa[s][NV - 1].w};
                const v8i bv = v8i{(int)bw[s][0].x, (int)bw[s][0].y, (int)bw[s][0].z, (int)bw[s][0].w,
                                   (int)bw[s][NV - 1].x, (int)bw[s][NV - 1].y, (int)bw[s][NV - 1].z, (int)bw[s][NV - 1].w};
                acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, KIND == 2 ? 1 : 0, KIND == 2 ? 1 : 0,
                                                                      0, 127, 0, 127);
            }
        }
        slot ^= 1;
#pragma unroll
        for (int r = 0; r < 4; ++r) red[buf][wave][(lane >> 4) * 4 + r][fr] = acc[r];
        __syncthreads();
        float sum = red[buf][0][my_m][my_c] + red[buf][1][my_m][my_c] + red[buf][2][my_m][my_c] + red[buf][3][my_m][my_c];
        const int64_t row = tile * 16 + my_c;
        if (my_m < m && row < v) {
            uint16_t bf;
            if constexpr (KIND == 0) {
                bf = fhip::bf16_encode(sum);
            } else {
                const uint8_t code = fhip::fp8_encode(sum * hp.ab_scale / hp.out_scale, KIND == 2);
                sum = fhip::fp8_decode(code, KIND == 2) * hp.out_scale;
                bf = fhip::bf16_encode(sum);
            }
            const unsigned long long key = make_key(bf, row);
            best = key > best ? key : best;
            if (hp.logits != nullptr) hp.logits[my_m * v + row] = sum;
        }
        buf ^= 1;
    }
    wait_vmcnt<0>();
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) {
        const unsigned long long x = __shfl_xor(best, o, 64);
        best = x > best ? x : best;
    }
    __shared__ unsigned long long row_key[16];
    if (my_c == 0) row_key[my_m] = best;
    __syncthreads();
    if (threadIdx.x < 16) publish_key(&partials[(int64_t)blockIdx.x * 16 + threadIdx.x], row_key[threadIdx.x]);
    ticket_and_finish<16, false>(partials, m, scratch, tokens);
}

// Grid and partial-key workspace of one call.  The grid strides over the vocabulary; measured on the C5
// head: the MFMA kernel (m >= 2) is fastest with 2 blocks per CU (1, 3, 4: 79, 68, 77 us against 62),
// the m = 1 kernel with 1 (54.2 against 55.1 us).  The workspace is sized for either kernel's grid, so a
// later call with other rows does not need a bigger one (e.g. under capture).
struct Plan {
    int64_t grid1;      // blocks of the m = 1 kernel
    int64_t mgrid;      // blocks of the MFMA kernel
    size_t ws_bytes;    // partial keys: 16 per block
};

Plan plan_for(int device, int64_t v) {
    int dev_cus = 256;
    (void)hipDeviceGetAttribute(&dev_cus, hipDeviceAttributeMultiprocessorCount, device);
    const int64_t rows_per_block = (int64_t)kWaves * kRows;
    const int64_t cap = (int64_t)dev_cus * 2;
    Plan p;
    p.grid1 = std::min<int64_t>((v + rows_per_block - 1) / rows_per_block, dev_cus);
    p.mgrid = std::min<int64_t>((v + 15) / 16, cap);
    const int64_t ws_blocks = std::max(p.mgrid, p.grid1);
    p.ws_bytes = (size_t)ws_blocks * 16 * sizeof(unsigned long long);
    return p;
}

// Enqueues the kernel for (m, k) on `stream`.  Returns FHIP_OK, FHIP_ERR_UNSUPPORTED (m > 16) or the
// launch error as FHIP_ERR_HIP (with *err set).
template <int KIND>
int launch_on(hipStream_t stream, const Plan& plan, const uint8_t* a, int64_t m, int64_t k, const uint8_t* w,
              int64_t v, HeadParams hp, unsigned long long* partials, ArgmaxScratch* tickets, int64_t* tokens,
              hipError_t* err) {
    const int64_t bytes = k * (KIND == 0 ? 2 : 1);
    if (m >= 2) {
        const int64_t step_bytes = KIND == 0 ? 64 : 128;
        const int64_t spw_need = ((bytes + step_bytes - 1) / step_bytes + kWaves - 1) / kWaves;
#define FHIP_ARGMAX_MFMA_CASE(SPW)                                                                              \
        if (spw_need <= (SPW)) {                                                                                \
            constexpr size_t lds = mfma_ring_bytes<KIND, SPW>();                                                \
            if (lds > 65536) {                                                                                  \
                static std::once_flag once;                                                                     \
                static hipError_t attr = hipSuccess;                                                            \
                std::call_once(once, [] {                                                                       \
                    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_argmax_mfma_kernel<KIND, SPW>), \
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);           \
                });                                                                                             \
                if (attr != hipSuccess) {                                                                       \
                    *err = attr;                                                                                \
                    return FHIP_ERR_HIP;                                                                        \
                }                                                                                               \
            }                                                                                                   \
            gemv_argmax_mfma_kernel<KIND, SPW><<<(unsigned)plan.mgrid, kThreads, lds, stream>>>(a, m, k, w, v, hp, \
                                                                                 partials, tickets, tokens);    \
            *err = hipGetLastError();                                                                           \
            return *err == hipSuccess ? FHIP_OK : FHIP_ERR_HIP;                                                 \
        }
        FHIP_ARGMAX_MFMA_CASE(2)
        FHIP_ARGMAX_MFMA_CASE(4)
        FHIP_ARGMAX_MFMA_CASE(8)
        FHIP_ARGMAX_MFMA_CASE(KIND == 0 ? 16 : 8)
#undef FHIP_ARGMAX_MFMA_CASE
    }
    // m = 1 (and rows beyond the MFMA kernel's K, one launch per activation row): the LDS-ring kernel.
    // Unit shape: 4 rows x 2 segments when the row is 1-2 KiB (the C5 head), else 8 rows x 1 segment.
    const int64_t nseg = (bytes + 1023) / 1024;
    for (int64_t j = 0; j < m; ++j) {
        const uint8_t* aj = a + j * bytes;
        HeadParams hpj = hp;
        if (hp.logits) hpj.logits = hp.logits + j * v;
        if (nseg == 2) {
            gemv_argmax_kernel<KIND, 4, 2, true><<<(unsigned)plan.grid1, kThreads, kRingBytes, stream>>>(
                aj, k, w, v, hpj, partials, tickets, tokens + j);
        } else if (nseg == 1) {
            gemv_argmax_kernel<KIND, 8, 1, true><<<(unsigned)plan.grid1, kThreads, kRingBytes, stream>>>(
                aj, k, w, v, hpj, partials, tickets, tokens + j);
        } else {
            const size_t lds = (size_t)kRingBytes + (size_t)nseg * 1024;
            static std::once_flag once;
            static hipError_t attr = hipSuccess;
            std::call_once(once, [] {
                attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_argmax_kernel<KIND, 8, 1, false>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           kRingBytes + kArgmaxMaxRowBytes);
            });
            if (attr != hipSuccess) {
                *err = attr;
                return FHIP_ERR_HIP;
            }
            gemv_argmax_kernel<KIND, 8, 1, false><<<(unsigned)plan.grid1, kThreads, lds, stream>>>(
                aj, k, w, v, hpj, partials, tickets, tokens + j);
        }
        *err = hipGetLastError();
        if (*err != hipSuccess) return FHIP_ERR_HIP;
    }
    return FHIP_OK;
}

template <int KIND>
int launch(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k, const uint8_t* w, int64_t v, HeadParams hp,
           int64_t* tokens, const char* name) {
    const Plan plan = plan_for(ctx->device, v);
    void* ws = nullptr;
    int rc = fhip::acquire_workspace(ctx, plan.ws_bytes, &ws);
    if (rc != FHIP_OK) return rc;
    hipError_t err = hipSuccess;
    rc = launch_on<KIND>(ctx->stream, plan, a, m, k, w, v, hp, static_cast<unsigned long long*>(ws), ctx->scratch,
                         tokens, &err);
    if (rc == FHIP_ERR_HIP) return fhip::check_hip(ctx, err, "gemv_argmax launch");
    if (rc != FHIP_OK) return fhip::set_error(ctx, rc, "gemv_argmax: m > 16");
    ctx->last_backend = name;
    return FHIP_OK;
}

// ---- the allocation-free variant -------------------------------------------------------------------
// One array per GPU holds the ticket counters (first kNoAllocTicketBytes) and the per-block partial
// keys.  Host code never passes `scratch` itself to a kernel: its address on each device comes from
// hipGetSymbolAddress at context creation (noalloc_setup), kept per device in g_scratch_ptr.
constexpr size_t kNoAllocTicketBytes = 8192;
static_assert(sizeof(ArgmaxScratch) <= kNoAllocTicketBytes, "ticket block must fit its reserved space");
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Zeroes the ticket counters with an ordinary kernel (a memset node would misbehave under graph capture).
__global__ void clear_tickets_kernel(unsigned int* t, int words) {
    for (int i = threadIdx.x; i < words; i += blockDim.x) t[i] = 0u;
}

}  // namespace

namespace fhip {

int noalloc_setup(fhip_context ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices)
        return set_error(ctx, FHIP_ERR_UNSUPPORTED, "device index beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[ctx->device]) return FHIP_OK;
    void* ptr = nullptr;  // the caller made ctx->device current
    int rc = check_hip(ctx, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc != FHIP_OK) return rc;
    g_scratch_ptr[ctx->device] = ptr;
    return FHIP_OK;
}

}  // namespace fhip

namespace {

template <int KIND>
int launch_noalloc(fhip_context ctx, const uint8_t* a, int64_t m, int64_t k, const uint8_t* w, int64_t v,
                   HeadParams hp, int64_t* tokens, const char* name) {
    void* base = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        base = ctx->device >= 0 && ctx->device < kMaxDevices ? g_scratch_ptr[ctx->device] : nullptr;
    }
    if (!base) return fhip::set_error(ctx, FHIP_ERR_STATE, "no-alloc scratch was not set up for this device");
    const Plan plan = plan_for(ctx->device, v);
    if (kNoAllocTicketBytes + plan.ws_bytes > kNoAllocScratchBytes)
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED,
                               "gemv_argmax_noalloc: " + std::to_string(kNoAllocTicketBytes + plan.ws_bytes) +
                                   " B of scratch needed, the static scratch holds " +
                                   std::to_string(kNoAllocScratchBytes) + " B");
    auto* tickets = static_cast<ArgmaxScratch*>(base);
    auto* partials = reinterpret_cast<unsigned long long*>(static_cast<unsigned char*>(base) + kNoAllocTicketBytes);
    clear_tickets_kernel<<<1, 256, 0, ctx->stream>>>(static_cast<unsigned int*>(base),
                                                     (int)(sizeof(ArgmaxScratch) / sizeof(unsigned int)));
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fhip::check_hip(ctx, err, "clear_tickets_kernel");
    int rc = launch_on<KIND>(ctx->stream, plan, a, m, k, w, v, hp, partials, tickets, tokens, &err);
    if (rc == FHIP_ERR_HIP) return fhip::check_hip(ctx, err, "gemv_argmax launch");
    if (rc != FHIP_OK) return fhip::set_error(ctx, rc, "gemv_argmax: m > 16");
    ctx->last_backend = name;
    return FHIP_OK;
}

}  // namespace

namespace {

// Argument checks of the BF16 head (both entry points).  Returns FHIP_OK with nothing to do for m == 0.
int check_bf16_args(fhip_context ctx, const uint16_t* a, int64_t m, int64_t k, const uint16_t* w, int64_t v,
                    const int64_t* tokens, const char* fn) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (m == 0) return FHIP_OK;  // no rows: nothing to select (the reference's loops run zero times)
    if (m > 0 && (k == 0 || v == 0))
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, std::string(fn) + ": empty K or vocabulary");
    if (!a || !w || !tokens || m < 0 || k < 0 || v < 0)
        return fhip::set_error(ctx, FHIP_ERR_INVALID, std::string(fn) + ": bad arguments");
    if (m > kArgmaxMaxRows || (k * 2) % 16 != 0 || k * 2 > kArgmaxMaxRowBytes || v >= (int64_t(1) << 32))
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, std::string(fn) + ": needs m <= 16, k % 8 == 0, k <= 32768");
    if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(w)) & 15)
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, std::string(fn) + ": pointers must be 16-byte aligned");
    return FHIP_OK;
}

}  // namespace

extern "C" {

int fhip_bf16_gemv_argmax(fhip_context ctx, const uint16_t* a, int64_t m, int64_t k, const uint16_t* w, int64_t v,
                          int64_t* tokens, float* logits) {
    int rc = check_bf16_args(ctx, a, m, k, w, v, tokens, "bf16_gemv_argmax");
    if (rc != FHIP_OK || m == 0) return rc;
    HeadParams hp{1.0f, 1.0f, logits};
    return launch<0>(ctx, reinterpret_cast<const uint8_t*>(a), m, k, reinterpret_cast<const uint8_t*>(w), v, hp, tokens,
                     "bf16_gemv_argmax");
}

int fhip_bf16_gemv_argmax_noalloc(fhip_context ctx, const uint16_t* a, int64_t m, int64_t k, const uint16_t* w,
                                  int64_t v, int64_t* tokens, float* logits) {
    int rc = check_bf16_args(ctx, a, m, k, w, v, tokens, "bf16_gemv_argmax_noalloc");
    if (rc != FHIP_OK || m == 0) return rc;
    HeadParams hp{1.0f, 1.0f, logits};
    return launch_noalloc<0>(ctx, reinterpret_cast<const uint8_t*>(a), m, k, reinterpret_cast<const uint8_t*>(w), v,
                             hp, tokens, "bf16_gemv_argmax_noalloc");
}

int fhip_fp8_gemv_argmax(fhip_context ctx, int dtype, const uint8_t* a, float a_scale, int64_t m, int64_t k,
                         const uint8_t* w, float w_scale, int64_t v, float out_scale, int64_t* tokens) {
    if (!ctx) return FHIP_ERR_INVALID;
    if (m == 0) return FHIP_OK;
    if (m > 0 && (k == 0 || v == 0))
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8_gemv_argmax: empty K or vocabulary");
    if (!a || !w || !tokens || m < 0 || k < 0 || v < 0 || (dtype != FHIP_FP8E4M3 && dtype != FHIP_FP8E5M2))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "fp8_gemv_argmax: bad arguments");
    if (!fhip::valid_scale(a_scale) || !fhip::valid_scale(w_scale) || !fhip::valid_scale(out_scale))
        return fhip::set_error(ctx, FHIP_ERR_INVALID, "fp8_gemv_argmax: scales must be finite and positive");
    if (m > kArgmaxMaxRows || k % 16 != 0 || k > kArgmaxMaxRowBytes || v >= (int64_t(1) << 32))
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8_gemv_argmax: needs m <= 16, k % 16 == 0, k <= 65536");
    if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(w)) & 15)
        return fhip::set_error(ctx, FHIP_ERR_UNSUPPORTED, "fp8_gemv_argmax: pointers must be 16-byte aligned");
    HeadParams hp{a_scale * w_scale, out_scale, nullptr};
    if (dtype == FHIP_FP8E5M2) return launch<2>(ctx, a, m, k, w, v, hp, tokens, "fp8e5m2_gemv_argmax");
    return launch<1>(ctx, a, m, k, w, v, hp, tokens, "fp8e4m3_gemv_argmax");
}

}  // extern "C"
