/*
 * fhip.h -- C ABI of the MI355X (gfx950) backend for Feather's quantized linear hot path.
 *
 * Library: infer_amd/libfhip.so.  Every entry point returns an int status (FHIP_OK = 0, < 0 on
 * error; the message is in fhip_last_error) and takes caller-owned device pointers.  No C++ or
 * torch types cross this boundary.  Work is enqueued on the context's stream; results are ready
 * after fhip_synchronize (or any later stream-ordered operation).
 *
 * Reference interfaces replaced (paths into the Feather tree, JPChen2000/Infer):
 *   - KernelBase::compute()/Prepare()/Supports() of the operators below: include/core/kernel.h:81-196
 *   - BackendContext (stream, capture, workspace/weight-cache budgets): include/core/backend.h:43-96
 *   - the CUDA device runtime it generalises: src/kernel/cuda/runtime.h:39-157
 */
#ifndef FHIP_H
#define FHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------------ */
#define FHIP_OK 0
#define FHIP_ERR_INVALID (-1)     /* the reference kernel returns -1 for these arguments          */
#define FHIP_ERR_UNSUPPORTED (-2) /* valid, but outside this backend: Supports() -> kUnsupported  */
#define FHIP_ERR_HIP (-3)         /* a HIP runtime call failed                                     */
#define FHIP_ERR_BUDGET (-4)      /* workspace or prepared-weight budget would be exceeded         */
#define FHIP_ERR_STATE (-5)       /* call not allowed in the current state (e.g. during capture)   */

/* ---- Feather DataType values (include/util/types.h:32-47) -------------------------------- */
#define FHIP_INT8 1
#define FHIP_FP16 3
#define FHIP_FP32 4
#define FHIP_INT32 5
#define FHIP_INT64 6
#define FHIP_BF16 11
#define FHIP_FP8E4M3 12
#define FHIP_FP8E5M2 13

/* Bias layouts (src/kernel/x86/linear_fp32.h:26-30 LinearBiasType). */
#define FHIP_BIAS_NONE 0
#define FHIP_BIAS_VECTOR 1 /* [N]                */
#define FHIP_BIAS_MATRIX 2 /* [M, N], row-major  */

/* Weight source layouts. */
#define FHIP_LAYOUT_KN 0 /* [K, N] row-major: MatMul b, FC w, Gemm with transB = 0 */
#define FHIP_LAYOUT_NK 1 /* [N, K] row-major: Gemm with transB = 1 (ONNX Linear)  */

/* INT8 linear flavours (their accumulation/bias rules differ). */
#define FHIP_I8_MATMUL 0 /* src/kernel/common/matmul.cc:156-261: no bias                          */
#define FHIP_I8_FC 1     /* src/kernel/common/fc.cc:105-159: int32 bias added to the accumulator    */
#define FHIP_I8_GEMM 2   /* src/kernel/common/gemm.cc:136-198: alpha*dot + beta*bias in double      */

/* Image layouts for Conv2D. */
#define FHIP_NCHW 0
#define FHIP_NHWC 1

typedef struct fhip_context_s* fhip_context;
typedef struct fhip_weight_s* fhip_weight;
typedef struct fhip_graph_s* fhip_graph;

/* ---- context (BackendContext, include/core/backend.h:43-96; runtime.h:39-157) ------------ */
/* Sizes: an empty input (m, count or batch 0) returns FHIP_OK without launching anything -- the
 * reference's loops run zero times and its kernels return 0; an empty K, N or vocabulary returns
 * FHIP_ERR_UNSUPPORTED so the caller's Common kernel produces the reference's result. */
int fhip_version(void);
/* Creates a context bound to `device` with its own non-blocking stream and a scratch arena. */
int fhip_context_create(int device, fhip_context* out);
int fhip_context_destroy(fhip_context ctx);
/* Enqueue on a caller stream (hipStream_t) instead; NULL restores the context's own stream. */
int fhip_context_set_stream(fhip_context ctx, void* stream);
void* fhip_context_stream(fhip_context ctx);
/* BackendContext::SetWorkspaceLimit (backend.h:80; runtime.cu:702-706, 810-846). */
int fhip_set_workspace_limit(fhip_context ctx, size_t bytes);
/* BackendContext::SetFp8WeightCacheLimit (backend.h:81): budget for prepared weights. */
int fhip_set_weight_cache_limit(fhip_context ctx, size_t bytes);
int fhip_weight_cache_bytes(fhip_context ctx, size_t* bytes);
/* BackendContext::Synchronize. */
int fhip_synchronize(fhip_context ctx);
const char* fhip_last_error(fhip_context ctx);
/* Name of the kernel path the last call ran (cf. LastCudaFp8MatmulBackend, runtime.h:100-105). */
const char* fhip_last_backend(fhip_context ctx);

/* ---- tensor memory (the device replicas a BackendContext keeps for a session's tensors:
 *      AcquireTensorDevice / SyncTensorToHost / ReleaseTensorDevice of the CUDA runtime,
 *      src/kernel/cuda/runtime.h:106-145) ------------------------------------------------------
 * alloc/free/upload/download are refused during capture (FHIP_ERR_STATE).  free waits for the work
 * queued on the context's stream; upload and download are ordered after it and return once the host
 * bytes have been read or written; copy (device to device) is stream-ordered and may be captured. */
int fhip_memory_alloc(fhip_context ctx, size_t bytes, void** out);
int fhip_memory_free(fhip_context ctx, void* ptr);
int fhip_memory_upload(fhip_context ctx, void* dst, const void* host, size_t bytes);
int fhip_memory_download(fhip_context ctx, void* host, const void* src, size_t bytes);
int fhip_memory_copy(fhip_context ctx, void* dst, const void* src, size_t bytes);

/* ---- prepared weights (Prepare(): x86 PackedFp8Rhs, linear_fp8.h:31-81;
 *      CUDA PackFp8WeightColumnMajor + cache, linear_kernels.cuh:211-221, 528-567) ---------- */
/* Re-lays an immutable linear weight out for the MFMA/GEMV kernels.  dtype: FP8E4M3, FP8E5M2
 * or INT8.  For INT8, scales/zero points (host arrays, 1 or N entries) travel with the weight
 * (the per-output-channel QuantizationParams of the weight tensor).  Identical (src, dtype,
 * k, n, layout, version) requests return the cached handle with its reference count raised. */
int fhip_weight_prepare(fhip_context ctx, const void* src, int dtype, int64_t k, int64_t n, int src_layout,
                        const float* scales, int64_t n_scale, const int32_t* zero_points, int64_t n_zp,
                        uint64_t version, fhip_weight* out);
/* The same preparation from host memory, at model load (a load-time pre-swizzle): the bytes are
 * uploaded, re-laid out as above and keyed on (host_src, dtype, K, N, layout, version), so a loader can
 * prepare every immutable weight once straight from the (mmapped) model file instead of at the first
 * Prepare() from a device tensor (src/model/model_io.cc, weight_store.cc; kernel.h:160-162).  The
 * transient device copy is freed before the call returns; the call synchronises the context's stream. */
int fhip_weight_prepare_host(fhip_context ctx, const void* host_src, int dtype, int64_t k, int64_t n, int src_layout,
                             const float* scales, int64_t n_scale, const int32_t* zero_points, int64_t n_zp,
                             uint64_t version, fhip_weight* out);

/* Conv2D weight [OC, IC/group, KH, KW] INT8 with per-output-channel scales (axis 0). */
int fhip_conv_weight_prepare(fhip_context ctx, const int8_t* src, int64_t oc, int64_t icg, int64_t kh,
                             int64_t kw, int32_t group, const float* scales, int64_t n_scale,
                             const int32_t* zero_points, int64_t n_zp, uint64_t version, fhip_weight* out);
int fhip_weight_release(fhip_weight w);
/* 1 when `w` was prepared from (src, version); used to reject stale handles after mutation. */
int fhip_weight_matches(fhip_weight w, const void* src, uint64_t version);

/* ---- Cast (CastKernel<*, FP8*>, src/kernel/common/cast.cc:62-165; x86/cast.cc:147-200) ----
 * src/dst dtypes: FP32, BF16, FP16, FP8E4M3, FP8E5M2.  FP8 sources decode as Dec(c)*src_scale,
 * FP8 destinations encode Enc(x / dst_scale) (kernel_io.h:58-78). */
int fhip_cast(fhip_context ctx, int src_dtype, const void* src, float src_scale, int64_t count, int dst_dtype,
              void* dst, float dst_scale);

/* ---- FP8 linear: MatMul/Gemm/FC <FP8E4M3|FP8E5M2> (common/matmul.cc:56-130, gemm.cc:62-100,
 *      fc.cc:48-73; x86/linear_fp8.cc:168-731) --------------------------------------------
 * out[m, n] = Enc( (alpha * sum_k A[m,k] * W[k,n] + beta * Dec(bias)*bias_scale) / out_scale )
 * with A[m,k] = Dec(a)*a_scale, W = Dec(w)*w_scale, fp32 accumulation.  MatMul: alpha = beta = 1,
 * no bias; FC: alpha = beta = 1.
 * a_dtype: the weight's FP8 dtype (a holds FP8 codes), or FHIP_BF16 / FHIP_FP32 -- then `a` holds
 * activations and is first encoded as Enc(x / a_scale), exactly the preceding Cast node.
 * out_dtype: the weight's FP8 dtype (the reference operator), or FHIP_BF16 / FHIP_FP32 -- then the
 * FP8 code is decoded again, Dec(code) * out_scale, exactly the following Cast(fp8 -> bf16) node.
 * Decode rows (m <= 16) run the bandwidth GEMV; larger m run the MFMA GEMM. */
int fhip_fp8_linear(fhip_context ctx, int a_dtype, const void* a, float a_scale, int64_t m, fhip_weight w,
                    float w_scale, const uint8_t* bias, float bias_scale, int bias_kind, float alpha, float beta,
                    int out_dtype, void* out, float out_scale);

/* ---- INT8 linear: MatMul/FC/Gemm <INT8> (common/matmul.cc:156-261, fc.cc:105-159,
 *      gemm.cc:136-198; x86/int8.cc:461-683) ----------------------------------------------
 * int32 accumulation of (a - zp_a) * (w - zp_w[n]), bias per `kind`, requantized exactly as the
 * Common kernels: round-half-away(real / double(s_out) + zp_out) with
 * real = acc * (double(s_a) * double(s_w[n])), clamped to [-128, 127].
 * Returns FHIP_ERR_UNSUPPORTED when an int32 partial sum could overflow (the Common kernel then
 * decides, returning -1 exactly where it overflows). */
int fhip_i8_linear(fhip_context ctx, int kind, const int8_t* a, float s_a, int32_t zp_a, int64_t m, fhip_weight w,
                   const int32_t* bias, int bias_kind, int32_t bias_abs_max, float alpha, float beta, int8_t* out,
                   float s_out, int32_t zp_out);
/* The same INT8 linear followed by the graph's DequantizeLinear of its output, in one launch
 * (common/quantize_linear_utils.h:291-341, per tensor): out_dtype FHIP_INT8 is fhip_i8_linear;
 * FHIP_FP32 / FHIP_FP16 / FHIP_BF16 write float((q - dq_zp) * dq_scale) encoded as DequantizeLinear does,
 * where q is the INT8 result fhip_i8_linear would write (out_scale / out_zp).  Equal, value for value, to
 * the two nodes run one after the other (the Q -> Gemm -> DQ chain of the INT8 export). */
int fhip_i8_linear_ex(fhip_context ctx, int kind, const int8_t* a, float s_a, int32_t zp_a, int64_t m, fhip_weight w,
                      const int32_t* bias, int bias_kind, int32_t bias_abs_max, float alpha, float beta, int out_dtype,
                      void* out, float s_out, int32_t zp_out, float dq_scale, int32_t dq_zp);

/* ---- INT8 Conv2D as implicit GEMM (common/conv2d.cc:482-581; x86/int8.cc:684-2346) ------- */
int fhip_i8_conv2d(fhip_context ctx, const int8_t* in, int64_t n, int64_t c, int64_t h, int64_t w, int layout,
                   float s_in, int32_t zp_in, fhip_weight wt, const int32_t* bias, int32_t bias_abs_max,
                   int32_t stride_h, int32_t stride_w, int32_t pad_h, int32_t pad_w, int32_t dil_h, int32_t dil_w,
                   int8_t* out, int64_t oh, int64_t ow, float s_out, int32_t zp_out);

/* ---- QuantizeLinear / DequantizeLinear (common/quantize_linear_utils.h:187-341) ----------
 * Element i uses parameter index (i / inner) % channels (channels = 1: per tensor).  Scales and
 * zero points are host arrays of `channels` entries (zero points: 1 or `channels`). */
int fhip_quantize_linear(fhip_context ctx, int src_dtype, const void* src, int64_t count, int64_t channels,
                         int64_t inner, const float* scales, const int32_t* zero_points, int64_t n_zp,
                         int8_t* out);
int fhip_dequantize_linear(fhip_context ctx, const int8_t* src, int64_t count, int64_t channels, int64_t inner,
                           const float* scales, const int32_t* zero_points, int64_t n_zp, int dst_dtype,
                           void* out);

/* ---- QwenGemmArgmax (operator/qwen_gemm_argmax_op.cc:28-113; common/qwen_gemm_argmax.cc:28-49;
 *      x86/linear.cc:603-760; cuda/qwen_gemm_argmax.cu:82-171) -------------------------------
 * For each of m rows (the reference operator takes m = 1; rows are independent): fp32 dot of the
 * BF16 row with every vocabulary row of w [v, k], rounded to BF16; NaN skipped; first strict
 * maximum (lowest index among equal values, +0 == -0); 0 when every value is NaN.
 * logits (optional, [m, v] fp32) receives the fp32 sums.  Rows of up to 64 KiB (K <= 32768), K % 8 == 0,
 * m <= 16, v < 2^32; otherwise FHIP_ERR_UNSUPPORTED. */
int fhip_bf16_gemv_argmax(fhip_context ctx, const uint16_t* a, int64_t m, int64_t k, const uint16_t* w, int64_t v,
                          int64_t* tokens, float* logits);
/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the same computation
 * and results as fhip_bf16_gemv_argmax, but the kernels' ticket counters and per-block partial
 * keys live in a static device array of 128 KiB per GPU (set up once per device by
 * fhip_context_create) instead of the context's workspace, so the call allocates nothing.
 * Returns FHIP_ERR_UNSUPPORTED when the vocabulary needs more partial keys than the array holds
 * (not the case up to 2 blocks per CU on 480 CUs).  Every context on one GPU shares the array:
 * calls that overlap on one GPU (two streams, two contexts, two host threads) race and must be
 * ordered by the caller.  Each call clears the counters with a kernel before it starts. */
int fhip_bf16_gemv_argmax_noalloc(fhip_context ctx, const uint16_t* a, int64_t m, int64_t k, const uint16_t* w,
                                  int64_t v, int64_t* tokens, float* logits);
/* FP8 head: Gemm(transB) with out_scale, Cast(fp8 -> bf16), greedy selection
 * (x86/linear_fp8.cc:733-1004; qwen_gemm_argmax_fusion_pass.cc:142-181).  K <= 65536, K % 16 == 0. */
int fhip_fp8_gemv_argmax(fhip_context ctx, int dtype, const uint8_t* a, float a_scale, int64_t m, int64_t k,
                         const uint8_t* w, float w_scale, int64_t v, float out_scale, int64_t* tokens);

/* ---- execution capture (BackendContext::Capture -> ExecutionCapture, backend.h:29-41, 84;
 *      CUDA precedent backend.cc:80-123) ----------------------------------------------------- */
int fhip_capture_begin(fhip_context ctx);
int fhip_capture_end(fhip_context ctx, fhip_graph* out);
int fhip_graph_launch(fhip_context ctx, fhip_graph g);
int fhip_graph_destroy(fhip_graph g);

#ifdef __cplusplus
}
#endif
#endif /* FHIP_H */
