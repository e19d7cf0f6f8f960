/*
 * feather_oracle.h -- CPU restatement of Feather's Common-backend semantics for the
 * quantized linear hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP backend.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The shipped library (infer_amd/libfhip.so) never links, loads or calls it.
 *
 * Every function names the reference file:line it restates (paths are relative to the
 * Feather source tree, JPChen2000/Infer).
 *
 * Status convention (as the reference's kernels): 0 = ok, -1 = the reference kernel
 * would return -1 (invalid arguments, int32 overflow, non-finite requantization).
 */
#ifndef FEATHER_ORACLE_H
#define FEATHER_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Feather DataType values (include/util/types.h:32-47). */
enum {
    FO_INT8 = 1, FO_UINT8 = 2, FO_FP16 = 3, FO_FP32 = 4, FO_INT32 = 5, FO_INT64 = 6,
    FO_BF16 = 11, FO_FP8E4M3 = 12, FO_FP8E5M2 = 13
};

/* Bias layouts of the FP8/INT8 linear kernels. */
enum { FO_BIAS_NONE = 0, FO_BIAS_VECTOR = 1, FO_BIAS_MATRIX = 2 };

/* ---- codecs ---------------------------------------------------------------------------- */
uint8_t fo_fp8_encode(int dtype, float value);          /* include/util/fp8.h:66-211 */
float   fo_fp8_decode(int dtype, uint8_t code);         /* include/util/fp8.h:158-200 */
uint16_t fo_bf16_encode(float value);                   /* include/util/bf16.h:36-46 (NaN quieted) */
float    fo_bf16_decode(uint16_t bits);                 /* include/util/bf16.h:27-32 */
uint16_t fo_bf16_encode_plain(float value);             /* quantize_linear_utils.h:110-117 (no NaN quieting) */
uint16_t fo_fp16_encode(float value);                   /* quantize_linear_utils.h:70-101 (DequantizeLinear) */
uint16_t fo_fp16_encode_cast(float value);              /* include/util/fp16.h FloatToHalf (Cast) */
float    fo_fp16_decode(uint16_t bits);                 /* quantize_linear_utils.h:50-68 */

/* Vectorised codecs for the tests (count elements). */
void fo_fp8_encode_array(int dtype, const float* in, uint8_t* out, int64_t count);
void fo_fp8_encode_bits_range(int dtype, uint32_t first_bits, int64_t count, uint8_t* out);
void fo_bf16_encode_array(const float* in, uint16_t* out, int64_t count);
void fo_bf16_encode_bits_range(uint32_t first_bits, int64_t count, uint16_t* out);
void fo_bf16_plain_encode_bits_range(uint32_t first_bits, int64_t count, uint16_t* out);
/* cast_rule 1: fo_fp16_encode_cast (Cast), 0: fo_fp16_encode (DequantizeLinear) */
void fo_fp16_encode_bits_range(int cast_rule, uint32_t first_bits, int64_t count, uint16_t* out);

/* ---- Cast (src/kernel/common/cast.cc:62-165) ------------------------------------------ */
/* bf16/fp32 -> fp8 code with the output scale: code = Enc(x / out_scale). */
int fo_cast_to_fp8(int src_dtype, const void* src, int64_t count, int fp8_dtype, float out_scale, uint8_t* out);
/* fp8 code -> bf16/fp32: x = Dec(code) * in_scale, then the destination encoder. */
int fo_cast_from_fp8(int fp8_dtype, const uint8_t* src, float in_scale, int64_t count, int dst_dtype, void* out);

/* ---- FP8 linear ------------------------------------------------------------------------ */
/* MatMul (src/kernel/common/matmul.cc:56-130): a [M,K], b [K,N] row-major, fp32 sum in
 * K order of (Dec(a)*sa)*(Dec(b)*sb), out = Enc(sum / s_out). */
int fo_fp8_matmul(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb,
                  int64_t m, int64_t k, int64_t n, uint8_t* out, float s_out);
/* Gemm (src/kernel/common/gemm.cc:62-100): b is [N,K] when trans_b else [K,N];
 * sum *= alpha; sum += beta * Dec(bias)*s_bias; out = Enc(sum / s_out). */
int fo_fp8_gemm(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb, int trans_b,
                const uint8_t* bias, float s_bias, int bias_kind, float alpha, float beta,
                int64_t m, int64_t k, int64_t n, uint8_t* out, float s_out);
/* FC (src/kernel/common/fc.cc:48-73): w [K,N]; sum += Dec(bias)*s_bias (no alpha/beta). */
int fo_fp8_fc(int dtype, const uint8_t* a, float sa, const uint8_t* w, float sw,
              const uint8_t* bias, float s_bias, int bias_kind,
              int64_t m, int64_t k, int64_t n, uint8_t* out, float s_out);
/* fp32 sums only (before the FP8 output encode); used to separate order effects. */
int fo_fp8_gemm_f32(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb, int trans_b,
                    int64_t m, int64_t k, int64_t n, float* sums);

/* ---- INT8 linear ----------------------------------------------------------------------- */
enum { FO_I8_MATMUL = 0, FO_I8_FC = 1, FO_I8_GEMM = 2 };
/* kind MATMUL: matmul.cc:156-261 (b [K,N], per-channel axis = last, no bias)
 * kind FC:     fc.cc:105-159     (w [K,N], int32 bias added in int64, overflow checked)
 * kind GEMM:   gemm.cc:136-198   (b [N,K] if trans_b else [K,N]; acc = alpha*dot + beta*bias in double)
 * w_scales/w_zps have n_wscale / n_wzp entries (1 = per-tensor).  acc_out (optional) gets the
 * int32 dot product (without bias) for every output. */
int fo_i8_linear(int kind, const int8_t* a, float s_a, int32_t zp_a,
                 const int8_t* w, int trans_b, const float* w_scales, int64_t n_wscale,
                 const int32_t* w_zps, int64_t n_wzp,
                 const int32_t* bias, int bias_kind, float alpha, float beta,
                 int64_t m, int64_t k, int64_t n,
                 int8_t* out, float s_out, int32_t zp_out, int32_t* acc_out);

/* ---- INT8 Conv2D (src/kernel/common/conv2d.cc:482-581) -------------------------------- */
/* layout 0 = NCHW, 1 = NHWC for input and output; weight [OC, IC/group, KH, KW]. */
int fo_i8_conv2d(const int8_t* in, int64_t n, int64_t c, int64_t h, int64_t w, int layout,
                 float s_in, int32_t zp_in,
                 const int8_t* wt, int64_t oc, int64_t kh, int64_t kw,
                 const float* w_scales, int64_t n_wscale, const int32_t* w_zps, int64_t n_wzp,
                 const int32_t* bias,
                 int32_t stride_h, int32_t stride_w, int32_t pad_h, int32_t pad_w,
                 int32_t dil_h, int32_t dil_w, int32_t group,
                 int8_t* out, int64_t oh, int64_t ow, float s_out, int32_t zp_out);

/* ---- QuantizeLinear / DequantizeLinear (quantize_linear_utils.h:187-341) --------------- */
/* src_dtype FP32/FP16/BF16; dims[rank]; scales n_scale (1 = per tensor); zps n_zp; axis
 * (negative = from the back) used only when n_scale > 1. */
int fo_quantize_linear(int src_dtype, const void* src, const int64_t* dims, int rank,
                       const float* scales, int64_t n_scale, const int32_t* zps, int64_t n_zp,
                       int64_t axis, int8_t* out);
int fo_dequantize_linear(const int8_t* src, const int64_t* dims, int rank,
                         const float* scales, int64_t n_scale, const int32_t* zps, int64_t n_zp,
                         int64_t axis, int dst_dtype, void* out);

/* ---- QwenGemmArgmax -------------------------------------------------------------------- */
/* BF16 (src/kernel/common/qwen_gemm_argmax.cc:30-49): one row a [K], b [V,K].
 * logits (optional) receives the fp32 sums. */
int64_t fo_bf16_gemm_argmax(const uint16_t* a, const uint16_t* b, int64_t k, int64_t v, float* logits);
/* FP8 terminal head: the exported graph Gemm(transB, out scale) -> Cast(fp8->bf16) ->
 * greedy selection (src/kernel/x86/linear_fp8.cc:757-788; qwen_gemm_argmax_fusion_pass.cc). */
int64_t fo_fp8_gemm_argmax(int dtype, const uint8_t* a, float sa, const uint8_t* b, float sb,
                           int64_t k, int64_t v, float s_out);

/* ---- threading for the CPU-baseline leg ----------------------------------------------- */
/* The x86 INT8 conv and QuantizeLinear use every OpenMP thread (src/kernel/x86/int8.cc:2331-2334;
 * quantize_linear_utils.h:37-49); the conv and quantize restatements here parallelise the same
 * way.  Returns the thread count now in effect. */
int fo_set_threads(int threads);

#ifdef __cplusplus
}
#endif
#endif
