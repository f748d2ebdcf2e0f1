/*
 * oracle.h - CPU restatement of the SNEPPX-Alg quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker (or as the timed CPU
 * baseline), never as the thing measured or shipped.
 *
 * Two groups of functions:
 *
 *  1. Restatements of the reference C functions (kernel/quantization/
 *     {quantize_int8,quantize_fp8,awq,gptq}.c, the fp32 matmul order of kernel/tensor/tensor.c:1820-1823 and the
 *     fake-quant rule of kernel/tensor/tensor.c:2180-2195).  Same argument
 *     meaning, same return codes, same bits.  Each definition cites the
 *     reference lines it follows.  Pinned against oracle/_ref (the reference
 *     sources compiled unchanged) and the golden fixtures in tests/golden/.
 *
 *  2. Build-defined formats that the reference lacks (the W4A16 AWQ-style
 *     uint4 format, GPTQ act-order with g_idx, W8A8 int8/fp8 GEMM, bf16/fp16
 *     conversions).  Each is stated in closed
 *     form and pinned by the invariants listed in its comment.
 *
 * Pinned build flags: -O2 -ffp-contract=off (oracle/Makefile).
 */
#ifndef SNX_ORACLE_H
#define SNX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference ABI values (quantization.h:24-63, tensor header :27-41) -- */
enum { ORC_QUANT_NONE = 0, ORC_QUANT_INT8_SYM, ORC_QUANT_INT8_ASYM,
       ORC_QUANT_INT4_SYM, ORC_QUANT_FP8_E4M3, ORC_QUANT_FP8_E5M2,
       ORC_QUANT_AWQ, ORC_QUANT_GPTQ };

typedef struct {
    float scale;
    int32_t zero_point;
    float qmin;
    float qmax;
    float scale_max;
} orc_quant_params;

/* ---- 1. reference restatements ------------------------------------------ */
int orc_quantize_int8_sym(const float* in, int8_t* out, size_t n, float* scale_out);
int orc_dequantize_int8_sym(const int8_t* in, float* out, size_t n, float scale);
int orc_quantize_int8_asym(const float* in, int8_t* out, size_t n,
                           float* scale_out, int32_t* zp_out);
int orc_dequantize_int8_asym(const int8_t* in, float* out, size_t n,
                             float scale, int32_t zp);
int orc_quantize_int8_channel_rne(const float* in, int8_t* out, size_t rows, size_t cols,
                                  float* scales_out);
int orc_quantize_int8_channel(const float* in, int8_t* out, size_t rows,
                              size_t cols, float* scales_out);
int orc_quantize_int4_sym(const float* in, uint8_t* out, size_t n, float* scale_out);
int orc_dequantize_int4_sym(const uint8_t* in, float* out, size_t n, float scale);

uint8_t orc_float_to_fp8_e4m3(float v);
float   orc_fp8_e4m3_to_float(uint8_t c);
int     orc_quantize_fp8_e4m3(const float* in, uint8_t* out, size_t n);
int     orc_dequantize_fp8_e4m3(const uint8_t* in, float* out, size_t n);
uint8_t orc_float_to_fp8_e5m2(float v);
float   orc_fp8_e5m2_to_float(uint8_t c);
int     orc_quantize_fp8_e5m2(const float* in, uint8_t* out, size_t n);
int     orc_dequantize_fp8_e5m2(const uint8_t* in, float* out, size_t n);

int orc_awq_scale_weights(float* weights, size_t rows, size_t cols,
                          const float* act_scales, float* scale_out);
int orc_awq_quantize(const float* weights, int8_t* qweight, const float* act_scales,
                     float* scales, size_t rows, size_t cols, int group_size);

int orc_gptq_compute_hessian(float* h, const float* act, size_t n, size_t dim);
int orc_gptq_quantize_block(float* w, float* h_inv, float* qw, float* scale,
                            int32_t* zero, size_t block_size, int bits, int sym);
/* qweight is written as int8 bytes (the reference types it SNEPPXDtype*). */
int orc_gptq_quantize(float* weights, size_t rows, size_t cols, int group_size,
                      int bits, void* qweight, float* scales, int32_t* zeros, int sym);
/* Literal restatement (Cholesky of I, sequential error feedback), O(g^2) per
 * group; used only to pin the closed form that orc_gptq_quantize uses. */
int orc_gptq_quantize_literal(float* weights, size_t rows, size_t cols,
                              int group_size, int bits, void* qweight,
                              float* scales, int32_t* zeros, int sym);
int orc_cholesky_inv(float* h, size_t dim);

int orc_quant_params_create(orc_quant_params* p, int mode);
const char* orc_quant_mode_name(int mode);

/* weights.c:225-252 model-zoo int8 (multiplier 127/max, truncation) */
int orc_quantize_int8_modelzoo(const float* in, int8_t* out, size_t n, float* mult_out);

/* tensor.c:2180-2195 forward rule; returns -1 where the reference returns NULL */
int orc_fake_quant(const float* in, float* out, size_t n, float scale, int bits);

/* fp32 linear in the reference's order: y[m][n] = sum_k a[m][k]*b[k][n],
 * k ascending, starting from 0.0f (tensor.c:1820-1823, B is [K,N]). */
void orc_matmul_kn(const float* a, const float* b, float* y,
                   size_t M, size_t K, size_t N);
/* Same arithmetic with B stored [N,K] (output-major, y = a . W^T). */
void orc_matmul_nk(const float* a, const float* w, float* y,
                   size_t M, size_t K, size_t N);

/* ---- 2. build-defined formats -------------------------------------------- */
/* scalar helpers */
uint16_t orc_f32_to_bf16(float f);     /* round-to-nearest-even, NaN kept quiet */
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);      /* IEEE binary16, round-to-nearest-even */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_w4_scale_to_f16(float s); /* RNE, clamped to [2^-24, 65504] */

/* C2 / a20: W4 AWQ-style asymmetric uint4, group g along K.
 * qweight u32[N][K/8] (k at bits 4*(k%8)), scales f16[N][K/g],
 * qzeros u32[N][ceil(K/g/8)] (group j at bits 4*(j%8)).  K % 8 == 0, K % g == 0. */
int orc_w4_awq_quantize(const float* w, size_t N, size_t K, int group,
                        uint32_t* qweight, uint16_t* scales, uint32_t* qzeros);
/* C3 / a21: GPTQ act-order symmetric int4, zero 8 implicit.
 * Group of column k is g_idx[k]; scales f16[N][G] with G = max(g_idx)+1.
 * Codes follow orc_gptq_quantize(bits=4, sym=1) on the columns of each group
 * taken in ascending k, stored as code+8 clamped to [0,15]. */
int orc_w4_gptq_quantize(const float* w, const int32_t* g_idx, size_t N, size_t K,
                         size_t G, uint32_t* qweight, uint16_t* scales);
/* dequantize either format to fp32 [N][K]; qzeros NULL means symmetric zero 8 */
int orc_w4_dequantize(const uint32_t* qweight, const uint16_t* scales,
                      const uint32_t* qzeros, const int32_t* g_idx,
                      size_t N, size_t K, int group, float* w_out);
/* y[m][n] = sum_k bf16(x[m][k]) * deq[n][k] in fp32, k ascending */
int orc_w4a16_linear(const uint16_t* x_bf16, const uint32_t* qweight,
                     const uint16_t* scales, const uint32_t* qzeros,
                     const int32_t* g_idx, size_t M, size_t N, size_t K,
                     int group, float* y);

/* Bias term of QuantizedLinear.forward (quantization.py:451-454):
 * y[m][n] = y[m][n] + bias[n], one fp32 add after the product. */
void orc_add_bias(float* y, const float* bias, size_t M, size_t N);

/* C1 / a19: y[m][n] = sum_k x[m][k] * ((float)q[n][k] * s[n]), k ascending */
int orc_w8_linear(const float* x, const int8_t* q, const float* s,
                  size_t M, size_t N, size_t K, float* y);

/* C4 / a22 */
void orc_i8_gemm_i32(const int8_t* A, const int8_t* W, int32_t* C,
                     size_t M, size_t N, size_t K);
/* out[m][n] = ((float)acc * sA[m]) * sW[n] (fp32) */
void orc_w8a8_epilogue(const int32_t* acc, const float* sA, const float* sW,
                       size_t M, size_t N, float* out);
/* per-tensor fp8 (build-defined): s = amax/240 (1 if
 * amax < FLT_MIN), code = e4m3(x / s) with the reference encoder of
 * quantize_fp8.c:41-69.  Pinned by planted tensors whose x / s and
 * x * (1/s) give different codes. */
int orc_quantize_fp8_e4m3_scaled(const float* in, uint8_t* out, size_t n, float* scale_out);
/* out[m][n] = (sum_k dec(A)*dec(W), k ascending) * sA * sW */
void orc_fp8_gemm(const uint8_t* A, const uint8_t* W, float sA, float sW,
                  size_t M, size_t N, size_t K, float* out);

#ifdef __cplusplus
}
#endif
#endif
