/*
 * sneppx_quantization.h - the reference's C quantization API, served by HIP.
 *
 * Drop-in for include/neural_core/kernel/quantization.h (reference).  Same
 * enum ordinals, struct layouts, names, argument order, host pointers,
 * caller-allocated outputs and 0 / -1 return convention.  Every numeric
 * function runs its arithmetic in hand-written gfx950 kernels (copy in,
 * kernel, copy out; synchronous) and returns the reference's bits.  The FP8
 * scalar codecs and the two metadata helpers are host functions: there is
 * no device work in them.
 *
 * Library: libsneppx_quant.so (sneppx-alg_amd/).  A failed HIP call makes a
 * function return -1; SNEPPX_qlinear_last_error() then names the cause.
 *
 * Two guarded parts.  The types sit under the reference header's own guard
 * (SNEPPX_QUANTIZATION_H): they are the reference's types, so a translation
 * unit that already included the reference header keeps its definitions.
 * The prototypes sit under their own guard, so in such a unit they
 * redeclare the reference's 22 functions, and any difference in a return or
 * argument type is a compile error (tests/test_abi.py builds exactly that).
 */
#ifndef SNEPPX_QUANTIZATION_H
#define SNEPPX_QUANTIZATION_H

#include <stddef.h>
#include <stdint.h>

/* multidimensional_tensor_engine.h:27-41 (ordinal ABI) */
#ifndef SNEPPX_DTYPE_DEFINED
#define SNEPPX_DTYPE_DEFINED
typedef enum {
    SNEPPX_FLOAT32, SNEPPX_FLOAT64, SNEPPX_FLOAT16, SNEPPX_BFLOAT16, SNEPPX_FLOAT8,
    SNEPPX_INT32, SNEPPX_INT64, SNEPPX_INT16, SNEPPX_INT8, SNEPPX_UINT8, SNEPPX_BOOL,
    SNEPPX_COMPLEX64, SNEPPX_COMPLEX128,
} SNEPPXDtype;
#endif

/* quantization.h:24-33 */
typedef enum {
    SNEPPX_QUANT_NONE = 0,
    SNEPPX_QUANT_INT8_SYM,
    SNEPPX_QUANT_INT8_ASYM,
    SNEPPX_QUANT_INT4_SYM,
    SNEPPX_QUANT_FP8_E4M3,
    SNEPPX_QUANT_FP8_E5M2,
    SNEPPX_QUANT_AWQ,
    SNEPPX_QUANT_GPTQ,
} SNEPPXQuantMode;

/* quantization.h:35-40 */
typedef enum {
    SNEPPX_QUANT_PER_TENSOR = 0,
    SNEPPX_QUANT_PER_CHANNEL,
    SNEPPX_QUANT_PER_GROUP,
    SNEPPX_QUANT_PER_TOKEN,
} SNEPPXQuantGranularity;

/* quantization.h:42-48 */
typedef struct {
    float scale;
    int32_t zero_point;
    float qmin;
    float qmax;
    float scale_max;
} SNEPPXQuantParams;

/* quantization.h:50-55 */
typedef struct {
    float* scales;
    int32_t* zero_points;
    size_t num_params;
    SNEPPXQuantGranularity granularity;
} SNEPPXQuantState;

/* quantization.h:57-63 */
typedef struct {
    float* weights;
    float* hessian;
    size_t rows;
    size_t cols;
    int group_size;
} SNEPPXGPTQState;

#endif /* SNEPPX_QUANTIZATION_H: the reference's types */

#ifndef SNEPPX_QUANTIZATION_API_H
#define SNEPPX_QUANTIZATION_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* replaces quantization.h:80-81 / quantize_int8.c:43-65 */
int SNEPPX_quantize_int8_sym(const float* input, int8_t* output,
                             size_t n, float* scale_out);
/* replaces quantization.h:92-93 / quantize_int8.c:77-85 */
int SNEPPX_dequantize_int8_sym(const int8_t* input, float* output,
                               size_t n, float scale);
/* replaces quantization.h:107-108 / quantize_int8.c:98-123 */
int SNEPPX_quantize_int8_asym(const float* input, int8_t* output,
                              size_t n, float* scale_out, int32_t* zp_out);
/* replaces quantization.h:120-121 / quantize_int8.c:136-144 */
int SNEPPX_dequantize_int8_asym(const int8_t* input, float* output,
                                size_t n, float scale, int32_t zp);
/* replaces quantization.h:135-137 / quantize_int8.c:157-177 */
int SNEPPX_quantize_int8_channel(const float* input, int8_t* output,
                                 size_t rows, size_t cols, float* scales_out);
/* replaces quantization.h:150-151 / quantize_int8.c:189-218 */
int SNEPPX_quantize_int4_sym(const float* input, uint8_t* output,
                             size_t n, float* scale_out);
/* replaces quantization.h:162-163 / quantize_int8.c:230-247 */
int SNEPPX_dequantize_int4_sym(const uint8_t* input, float* output,
                               size_t n, float scale);

/* replaces quantization.h:173 / quantize_fp8.c:41-69 (host codec) */
uint8_t SNEPPX_float_to_fp8_e4m3(float value);
/* replaces quantization.h:181 / quantize_fp8.c:78-100 (host codec) */
float SNEPPX_fp8_e4m3_to_float(uint8_t fp8);
/* replaces quantization.h:191 / quantize_fp8.c:111-118 */
int SNEPPX_quantize_fp8_e4m3(const float* input, uint8_t* output, size_t n);
/* replaces quantization.h:201 / quantize_fp8.c:129-136 */
int SNEPPX_dequantize_fp8_e4m3(const uint8_t* input, float* output, size_t n);
/* replaces quantization.h:211 / quantize_fp8.c:146-172 (host codec) */
uint8_t SNEPPX_float_to_fp8_e5m2(float value);
/* replaces quantization.h:219 / quantize_fp8.c:180-201 (host codec) */
float SNEPPX_fp8_e5m2_to_float(uint8_t fp8);
/* replaces quantization.h:229 / quantize_fp8.c:212-219 */
int SNEPPX_quantize_fp8_e5m2(const float* input, uint8_t* output, size_t n);
/* replaces quantization.h:239 / quantize_fp8.c:230-237 */
int SNEPPX_dequantize_fp8_e5m2(const uint8_t* input, float* output, size_t n);

/* replaces quantization.h:253-254 / awq.c:106-120 (weights updated in place) */
int SNEPPX_awq_scale_weights(float* weights, size_t rows, size_t cols,
                             const float* act_scales, float* scale_out);
/* replaces quantization.h:268-270 / awq.c:135-161 (act_scales may be NULL) */
int SNEPPX_awq_quantize(const float* weights, int8_t* qweight,
                        const float* act_scales, float* scales,
                        size_t rows, size_t cols, int group_size);

/* replaces quantization.h:288-291 / gptq.c:189-239 (qweight receives int8 bytes) */
int SNEPPX_gptq_quantize(float* weights, size_t rows, size_t cols,
                         int group_size, int bits,
                         SNEPPXDtype* qweight, float* scales,
                         int32_t* zeros, int sym);
/* replaces quantization.h:302-303 / gptq.c:55-79 */
int SNEPPX_gptq_compute_hessian(float* hessian, const float* activation,
                                size_t n, size_t dim);
/* replaces quantization.h:318-320 / gptq.c:134-172 (w updated in place) */
int SNEPPX_gptq_quantize_block(float* w, float* h_inv,
                               float* qw, float* scale, int32_t* zero,
                               size_t block_size, int bits, int sym);

/* replaces quantization.h:331 / awq.c:171-201 */
int SNEPPX_quant_params_create(SNEPPXQuantParams* params, SNEPPXQuantMode mode);
/* replaces quantization.h:339 / awq.c:210-223 */
const char* SNEPPX_quant_mode_name(SNEPPXQuantMode mode);

#ifdef __cplusplus
}
#endif

#endif /* SNEPPX_QUANTIZATION_API_H */
