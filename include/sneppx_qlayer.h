/*
 * sneppx_qlayer.h - quantized linear layers for the reference's linear call
 * sites.
 *
 * The reference's inference linears are fp32 matmuls y = x . W with W stored
 * [K, N] (K inputs, N outputs; kernel/attention/attention.c:71-80 creates
 * w_q/w_k/w_v as [d_model, heads*head_dim], matmul_3d at attention.c:324-345
 * multiplies [B, S, D] by [D, Dk]; the LM head at
 * kernel/inference/inference_engine.c:264 is SNEPPX_tensor_matmul(flat,
 * unembed_weight [d_model, vocab])).  A SNEPPXQLayer holds one such W
 * quantized on the device in the layout of sneppx_qlinear.h ([N, K],
 * output-major) and computes the same product:
 *
 *   attention.c:366   q = matmul_3d(x, w->w_q)
 *   becomes           SNEPPX_qlayer_matmul_host(wq, x->data, q->data, B * S)
 *   (host buffers, synchronous: the literal drop-in), or
 *                     SNEPPX_qlayer_forward_f32(wq, d_x, d_q, B * S, stream)
 *   when activations stay on the device between layers.
 *
 * Formats: SNEPPX_QLAYER_W8 = per-output-channel int8 codes, fp32 math
 * (SNEPPX_qlinear_w8_gemv; y within 1e-4 of the fp32 product on the
 * dequantized weights); SNEPPX_QLAYER_W4 = AWQ-style asymmetric uint4 with
 * groups of `group` inputs (SNEPPX_qlinear_w4a16: activations are rounded to
 * bf16 on the way in, y within 1e-2).  Layers loaded from a file may also be
 * GPTQ act-order (g_idx); those are prepared once at load.
 *
 * Return codes as in sneppx_qlinear.h (0 / -1, NULL for constructors; text in
 * SNEPPX_qlinear_last_error()).
 */
#ifndef SNEPPX_QLAYER_H
#define SNEPPX_QLAYER_H

#include <stddef.h>
#include <stdint.h>

#include "sneppx_qlinear.h"
#include "sneppx_qstore.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { SNEPPX_QLAYER_W8 = 0, SNEPPX_QLAYER_W4 = 1 } SNEPPXQLayerFormat;

typedef struct SNEPPXQLayer SNEPPXQLayer;

/* Quantize W [K][N] fp32 (host pointer, the reference's layout) on the
 * device; `group` is used by SNEPPX_QLAYER_W4 (K % group == 0, group % 8 ==
 * 0).  Synchronous. */
SNEPPXQLayer* SNEPPX_qlayer_create_kn(const float* w_kn, size_t K, size_t N,
                                      SNEPPXQLayerFormat format, int group, SNEPPXStream stream);

/* Same from a device copy of W [K][N]. */
SNEPPXQLayer* SNEPPX_qlayer_create_kn_device(const float* d_w_kn, size_t K, size_t N,
                                             SNEPPXQLayerFormat format, int group,
                                             SNEPPXStream stream);

/* Load layer <prefix> written by SNEPPX_qlayer_save or the qstore helpers
 * (W4 with or without zero points or g_idx; W8). */
SNEPPXQLayer* SNEPPX_qlayer_load(const SNEPPXQStore* st, const char* prefix, SNEPPXStream stream);

int SNEPPX_qlayer_save(const SNEPPXQLayer* layer, SNEPPXQStoreWriter* w, const char* prefix,
                       SNEPPXStream stream);

void SNEPPX_qlayer_destroy(SNEPPXQLayer* layer);

/* Bias of the layer, fp32 [N] (the `bias` of QuantizedLinear,
 * bindings/python/.../quantization.py:451-454): every forward then returns
 * x . W + bias.  From host memory (synchronous) or device memory; NULL
 * removes it.  SNEPPX_qlayer_save writes it as <prefix>.bias and
 * SNEPPX_qlayer_load reads it back when present. */
int SNEPPX_qlayer_set_bias(SNEPPXQLayer* layer, const float* bias, SNEPPXStream stream);
int SNEPPX_qlayer_set_bias_device(SNEPPXQLayer* layer, const float* d_bias, SNEPPXStream stream);

/* K, N and format of a layer. */
size_t SNEPPX_qlayer_in_features(const SNEPPXQLayer* layer);
size_t SNEPPX_qlayer_out_features(const SNEPPXQLayer* layer);
int SNEPPX_qlayer_format(const SNEPPXQLayer* layer);

/* y[M][N] = x[M][K] . W, fp32 device buffers, asynchronous on `stream`. */
int SNEPPX_qlayer_forward_f32(const SNEPPXQLayer* layer, const float* d_x, float* d_y, size_t M,
                              SNEPPXStream stream);

/* The same with bf16 activations in and out (W4 layers; W8 layers take fp32
 * activations and return -1 here). */
int SNEPPX_qlayer_forward_bf16(const SNEPPXQLayer* layer, const uint16_t* d_x, uint16_t* d_y,
                               size_t M, SNEPPXStream stream);

/* Host buffers in and out (the reference's tensors): copy x in, run, copy y
 * out, return when y is in host memory.  Reentrant like the matmul_3d it
 * replaces: each call stages its buffers in device memory of its own, on a
 * stream of its own, so host threads may call it at the same time (on one
 * layer or several). */
int SNEPPX_qlayer_matmul_host(const SNEPPXQLayer* layer, const float* x, float* y, size_t M);

#ifdef __cplusplus
}
#endif

#endif /* SNEPPX_QLAYER_H */
