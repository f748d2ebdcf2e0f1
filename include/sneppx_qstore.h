/*
 * sneppx_qstore.h - quantized weights on disk (safetensors) and the model-zoo
 * INT8 path.
 *
 * The reference reads and writes safetensors with fs/format/safetensors.c
 * (SNEPPX_safetensors_*; dtype codes SNEPPXSafetensorsDType in
 * fs/format/safetensors.h:24-37) but has no quantized-weight format and its
 * loaders are stubs (algorithms/model_zoo/weights.c:268-291).  This file
 * defines one, readable and writable by any conforming safetensors tool:
 *
 *   <prefix>.qweight   I32 [N, K/8]        W4 codes, element k at bits 4*(k%8)
 *   <prefix>.scales    F16 [N, G]          per-group scales
 *   <prefix>.qzeros    I32 [N, ceil(G/8)]  zero points, group j at bits 4*(j%8)
 *                                          (absent for symmetric codes, zero 8)
 *   <prefix>.g_idx     I32 [K]             GPTQ act-order group of column k
 *                                          (absent for contiguous groups)
 *   <prefix>.weight    I8  [N, K]          W8 codes (per-output-channel)
 *   <prefix>.weight_scale F32 [N]          W8 scales
 *   __metadata__       "<prefix>.format" = "w4" | "w8", "<prefix>.group_size"
 *
 * These are the layouts the device entry points of sneppx_qlinear.h take, so
 * a load is a straight copy into device memory.  Files are memory-mapped;
 * tensor data is copied host->device from the mapping.
 *
 * Reading accepts files whose header length excludes the zero padding the
 * reference's writer appends after the JSON (safetensors.c:466-474 writes the
 * unpadded length, then pads to 8 bytes): the data block is located from the
 * file size.  Writing follows the safetensors rule (header padded with spaces,
 * length included), which both readers accept.
 *
 * All functions return 0 on success and -1 on error (NULL for constructors);
 * the reason is in SNEPPX_qlinear_last_error().
 */
#ifndef SNEPPX_QSTORE_H
#define SNEPPX_QSTORE_H

#include <stddef.h>
#include <stdint.h>

#include "sneppx_qlinear.h"

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: the ordinals of the reference's SNEPPXSafetensorsDType
 * (fs/format/safetensors.h:24-37), so codes pass between the two APIs */
typedef enum {
    SNEPPX_QST_F32 = 0,
    SNEPPX_QST_F16,
    SNEPPX_QST_F64,
    SNEPPX_QST_I64,
    SNEPPX_QST_I32,
    SNEPPX_QST_I16,
    SNEPPX_QST_I8,
    SNEPPX_QST_U8,
    SNEPPX_QST_BOOL,
    SNEPPX_QST_BF16,
    SNEPPX_QST_F8_E5M2,
    SNEPPX_QST_F8_E4M3FN
} SNEPPXQStoreDType;

#define SNEPPX_QST_MAX_DIMS 8

/* ---- reading ------------------------------------------------------------ */

typedef struct SNEPPXQStore SNEPPXQStore;

/* Open and index a safetensors file (read-only mapping). */
SNEPPXQStore* SNEPPX_qstore_open(const char* path);
void SNEPPX_qstore_close(SNEPPXQStore* st);

/* Number of tensors and the name of tensor i (valid until close). */
size_t SNEPPX_qstore_count(const SNEPPXQStore* st);
const char* SNEPPX_qstore_name(const SNEPPXQStore* st, size_t i);

/* dtype, shape (up to SNEPPX_QST_MAX_DIMS) and byte size of a tensor; -1 if
 * absent (no error text is set for a missing name). */
int SNEPPX_qstore_info(const SNEPPXQStore* st, const char* name, int* dtype, size_t* shape,
                       size_t* ndim, size_t* nbytes);

/* Host view of a tensor's bytes inside the mapping (NULL if absent). */
const void* SNEPPX_qstore_data(const SNEPPXQStore* st, const char* name, size_t* nbytes);

/* Copy a tensor to device memory: nbytes must equal its size.  Returns after
 * the copy has completed (the mapping is pageable host memory). */
int SNEPPX_qstore_read_device(const SNEPPXQStore* st, const char* name, void* d_dst,
                              size_t nbytes, SNEPPXStream stream);

/* Value of a string entry of __metadata__, or NULL. */
const char* SNEPPX_qstore_metadata(const SNEPPXQStore* st, const char* key);

/* ---- writing ------------------------------------------------------------ */

typedef struct SNEPPXQStoreWriter SNEPPXQStoreWriter;

SNEPPXQStoreWriter* SNEPPX_qstore_writer_open(const char* path);

/* Append a tensor from host memory (copied now) or from device memory
 * (copied to the host now; the call waits for `stream`). */
int SNEPPX_qstore_writer_add_host(SNEPPXQStoreWriter* w, const char* name, int dtype,
                                  const size_t* shape, size_t ndim, const void* data);
int SNEPPX_qstore_writer_add_device(SNEPPXQStoreWriter* w, const char* name, int dtype,
                                    const size_t* shape, size_t ndim, const void* d_data,
                                    SNEPPXStream stream);
int SNEPPX_qstore_writer_set_metadata(SNEPPXQStoreWriter* w, const char* key,
                                      const char* value);

/* Write the file and free the writer (also on error). */
int SNEPPX_qstore_writer_close(SNEPPXQStoreWriter* w);

/* ---- quantized layers ---------------------------------------------------- */

/* W4 layer <prefix>: device buffers in the sneppx_qlinear.h W4 layout.
 * qzeros may be NULL (symmetric), g_idx may be NULL (contiguous groups of
 * `group` columns; G = K / group). */
int SNEPPX_qstore_save_w4(SNEPPXQStoreWriter* w, const char* prefix, const uint32_t* d_qweight,
                          const uint16_t* d_scales, const uint32_t* d_qzeros,
                          const int32_t* d_g_idx, size_t N, size_t K, int group, size_t G,
                          SNEPPXStream stream);

/* Shape of a stored W4 layer: N, K, G, group (0 if stored with g_idx),
 * whether it has zero points and g_idx.  -1 if the tensors are absent or
 * inconsistent. */
int SNEPPX_qstore_query_w4(const SNEPPXQStore* st, const char* prefix, size_t* N, size_t* K,
                           size_t* G, int* group, int* has_zeros, int* has_g_idx);

/* Load into caller-allocated device buffers of the sizes query_w4 implies
 * (qzeros / g_idx ignored when NULL; -1 if the file has them and they are
 * NULL, or has not and they are given). */
int SNEPPX_qstore_load_w4(const SNEPPXQStore* st, const char* prefix, uint32_t* d_qweight,
                          uint16_t* d_scales, uint32_t* d_qzeros, int32_t* d_g_idx,
                          SNEPPXStream stream);

/* W8 layer <prefix>: codes int8 [N, K] and scales fp32 [N] (device). */
int SNEPPX_qstore_save_w8(SNEPPXQStoreWriter* w, const char* prefix, const int8_t* d_q,
                          const float* d_scales, size_t N, size_t K, SNEPPXStream stream);
int SNEPPX_qstore_query_w8(const SNEPPXQStore* st, const char* prefix, size_t* N, size_t* K);
int SNEPPX_qstore_load_w8(const SNEPPXQStore* st, const char* prefix, int8_t* d_q,
                          float* d_scales, SNEPPXStream stream);

/* ---- the model-zoo INT8 quantizer ---------------------------------------- */

/* algorithms/model_zoo/weights.c:225-252 (weight_tensor_quantize_int8), the
 * second INT8 rule of the reference: one multiplier m = 127 / max|x| for the
 * whole tensor (1 when the maximum is 0), codes (int8)clamp(x * m, -128, 127)
 * truncated toward zero (NaN gives 0, the x86 conversion's result).  The
 * reference drops m; here it is returned so codes can be dequantized as
 * q / m.  Host pointers, synchronous, like sneppx_quantization.h. */
int SNEPPX_quantize_int8_modelzoo(const float* input, int8_t* output, size_t n,
                                  float* multiplier_out);

/* Device form: in, q device pointers; *d_multiplier_out a device float. */
int SNEPPX_dev_quantize_int8_modelzoo(const float* in, int8_t* q, float* d_multiplier_out,
                                      size_t n, SNEPPXStream stream);

#ifdef __cplusplus
}
#endif

#endif /* SNEPPX_QSTORE_H */
