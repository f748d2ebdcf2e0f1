/*
 * quant_api.c - the reference's host-pointer quantization API
 * (include/sneppx_quantization.h) over the HIP kernels.
 *
 * Each numeric function keeps the reference's argument checks and return
 * codes, stages its inputs in device memory (one allocation per call), runs
 * the gfx950 kernels on the default stream, copies the outputs back and
 * returns when they are in host memory.  No arithmetic happens on the host:
 * a missing or failing device makes the call return -1.
 */
#include <float.h>
#include <stdlib.h>
#include <string.h>

#include "sneppx_quantization.h"
#include "sneppx_qlinear.h"
#include "sneppx_qstore.h"
#include "snx_hip.h"
#include "../snx_internal.h"

/* One device allocation carved into 256-byte aligned pieces. */
typedef struct {
    char* base;
    size_t size, used;
} arena;

static int arena_open(arena* a, size_t bytes) {
    a->base = NULL;
    a->used = 0;
    a->size = bytes;
    return snx_hip_malloc((void**)&a->base, bytes ? bytes : 1);
}

static void* arena_take(arena* a, size_t bytes) {
    size_t off = (a->used + 255) & ~(size_t)255;
    a->used = off + bytes;
    return a->base + off;
}

static size_t pad(size_t bytes) { return ((bytes + 255) & ~(size_t)255) + 256; }

static void arena_close(arena* a) {
    if (a->base) snx_hip_free(a->base);
    a->base = NULL;
}

#define TRY(expr)                 \
    do {                          \
        if ((expr) != 0) goto out; \
    } while (0)

/* absmax/minmax -> scale record for one flat vector already on the device */
static int scale_record(const float* dx, size_t n, int kind, float* dpart, float* drec) {
    int parts = snx_reduce_parts(n);
    if (kind == SNX_SCALE_ASYM255) {
        if (snx_k_minmax(dx, n, dpart, parts, NULL)) return -1;
    } else {
        if (snx_k_absmax(dx, n, dpart, parts, NULL)) return -1;
    }
    return snx_k_finalize_scale(dpart, parts, kind, dx, drec, NULL, NULL);
}

static size_t parts_bytes(size_t n) { return (size_t)snx_reduce_parts(n) * 2 * sizeof(float); }

/* quantize_int8.c:43-65 */
int SNEPPX_quantize_int8_sym(const float* input, int8_t* output, size_t n, float* scale_out) {
    if (!input || !output || !scale_out || n == 0) return -1;
    int rc = -1;
    float rec[SNX_SCALE_REC];
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(n) + pad(parts_bytes(n)) + pad(16))) return -1;
    float* dx = arena_take(&a, n * 4);
    int8_t* dq = arena_take(&a, n);
    float* dpart = arena_take(&a, parts_bytes(n));
    float* drec = arena_take(&a, 16);
    TRY(snx_hip_memcpy_h2d(dx, input, n * 4, NULL));
    TRY(scale_record(dx, n, SNX_SCALE_SYM127, dpart, drec));
    TRY(snx_k_quant_int8_sym(dx, dq, n, drec, NULL));
    TRY(snx_hip_memcpy_d2h(output, dq, n, NULL));
    TRY(snx_hip_memcpy_d2h(rec, drec, sizeof rec, NULL));
    TRY(snx_hip_stream_sync(NULL));
    *scale_out = rec[0];
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* quantize_int8.c:77-85 */
int SNEPPX_dequantize_int8_sym(const int8_t* input, float* output, size_t n, float scale) {
    if (!input || !output || n == 0) return -1;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n) + pad(n * 4))) return -1;
    int8_t* dq = arena_take(&a, n);
    float* dy = arena_take(&a, n * 4);
    TRY(snx_hip_memcpy_h2d(dq, input, n, NULL));
    TRY(snx_k_dequant_int8_sym(dq, dy, n, scale, NULL));
    TRY(snx_hip_memcpy_d2h(output, dy, n * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* quantize_int8.c:98-123 */
int SNEPPX_quantize_int8_asym(const float* input, int8_t* output, size_t n, float* scale_out,
                              int32_t* zp_out) {
    if (!input || !output || !scale_out || !zp_out || n == 0) return -1;
    int rc = -1;
    float rec[SNX_SCALE_REC];
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(n) + pad(parts_bytes(n)) + pad(16))) return -1;
    float* dx = arena_take(&a, n * 4);
    int8_t* dq = arena_take(&a, n);
    float* dpart = arena_take(&a, parts_bytes(n));
    float* drec = arena_take(&a, 16);
    TRY(snx_hip_memcpy_h2d(dx, input, n * 4, NULL));
    TRY(scale_record(dx, n, SNX_SCALE_ASYM255, dpart, drec));
    TRY(snx_k_quant_int8_asym(dx, dq, n, drec, NULL));
    TRY(snx_hip_memcpy_d2h(output, dq, n, NULL));
    TRY(snx_hip_memcpy_d2h(rec, drec, sizeof rec, NULL));
    TRY(snx_hip_stream_sync(NULL));
    *scale_out = rec[0];
    *zp_out = (int32_t)rec[2];
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* quantize_int8.c:136-144 */
int SNEPPX_dequantize_int8_asym(const int8_t* input, float* output, size_t n, float scale,
                                int32_t zp) {
    if (!input || !output || n == 0) return -1;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n) + pad(n * 4))) return -1;
    int8_t* dq = arena_take(&a, n);
    float* dy = arena_take(&a, n * 4);
    TRY(snx_hip_memcpy_h2d(dq, input, n, NULL));
    TRY(snx_k_dequant_int8_asym(dq, dy, n, scale, zp, NULL));
    TRY(snx_hip_memcpy_d2h(output, dy, n * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* quantize_int8.c:157-177 */
int SNEPPX_quantize_int8_channel(const float* input, int8_t* output, size_t rows, size_t cols,
                                 float* scales_out) {
    if (!input || !output || !scales_out || rows == 0 || cols == 0) return -1;
    size_t n = rows * cols;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(n) + pad(rows * 4))) return -1;
    float* dx = arena_take(&a, n * 4);
    int8_t* dq = arena_take(&a, n);
    float* ds = arena_take(&a, rows * 4);
    TRY(snx_hip_memcpy_h2d(dx, input, n * 4, NULL));
    TRY(snx_k_quant_int8_rows(dx, dq, ds, rows, cols, 0, NULL));
    TRY(snx_hip_memcpy_d2h(output, dq, n, NULL));
    TRY(snx_hip_memcpy_d2h(scales_out, ds, rows * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* quantize_int8.c:189-218 */
int SNEPPX_quantize_int4_sym(const float* input, uint8_t* output, size_t n, float* scale_out) {
    if (!input || !output || !scale_out || n == 0) return -1;
    size_t nb = (n + 1) / 2;
    int rc = -1;
    float rec[SNX_SCALE_REC];
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(nb) + pad(parts_bytes(n)) + pad(16))) return -1;
    float* dx = arena_take(&a, n * 4);
    uint8_t* dp = arena_take(&a, nb);
    float* dpart = arena_take(&a, parts_bytes(n));
    float* drec = arena_take(&a, 16);
    TRY(snx_hip_memcpy_h2d(dx, input, n * 4, NULL));
    TRY(scale_record(dx, n, SNX_SCALE_SYM7, dpart, drec));
    TRY(snx_k_quant_int4_sym(dx, dp, n, drec, NULL));
    TRY(snx_hip_memcpy_d2h(output, dp, nb, NULL));
    TRY(snx_hip_memcpy_d2h(rec, drec, sizeof rec, NULL));
    TRY(snx_hip_stream_sync(NULL));
    *scale_out = rec[0];
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* quantize_int8.c:230-247 */
int SNEPPX_dequantize_int4_sym(const uint8_t* input, float* output, size_t n, float scale) {
    if (!input || !output || n == 0) return -1;
    size_t nb = (n + 1) / 2;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(nb) + pad(n * 4))) return -1;
    uint8_t* dp = arena_take(&a, nb);
    float* dy = arena_take(&a, n * 4);
    TRY(snx_hip_memcpy_h2d(dp, input, nb, NULL));
    TRY(snx_k_dequant_int4_sym(dp, dy, n, scale, NULL));
    TRY(snx_hip_memcpy_d2h(output, dy, n * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

static int fp8_array(const float* in, uint8_t* out, size_t n, int fmt) {
    if (!in || !out) return -1;
    if (n == 0) return 0;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(n))) return -1;
    float* dx = arena_take(&a, n * 4);
    uint8_t* dc = arena_take(&a, n);
    TRY(snx_hip_memcpy_h2d(dx, in, n * 4, NULL));
    TRY(snx_k_fp8_encode(dx, dc, n, fmt, NULL, NULL));
    TRY(snx_hip_memcpy_d2h(out, dc, n, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

static int fp8_array_dec(const uint8_t* in, float* out, size_t n, int fmt) {
    if (!in || !out) return -1;
    if (n == 0) return 0;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n) + pad(n * 4))) return -1;
    uint8_t* dc = arena_take(&a, n);
    float* dy = arena_take(&a, n * 4);
    TRY(snx_hip_memcpy_h2d(dc, in, n, NULL));
    TRY(snx_k_fp8_decode(dc, dy, n, fmt, NULL));
    TRY(snx_hip_memcpy_d2h(out, dy, n * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* quantize_fp8.c:111-136, 212-237 (n == 0 succeeds, as in the reference) */
int SNEPPX_quantize_fp8_e4m3(const float* input, uint8_t* output, size_t n) {
    return fp8_array(input, output, n, 0);
}
int SNEPPX_dequantize_fp8_e4m3(const uint8_t* input, float* output, size_t n) {
    return fp8_array_dec(input, output, n, 0);
}
int SNEPPX_quantize_fp8_e5m2(const float* input, uint8_t* output, size_t n) {
    return fp8_array(input, output, n, 1);
}
int SNEPPX_dequantize_fp8_e5m2(const uint8_t* input, float* output, size_t n) {
    return fp8_array_dec(input, output, n, 1);
}

/* awq.c:106-120 (weights scaled in place, scale_out is rows x cols) */
int SNEPPX_awq_scale_weights(float* weights, size_t rows, size_t cols, const float* act_scales,
                             float* scale_out) {
    if (!weights || !act_scales || !scale_out || rows == 0 || cols == 0) return -1;
    size_t n = rows * cols;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n * 4) * 2 + pad(cols * 4))) return -1;
    float* dw = arena_take(&a, n * 4);
    float* ds = arena_take(&a, n * 4);
    float* dact = arena_take(&a, cols * 4);
    TRY(snx_hip_memcpy_h2d(dw, weights, n * 4, NULL));
    TRY(snx_hip_memcpy_h2d(dact, act_scales, cols * 4, NULL));
    TRY(snx_k_awq_scale_weights(dw, dact, ds, rows, cols, NULL));
    TRY(snx_hip_memcpy_d2h(weights, dw, n * 4, NULL));
    TRY(snx_hip_memcpy_d2h(scale_out, ds, n * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* awq.c:135-161 (act_scales is accepted and unused, as in the reference) */
int SNEPPX_awq_quantize(const float* weights, int8_t* qweight, const float* act_scales,
                        float* scales, size_t rows, size_t cols, int group_size) {
    (void)act_scales;
    if (!weights || !qweight || !scales || rows == 0 || cols == 0) return -1;
    size_t g = group_size <= 0 ? 128 : (size_t)group_size;
    size_t ng = (cols + g - 1) / g, n = rows * cols;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(n) + pad(rows * ng * 4))) return -1;
    float* dw = arena_take(&a, n * 4);
    int8_t* dq = arena_take(&a, n);
    float* ds = arena_take(&a, rows * ng * 4);
    TRY(snx_hip_memcpy_h2d(dw, weights, n * 4, NULL));
    TRY(snx_k_awq_quantize(dw, dq, ds, rows, cols, g, NULL));
    TRY(snx_hip_memcpy_d2h(qweight, dq, n, NULL));
    TRY(snx_hip_memcpy_d2h(scales, ds, rows * ng * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* gptq.c:189-239.  The weights are not modified (the reference quantizes a
 * copy of each group); codes are stored as int8 bytes only for bits <= 8. */
int SNEPPX_gptq_quantize(float* weights, size_t rows, size_t cols, int group_size, int bits,
                         SNEPPXDtype* qweight, float* scales, int32_t* zeros, int sym) {
    if (!weights || !qweight || !scales || rows == 0 || cols == 0) return -1;
    size_t g = group_size <= 0 ? 128 : (size_t)group_size;
    if (bits <= 0 || bits > 16) bits = 8;
    size_t ng = (cols + g - 1) / g, n = rows * cols;
    int store = bits <= 8;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(n) + pad(rows * ng * 4) * 2)) return -1;
    float* dw = arena_take(&a, n * 4);
    int8_t* dq = arena_take(&a, n);
    float* ds = arena_take(&a, rows * ng * 4);
    int32_t* dz = arena_take(&a, rows * ng * 4);
    TRY(snx_hip_memcpy_h2d(dw, weights, n * 4, NULL));
    TRY(snx_k_gptq_quantize(dw, store ? dq : NULL, ds, zeros ? dz : NULL, rows, cols, g, bits,
                            sym, NULL));
    if (store) TRY(snx_hip_memcpy_d2h(qweight, dq, n, NULL));
    TRY(snx_hip_memcpy_d2h(scales, ds, rows * ng * 4, NULL));
    if (zeros) TRY(snx_hip_memcpy_d2h(zeros, dz, rows * ng * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* gptq.c:55-79 */
int SNEPPX_gptq_compute_hessian(float* hessian, const float* activation, size_t n, size_t dim) {
    if (!hessian || !activation || n == 0 || dim == 0) return -1;
    int rc = -1;
    arena a;
    if (arena_open(&a, pad(dim * dim * 4) + pad(n * dim * 4))) return -1;
    float* dh = arena_take(&a, dim * dim * 4);
    float* dact = arena_take(&a, n * dim * 4);
    TRY(snx_hip_memcpy_h2d(dact, activation, n * dim * 4, NULL));
    TRY(snx_k_gptq_hessian(dh, dact, n, dim, NULL));
    TRY(snx_hip_memcpy_d2h(hessian, dh, dim * dim * 4, NULL));
    TRY(snx_hip_stream_sync(NULL));
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* gptq.c:134-172.  bits outside 1..30 make the reference's shifts undefined;
 * they are rejected here. */
int SNEPPX_gptq_quantize_block(float* w, float* h_inv, float* qw, float* scale, int32_t* zero,
                               size_t block_size, int bits, int sym) {
    if (!w || !h_inv || !qw || !scale) return -1;
    if (bits < 1 || bits > 30) {
        snx_set_error("gptq_quantize_block: bits=%d outside 1..30", bits);
        return -1;
    }
    if (block_size == 0) {              /* empty block: max 0 < FLT_MIN path */
        *scale = 1.0f;
        if (zero) *zero = 0;
        return 0;
    }
    size_t n = block_size;
    int rc = -1;
    float res[2];
    arena a;
    if (arena_open(&a, pad(n * 4) * 2 + pad(n * n * 4) + pad(8))) return -1;
    float* dw = arena_take(&a, n * 4);
    float* dqw = arena_take(&a, n * 4);
    float* dh = arena_take(&a, n * n * 4);
    float* dres = arena_take(&a, 8);
    TRY(snx_hip_memcpy_h2d(dw, w, n * 4, NULL));
    TRY(snx_hip_memcpy_h2d(dh, h_inv, n * n * 4, NULL));
    TRY(snx_k_gptq_block(dw, dh, dqw, dres, n, bits, sym, NULL));
    TRY(snx_hip_memcpy_d2h(w, dw, n * 4, NULL));
    TRY(snx_hip_memcpy_d2h(qw, dqw, n * 4, NULL));
    TRY(snx_hip_memcpy_d2h(res, dres, 8, NULL));
    TRY(snx_hip_stream_sync(NULL));
    *scale = res[0];
    if (zero) *zero = 0;
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

/* awq.c:171-201 */
int SNEPPX_quant_params_create(SNEPPXQuantParams* params, SNEPPXQuantMode mode) {
    if (!params) return -1;
    params->scale = 1.0f;
    params->zero_point = 0;
    params->scale_max = 0.0f;
    float lo = -127.0f, hi = 127.0f;
    if (mode == SNEPPX_QUANT_INT8_SYM) {
        lo = -128.0f;
        hi = 127.0f;
    } else if (mode == SNEPPX_QUANT_INT8_ASYM) {
        lo = 0.0f;
        hi = 255.0f;
    } else if (mode == SNEPPX_QUANT_INT4_SYM) {
        lo = -8.0f;
        hi = 7.0f;
    } else if (mode == SNEPPX_QUANT_FP8_E4M3 || mode == SNEPPX_QUANT_FP8_E5M2) {
        lo = -448.0f;
        hi = 448.0f;
    }
    params->qmin = lo;
    params->qmax = hi;
    return 0;
}

/* awq.c:210-223 */
const char* SNEPPX_quant_mode_name(SNEPPXQuantMode mode) {
    static const char* const names[] = {"none", "int8_sym", "int8_asym", "int4_sym",
                                        "fp8_e4m3", "fp8_e5m2", "awq", "gptq"};
    return ((int)mode >= 0 && (int)mode < 8) ? names[mode] : "unknown";
}

/* algorithms/model_zoo/weights.c:225-252 (weight_tensor_quantize_int8) */
int SNEPPX_quantize_int8_modelzoo(const float* input, int8_t* output, size_t n,
                                  float* multiplier_out) {
    if (!input || !output || !multiplier_out || n == 0) return -1;
    int rc = -1;
    float rec[SNX_SCALE_REC];
    arena a;
    if (arena_open(&a, pad(n * 4) + pad(n) + pad(parts_bytes(n)) + pad(16))) return -1;
    float* dx = arena_take(&a, n * 4);
    int8_t* dq = arena_take(&a, n);
    float* dpart = arena_take(&a, parts_bytes(n));
    float* drec = arena_take(&a, 16);
    TRY(snx_hip_memcpy_h2d(dx, input, n * 4, NULL));
    TRY(scale_record(dx, n, SNX_SCALE_MODELZOO, dpart, drec));
    TRY(snx_k_quant_int8_modelzoo(dx, dq, n, drec, NULL));
    TRY(snx_hip_memcpy_d2h(output, dq, n, NULL));
    TRY(snx_hip_memcpy_d2h(rec, drec, sizeof rec, NULL));
    TRY(snx_hip_stream_sync(NULL));
    *multiplier_out = rec[0];
    rc = 0;
out:
    arena_close(&a);
    return rc;
}

int SNEPPX_dev_quantize_int8_modelzoo(const float* in, int8_t* q, float* d_multiplier_out,
                                      size_t n, SNEPPXStream stream) {
    if (!in || !q || !d_multiplier_out) {
        snx_set_error("dev_quantize_int8_modelzoo: NULL pointer");
        return -1;
    }
    if (n == 0) {
        snx_set_error("dev_quantize_int8_modelzoo: empty tensor");
        return -1;
    }
    snx_clear_error();
    const int parts = snx_reduce_parts(n);
    /* partial maxima and the scale record in the stream's workspace */
    float* ws = (float*)snx_workspace(((size_t)parts * 2 + SNX_SCALE_REC) * sizeof(float), 0, stream);
    if (!ws) return -1;
    float* rec = ws + (size_t)parts * 2;
    if (snx_k_absmax(in, n, ws, parts, stream)) return -1;
    if (snx_k_finalize_scale(ws, parts, SNX_SCALE_MODELZOO, in, rec, d_multiplier_out, stream))
        return -1;
    return snx_k_quant_int8_modelzoo(in, q, n, rec, stream);
}
