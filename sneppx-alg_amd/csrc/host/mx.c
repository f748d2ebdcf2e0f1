/*
 * mx.c - MX encode/decode entry points (include/sneppx_mx.h): argument
 * checks, block-size resolution (mx_formats.py:160-162: `block_size or
 * spec.block_size`, per tensor when that is <= 0), the per-tensor exponent
 * (checked on the host, where the reference raises) and the launches.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "sneppx_mx.h"
#include "snx_hip.h"
#include "../snx_internal.h"

static const int k_bits[6] = {8, 8, 6, 6, 4, 4};
static const int k_block[6] = {32, 32, 32, 32, 32, 0};
static const int k_row[6] = {0, 1, 2, 3, 4, 4};   /* element format of the kernels */

static int valid_fmt(SNEPPXMXFormat f) { return (int)f >= 0 && (int)f < 6; }

int SNEPPX_mx_bits(SNEPPXMXFormat fmt) { return valid_fmt(fmt) ? k_bits[fmt] : -1; }
int SNEPPX_mx_default_block(SNEPPXMXFormat fmt) { return valid_fmt(fmt) ? k_block[fmt] : -1; }

/* effective block size: > 0 blocked, 0 per tensor, -1 invalid */
static int block_of(SNEPPXMXFormat fmt, int block_size) {
    if (!valid_fmt(fmt)) return -1;
    const int bs = block_size ? block_size : k_block[fmt];
    if (bs <= 0) return 0;
    return bs % 8 == 0 ? bs : -1;
}

size_t SNEPPX_mx_packed_bytes(SNEPPXMXFormat fmt, size_t rows, size_t cols, int block_size) {
    const int bs = block_of(fmt, block_size);
    if (bs < 0) return 0;
    if (bs == 0) return (rows * cols * (size_t)k_bits[fmt] + 7) / 8;
    return rows * ((cols + (size_t)bs - 1) / (size_t)bs) * (size_t)bs * (size_t)k_bits[fmt] / 8;
}

size_t SNEPPX_mx_scale_count(SNEPPXMXFormat fmt, size_t rows, size_t cols, int block_size) {
    const int bs = block_of(fmt, block_size);
    if (bs < 0) return 0;
    return bs == 0 ? 1 : rows * ((cols + (size_t)bs - 1) / (size_t)bs);
}

#define REQUIRE(cond, ...)               \
    do {                                 \
        if (!(cond)) {                   \
            snx_set_error(__VA_ARGS__);  \
            return -1;                   \
        }                                \
    } while (0)

int SNEPPX_dev_quantize_mx(const float* x, uint8_t* packed, int8_t* scales, size_t rows,
                           size_t cols, SNEPPXMXFormat fmt, int block_size, SNEPPXStream stream) {
    REQUIRE(x && packed && scales, "dev_quantize_mx: NULL pointer");
    REQUIRE(valid_fmt(fmt), "dev_quantize_mx: unknown format %d", (int)fmt);
    REQUIRE(rows && cols, "dev_quantize_mx: empty tensor");
    const int bs = block_of(fmt, block_size);
    REQUIRE(bs >= 0, "dev_quantize_mx: block size %d must be a positive multiple of 8, 0 or -1",
            block_size);
    snx_clear_error();
    const int f = k_row[fmt];
    if (bs > 0) return snx_k_mx_quant_blocks(x, packed, scales, rows, cols, bs, f, stream);

    /* per tensor (mx_formats.py:164-173): peak = float(max|x|) (NaN -> 1.0
     * through a false `> 0`, an infinite peak raises), exponent in float64 */
    const size_t n = rows * cols;
    const int parts = snx_mx_tensor_parts(n);
    uint32_t* dpart = (uint32_t*)snx_workspace((size_t)parts * 2 * sizeof(uint32_t), 0, stream);
    if (!dpart) return -1;
    uint32_t* hpart = (uint32_t*)malloc((size_t)parts * 2 * sizeof(uint32_t));
    REQUIRE(hpart, "dev_quantize_mx: out of host memory");
    int rc = snx_k_mx_tensor_stats(x, n, dpart, parts, stream);
    if (!rc) rc = snx_hip_memcpy_d2h(hpart, dpart, (size_t)parts * 2 * sizeof(uint32_t), stream);
    if (!rc) rc = snx_hip_stream_sync(stream);
    if (rc) {
        free(hpart);
        return -1;
    }
    float peak = 0.0f;
    int nan = 0;
    for (int i = 0; i < parts; i++) {
        float m;
        memcpy(&m, &hpart[2 * i], 4);
        if (m > peak) peak = m;
        nan |= hpart[2 * i + 1] != 0;
    }
    free(hpart);
    if (nan || !(peak > 0.0f)) peak = 1.0f;
    REQUIRE(!isinf(peak), "dev_quantize_mx: infinite peak (the reference raises OverflowError)");
    uint32_t pb;
    memcpy(&pb, &peak, 4);
    const int s = snx_mx_scale_host(pb, f, 1);
    REQUIRE(s >= -128 && s <= 127,
            "dev_quantize_mx: per-tensor exponent %d outside int8 (the reference raises OverflowError)", s);
    const int8_t s8 = (int8_t)s;
    rc = snx_hip_memcpy_h2d(scales, &s8, 1, stream);
    if (!rc) rc = snx_k_mx_quant_tensor(x, packed, n, s, f, stream);
    if (!rc) rc = snx_hip_stream_sync(stream);   /* s8 lives on this stack frame */
    return rc;
}

int SNEPPX_dev_dequantize_mx(const uint8_t* packed, const int8_t* scales, float* y, size_t rows,
                             size_t cols, SNEPPXMXFormat fmt, int block_size, SNEPPXStream stream) {
    REQUIRE(packed && scales && y, "dev_dequantize_mx: NULL pointer");
    REQUIRE(valid_fmt(fmt), "dev_dequantize_mx: unknown format %d", (int)fmt);
    REQUIRE(rows && cols, "dev_dequantize_mx: empty tensor");
    const int bs = block_of(fmt, block_size);
    REQUIRE(bs >= 0, "dev_dequantize_mx: block size %d must be a positive multiple of 8, 0 or -1",
            block_size);
    snx_clear_error();
    const int f = k_row[fmt];
    if (bs > 0) return snx_k_mx_dequant_blocks(packed, scales, y, rows, cols, bs, f, stream);
    int8_t s8;
    if (snx_hip_memcpy_d2h(&s8, scales, 1, stream) || snx_hip_stream_sync(stream)) return -1;
    return snx_k_mx_dequant_tensor(packed, y, rows * cols, (int)s8, f, stream);
}

int SNEPPX_qlinear_mxfp4_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W,
                              const int8_t* sW, void* out, SNEPPXDtype out_dtype, size_t M,
                              size_t N, size_t K, SNEPPXStream stream) {
    REQUIRE(A && sA && W && sW && out, "qlinear_mxfp4_gemm: NULL pointer");
    REQUIRE(M && N && K, "qlinear_mxfp4_gemm: empty shape");
    REQUIRE(K % 64 == 0, "qlinear_mxfp4_gemm: K=%zu must be a multiple of 64", K);
    REQUIRE(out_dtype == SNEPPX_BFLOAT16 || out_dtype == SNEPPX_FLOAT32,
            "qlinear_mxfp4_gemm: out_dtype must be SNEPPX_BFLOAT16 or SNEPPX_FLOAT32");
    REQUIRE(((uintptr_t)A & 15u) == 0 && ((uintptr_t)W & 15u) == 0,
            "qlinear_mxfp4_gemm: A and W must be 16-byte aligned");
    snx_clear_error();
    if (K % 256 == 0 && M >= 128 && N >= 128 && ((uintptr_t)sA & 3u) == 0 && ((uintptr_t)sW & 3u) == 0)
        return snx_k_mxfp4_gemm_tiled(A, sA, W, sW, out, out_dtype == SNEPPX_FLOAT32, M, N, K, stream);
    return snx_k_mxfp4_gemm(A, sA, W, sW, out, out_dtype == SNEPPX_FLOAT32, M, N, K, stream);
}
