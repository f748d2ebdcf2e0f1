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

/* MFMA element format of an MX format: 0 e4m3, 1 e5m2, 2 e2m3, 3 e3m2, 4 e2m1 */
static int mfma_fmt(SNEPPXMXFormat f) {
    switch (f) {
        case SNEPPX_MXFP8_E4M3: return 0;
        case SNEPPX_MXFP8_E5M2: return 1;
        case SNEPPX_MXFP6_E2M3: return 2;
        case SNEPPX_MXFP6_E3M2: return 3;
        case SNEPPX_MXFP4_E2M1: return 4;
        default: return -1;
    }
}

int SNEPPX_mx_to_mfma(const uint8_t* packed, const int8_t* scales, uint8_t* out_packed,
                      int8_t* out_scales, size_t rows, size_t cols, SNEPPXMXFormat fmt,
                      unsigned int* rounded, SNEPPXStream stream) {
    REQUIRE(packed && scales && out_packed && out_scales, "mx_to_mfma: NULL pointer");
    REQUIRE(rows && cols, "mx_to_mfma: empty tensor");
    REQUIRE(mfma_fmt(fmt) >= 0, "mx_to_mfma: format %d has no block-32 matrix-core form", (int)fmt);
    REQUIRE(cols % 32 == 0, "mx_to_mfma: cols=%zu must be a multiple of the block (32)", cols);
    snx_clear_error();
    const size_t nblocks = rows * (cols / 32);
    if (fmt == SNEPPX_MXFP8_E4M3 || fmt == SNEPPX_MXFP8_E5M2) {
        REQUIRE(((uintptr_t)packed & 15u) == 0 && ((uintptr_t)out_packed & 15u) == 0,
                "mx_to_mfma: code buffers must be 16-byte aligned");
        return snx_k_mx_to_mfma(packed, scales, out_packed, out_scales, nblocks,
                                fmt == SNEPPX_MXFP8_E5M2, rounded, stream);
    }
    /* fp6 / fp4: the reference's codes are the matrix cores' own */
    int rc = snx_hip_memcpy_d2d(out_packed, packed, nblocks * 32 * (size_t)k_bits[fmt] / 8, stream);
    if (!rc) rc = snx_hip_memcpy_d2d(out_scales, scales, nblocks, stream);
    return rc;
}

static int mx_gemm_check(const char* who, const uint8_t* A, const int8_t* sA, const uint8_t* W,
                         const int8_t* sW, SNEPPXMXFormat fmt, void* out, SNEPPXDtype out_dtype,
                         size_t M, size_t N, size_t K) {
    REQUIRE(A && sA && W && sW && out, "%s: NULL pointer", who);
    REQUIRE(M && N && K, "%s: empty shape", who);
    REQUIRE(mfma_fmt(fmt) >= 0, "%s: format %d has no block-32 matrix-core form", who, (int)fmt);
    REQUIRE(out_dtype == SNEPPX_BFLOAT16 || out_dtype == SNEPPX_FLOAT32,
            "%s: out_dtype must be SNEPPX_BFLOAT16 or SNEPPX_FLOAT32", who);
    REQUIRE(((uintptr_t)A & 15u) == 0 && ((uintptr_t)W & 15u) == 0, "%s: A and W must be 16-byte aligned",
            who);
    if (fmt != SNEPPX_MXFP4_E2M1) {
        REQUIRE(K % 128 == 0, "%s: K=%zu must be a multiple of 128", who, K);
        REQUIRE(((uintptr_t)sA & 3u) == 0 && ((uintptr_t)sW & 3u) == 0,
                "%s: the exponent arrays must be 4-byte aligned", who);
    }
    return 0;
}

int SNEPPX_qlinear_mx_gemm_mfma(const uint8_t* A, const int8_t* sA, const uint8_t* W,
                                const int8_t* sW, SNEPPXMXFormat fmt, void* out,
                                SNEPPXDtype out_dtype, size_t M, size_t N, size_t K,
                                SNEPPXStream stream) {
    if (mx_gemm_check("qlinear_mx_gemm_mfma", A, sA, W, sW, fmt, out, out_dtype, M, N, K)) return -1;
    snx_clear_error();
    if (fmt == SNEPPX_MXFP4_E2M1)
        return SNEPPX_qlinear_mxfp4_gemm(A, sA, W, sW, out, out_dtype, M, N, K, stream);
    return snx_k_mx8_gemm(A, sA, W, sW, out, out_dtype == SNEPPX_FLOAT32, mfma_fmt(fmt), M, N, K,
                          stream);
}

int SNEPPX_qlinear_mx_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                           SNEPPXMXFormat fmt, void* out, SNEPPXDtype out_dtype, size_t M,
                           size_t N, size_t K, SNEPPXStream stream) {
    if (fmt == SNEPPX_NVFP4_E2M1)   /* per tensor by default (mx_formats.py:72-73) */
        return SNEPPX_qlinear_mx_gemm_bs(A, sA, W, sW, fmt, 0, out, out_dtype, M, N, K, stream);
    if (mx_gemm_check("qlinear_mx_gemm", A, sA, W, sW, fmt, out, out_dtype, M, N, K)) return -1;
    snx_clear_error();
    if (fmt != SNEPPX_MXFP8_E4M3 && fmt != SNEPPX_MXFP8_E5M2)
        return SNEPPX_qlinear_mx_gemm_mfma(A, sA, W, sW, fmt, out, out_dtype, M, N, K, stream);
    /* fp8: both operands through the conversion into the calling thread's workspace */
    const size_t ab = (M * K + 255) & ~(size_t)255, wb = (N * K + 255) & ~(size_t)255;
    const size_t asb = (M * (K / 32) + 255) & ~(size_t)255;
    uint8_t* ws = (uint8_t*)snx_workspace(ab + wb + asb + N * (K / 32), 0, stream);
    if (!ws) return -1;
    uint8_t* a2 = ws;
    uint8_t* w2 = ws + ab;
    int8_t* sa2 = (int8_t*)(ws + ab + wb);
    int8_t* sw2 = (int8_t*)(ws + ab + wb + asb);
    int rc = SNEPPX_mx_to_mfma(A, sA, a2, sa2, M, K, fmt, NULL, stream);
    if (!rc) rc = SNEPPX_mx_to_mfma(W, sW, w2, sw2, N, K, fmt, NULL, stream);
    if (!rc) rc = snx_k_mx8_gemm(a2, sa2, w2, sw2, out, out_dtype == SNEPPX_FLOAT32, mfma_fmt(fmt), M, N,
                                 K, stream);
    return rc;
}

/* Any block the reference's quantize_mx takes (mx_formats.py:147-150: the
 * format's own, an override, or per tensor) whose scales the matrix cores
 * can apply exactly: per tensor, or a multiple of 32 elements.  E2M1 per
 * tensor on the tiled kernel's shapes takes the two exponents as constant
 * scales; otherwise the exponents are rewritten into the block-32 form
 * (k_mx_expand_scales, into the calling thread's workspace) and the block-32
 * GEMM runs on the operands' own codes: NVFP4's and MXFP4's E2M1 codes are
 * the same, and with K a multiple of the block every row's codes start on a
 * byte. */
int SNEPPX_qlinear_mx_gemm_bs(const uint8_t* A, const int8_t* sA, const uint8_t* W,
                              const int8_t* sW, SNEPPXMXFormat fmt, int block_size, void* out,
                              SNEPPXDtype out_dtype, size_t M, size_t N, size_t K,
                              SNEPPXStream stream) {
    static const char* who = "qlinear_mx_gemm_bs";
    REQUIRE(valid_fmt(fmt), "%s: unknown format %d", who, (int)fmt);
    const int bs = block_of(fmt, block_size);
    REQUIRE(bs >= 0, "%s: block size %d must be a positive multiple of 8, 0 or -1", who, block_size);
    REQUIRE(bs == 0 || bs % 32 == 0,
            "%s: block %d: the matrix cores scale blocks of 32 elements, so a block must be per "
            "tensor or a multiple of 32", who, bs);
    REQUIRE(bs == 0 || K % (size_t)bs == 0, "%s: K=%zu must be a multiple of the block (%d)", who, K, bs);
    const SNEPPXMXFormat ef = fmt == SNEPPX_NVFP4_E2M1 ? SNEPPX_MXFP4_E2M1 : fmt;   /* element format */
    if (bs == 32) return SNEPPX_qlinear_mx_gemm(A, sA, W, sW, ef, out, out_dtype, M, N, K, stream);
    REQUIRE(A && sA && W && sW && out, "%s: NULL pointer", who);
    REQUIRE(M && N && K, "%s: empty shape", who);
    REQUIRE(K % 32 == 0, "%s: K=%zu must be a multiple of 32", who, K);
    if (bs == 0 && ef == SNEPPX_MXFP4_E2M1 && K % 256 == 0 && M >= 128 && N >= 128) {
        /* E2M1 with one exponent per operand (NVFP4): the tiled kernel splits
         * the two exponents itself and takes them as constant block scales */
        if (mx_gemm_check(who, A, sA, W, sW, ef, out, out_dtype, M, N, K)) return -1;
        snx_clear_error();
        return snx_k_mxfp4_gemm_tiled_pt(A, sA, W, sW, out, out_dtype == SNEPPX_FLOAT32, M, N, K, stream);
    }
    snx_clear_error();
    const size_t kb = K / 32, ab = (M * kb + 255) & ~(size_t)255;
    int8_t* ws = (int8_t*)snx_workspace(ab + N * kb, 1, stream);
    if (!ws) return -1;
    int8_t* sa32 = ws;
    int8_t* sw32 = ws + ab;
    const unsigned rep = (unsigned)(bs / 32);
    int rc = snx_k_mx_expand_scales(sA, sA, sW, sa32, M, kb, rep, 0, stream);
    if (!rc) rc = snx_k_mx_expand_scales(sW, sA, sW, sw32, N, kb, rep, 1, stream);
    if (!rc) rc = SNEPPX_qlinear_mx_gemm(A, sa32, W, sw32, ef, out, out_dtype, M, N, K, stream);
    return rc;
}
