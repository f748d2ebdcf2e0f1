/*
 * oracle_ext.c - CPU statement of the build-defined formats on the quantized
 * linear path (the reference has no W4 packed format, no GEMV/GEMM, no bf16).
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Each format reduces to reference primitives:
 *   - W4 AWQ-style (a20) is quantize_int8.c:98-123 (asymmetric, divide by the
 *     scale then add the zero point) with 255 -> 15, evaluated with the fp16
 *     scale that is stored, and packed in the nibble order of
 *     quantize_int8.c:206-216 generalised to 8 nibbles per little-endian u32.
 *   - GPTQ act-order (a21) is gptq.c:189-239 (bits 4, sym) applied to the
 *     columns of each g_idx group in ascending k; see orc_gptq_quantize.
 *   - Every linear is the fp32 dot of tensor.c:1820-1823 (k ascending).
 * Pins (tests/test_oracle_formats.py): brute-force dequantisation error
 * bounds, the a21 -> a13 reduction on permuted columns, int32 accumulators
 * against numpy int64 products, fp16/bf16 conversions against numpy's.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static int32_t round_to_i32(float v)
{
    float r = roundf(v);
    if (r >= -2147483648.0f && r < 2147483648.0f) return (int32_t)r;
    return INT32_MIN;
}

static int32_t clampi(int32_t v, int32_t lo, int32_t hi)
{
    return v < lo ? lo : (v > hi ? hi : v);
}

uint16_t orc_f32_to_bf16(float f)
{
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t orc_f32_to_f16(float f)
{
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u;           /* NaN */
    if (a >= 0x477FF000u) return sign | 0x7C00u;          /* >= 65520 -> Inf */
    if (a >= 0x38800000u) {                               /* normal binary16 */
        uint32_t h = ((a >> 23) - 112u) << 10 | ((a >> 13) & 0x3FFu);
        uint32_t rest = a & 0x1FFFu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
        return sign | (uint16_t)h;
    }
    if (a <= 0x33000000u) return sign;                    /* <= 2^-25 -> 0 */
    uint32_t full = (a & 0x7FFFFFu) | 0x800000u;          /* subnormal binary16 */
    uint32_t shift = 126u - (a >> 23);
    uint32_t h = full >> shift;
    uint32_t rest = full & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rest > half || (rest == half && (h & 1u))) h++;
    return sign | (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f;      /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t orc_w4_scale_to_f16(float s)
{
    uint16_t h = orc_f32_to_f16(s);
    if ((h & 0x7FFFu) == 0) return 0x0001u;               /* underflow -> 2^-24 */
    if ((h & 0x7FFFu) == 0x7C00u) return (uint16_t)((h & 0x8000u) | 0x7BFFu);
    return h;
}

static void put_nibble(uint32_t* words, size_t idx, uint32_t v)
{
    uint32_t sh = (uint32_t)(idx % 8) * 4u;
    words[idx / 8] = (words[idx / 8] & ~(0xFu << sh)) | ((v & 0xFu) << sh);
}

static uint32_t get_nibble(const uint32_t* words, size_t idx)
{
    return (words[idx / 8] >> ((idx % 8) * 4)) & 0xFu;
}

int orc_w4_awq_quantize(const float* w, size_t N, size_t K, int group,
                        uint32_t* qweight, uint16_t* scales, uint32_t* qzeros)
{
    if (!w || !qweight || !scales || !qzeros || N == 0 || K == 0 || group <= 0) return -1;
    size_t g = (size_t)group;
    if (K % 8 || K % g) return -1;
    size_t G = K / g, zw = (G + 7) / 8;
    memset(qweight, 0, N * (K / 8) * sizeof(uint32_t));
    memset(qzeros, 0, N * zw * sizeof(uint32_t));
    for (size_t n = 0; n < N; n++) {
        for (size_t j = 0; j < G; j++) {
            const float* x = w + n * K + j * g;
            float lo = x[0], hi = x[0];
            for (size_t i = 1; i < g; i++) {
                if (x[i] < lo) lo = x[i];
                if (x[i] > hi) hi = x[i];
            }
            uint16_t s16;
            int32_t z;
            if (hi - lo < FLT_MIN) {
                s16 = 0x3C00u;                            /* 1.0, zero 0, codes 0 */
                z = 0;
                for (size_t i = 0; i < g; i++) put_nibble(qweight + n * (K / 8), j * g + i, 0);
            } else {
                s16 = orc_w4_scale_to_f16((hi - lo) / 15.0f);
                float s = orc_f16_to_f32(s16);
                z = clampi(round_to_i32(-lo / s), 0, 15);
                for (size_t i = 0; i < g; i++) {
                    int32_t q = clampi(round_to_i32(x[i] / s + (float)z), 0, 15);
                    put_nibble(qweight + n * (K / 8), j * g + i, (uint32_t)q);
                }
            }
            scales[n * G + j] = s16;
            put_nibble(qzeros + n * zw, j, (uint32_t)z);
        }
    }
    return 0;
}

int orc_w4_gptq_quantize(const float* w, const int32_t* g_idx, size_t N, size_t K,
                         size_t G, uint32_t* qweight, uint16_t* scales)
{
    if (!w || !g_idx || !qweight || !scales || N == 0 || K == 0 || G == 0) return -1;
    if (K % 8) return -1;
    for (size_t k = 0; k < K; k++)
        if (g_idx[k] < 0 || (size_t)g_idx[k] >= G) return -1;
    float* gmax = (float*)malloc(G * sizeof(float));
    unsigned char* poisoned = (unsigned char*)malloc(G);
    if (!gmax || !poisoned) { free(gmax); free(poisoned); return -1; }
    memset(qweight, 0, N * (K / 8) * sizeof(uint32_t));
    for (size_t n = 0; n < N; n++) {
        const float* x = w + n * K;
        for (size_t j = 0; j < G; j++) gmax[j] = 0.0f;
        for (size_t k = 0; k < K; k++) {
            float a = fabsf(x[k]);
            if (a > gmax[g_idx[k]]) gmax[g_idx[k]] = a;
        }
        memset(poisoned, 0, G);
        for (size_t j = 0; j < G; j++) {
            float s = gmax[j] < FLT_MIN ? 1.0f : gmax[j] / 7.0f;
            scales[n * G + j] = orc_w4_scale_to_f16(s);
        }
        /* ascending k visits each group's columns in the order gptq.c
         * would see them after a stable argsort of g_idx */
        for (size_t k = 0; k < K; k++) {
            size_t j = (size_t)g_idx[k];
            int degenerate = gmax[j] < FLT_MIN;
            float s = degenerate ? 1.0f : gmax[j] / 7.0f;
            float v = poisoned[j] ? NAN : x[k];
            int32_t c = clampi(round_to_i32(v / s), -128, 127);
            put_nibble(qweight + n * (K / 8), k, (uint32_t)(clampi(c, -8, 7) + 8));
            if (!degenerate && !poisoned[j]) {
                float inv = 1.0f / s;
                float q = (float)clampi(round_to_i32(v * inv), -7, 7) * s;
                if (!isfinite(q - v)) poisoned[j] = 1;
            }
        }
    }
    free(gmax);
    free(poisoned);
    return 0;
}

int orc_w4_dequantize(const uint32_t* qweight, const uint16_t* scales,
                      const uint32_t* qzeros, const int32_t* g_idx,
                      size_t N, size_t K, int group, float* w_out)
{
    if (!qweight || !scales || !w_out || N == 0 || K == 0 || K % 8) return -1;
    if (!g_idx && (group <= 0 || K % (size_t)group)) return -1;
    size_t G;
    if (g_idx) {
        int32_t mx = -1;
        for (size_t k = 0; k < K; k++) {
            if (g_idx[k] < 0) return -1;
            if (g_idx[k] > mx) mx = g_idx[k];
        }
        G = (size_t)mx + 1;
    } else {
        G = K / (size_t)group;
    }
    size_t zw = (G + 7) / 8;
    for (size_t n = 0; n < N; n++)
        for (size_t k = 0; k < K; k++) {
            size_t j = g_idx ? (size_t)g_idx[k] : k / (size_t)group;
            int32_t q = (int32_t)get_nibble(qweight + n * (K / 8), k);
            int32_t z = qzeros ? (int32_t)get_nibble(qzeros + n * zw, j) : 8;
            w_out[n * K + k] = (float)(q - z) * orc_f16_to_f32(scales[n * G + j]);
        }
    return 0;
}

/* Row by row: dequantise row n (as orc_w4_dequantize), then the k-ascending
 * fp32 dot for every m.  Same bits as dequantising W whole and calling
 * orc_matmul_nk, without the N*K buffer. */
int orc_w4a16_linear(const uint16_t* x_bf16, const uint32_t* qweight,
                     const uint16_t* scales, const uint32_t* qzeros,
                     const int32_t* g_idx, size_t M, size_t N, size_t K,
                     int group, float* y)
{
    if (!x_bf16 || !y || M == 0) return -1;
    float* wd = (float*)malloc(K * sizeof(float));
    float* xf = (float*)malloc(M * K * sizeof(float));
    if (!wd || !xf) { free(wd); free(xf); return -1; }
    int rc = 0;
    for (size_t i = 0; i < M * K; i++) xf[i] = orc_bf16_to_f32(x_bf16[i]);
    size_t G = 0;
    if (g_idx) {
        for (size_t k = 0; k < K; k++)
            if ((size_t)g_idx[k] + 1 > G) G = (size_t)g_idx[k] + 1;
    }
    for (size_t n = 0; n < N && rc == 0; n++) {
        /* dequantise one row through the full-matrix routine's row layout */
        const uint32_t* qrow = qweight + n * (K / 8);
        const uint16_t* srow = scales + n * (g_idx ? G : K / (size_t)group);
        const uint32_t* zrow = NULL;
        if (qzeros) {
            size_t gg = g_idx ? G : K / (size_t)group;
            zrow = qzeros + n * ((gg + 7) / 8);
        }
        rc = orc_w4_dequantize(qrow, srow, zrow, g_idx, 1, K, group, wd);
        for (size_t m = 0; m < M && rc == 0; m++) {
            const float* xm = xf + m * K;
            float acc = 0.0f;
            for (size_t k = 0; k < K; k++) {
                float p = xm[k] * wd[k];
                acc = acc + p;
            }
            y[m * N + n] = acc;
        }
    }
    free(wd);
    free(xf);
    return rc;
}

/* quantization.py:453-454: `out = out + self.bias` on the fp32 product
 * (numpy broadcasts bias[n] over the rows). */
void orc_add_bias(float* y, const float* bias, size_t M, size_t N)
{
    for (size_t m = 0; m < M; m++)
        for (size_t n = 0; n < N; n++)
            y[m * N + n] = y[m * N + n] + bias[n];
}

int orc_w8_linear(const float* x, const int8_t* q, const float* s,
                  size_t M, size_t N, size_t K, float* y)
{
    if (!x || !q || !s || !y || M == 0 || N == 0 || K == 0) return -1;
    for (size_t m = 0; m < M; m++)
        for (size_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (size_t k = 0; k < K; k++) {
                float wv = (float)q[n * K + k] * s[n];
                float p = x[m * K + k] * wv;
                acc = acc + p;
            }
            y[m * N + n] = acc;
        }
    return 0;
}

void orc_i8_gemm_i32(const int8_t* A, const int8_t* W, int32_t* C,
                     size_t M, size_t N, size_t K)
{
    for (size_t m = 0; m < M; m++)
        for (size_t n = 0; n < N; n++) {
            int32_t acc = 0;
            for (size_t k = 0; k < K; k++)
                acc += (int32_t)A[m * K + k] * (int32_t)W[n * K + k];
            C[m * N + n] = acc;
        }
}

void orc_w8a8_epilogue(const int32_t* acc, const float* sA, const float* sW,
                       size_t M, size_t N, float* out)
{
    for (size_t m = 0; m < M; m++)
        for (size_t n = 0; n < N; n++)
            out[m * N + n] = (float)acc[m * N + n] * sA[m] * sW[n];
}

int orc_quantize_fp8_e4m3_scaled(const float* in, uint8_t* out, size_t n, float* scale_out)
{
    if (!in || !out || !scale_out || n == 0) return -1;
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = fabsf(in[i]);
        if (a > m) m = a;
    }
    float s = m < FLT_MIN ? 1.0f : m / 240.0f;
    *scale_out = s;
    for (size_t i = 0; i < n; i++) out[i] = orc_float_to_fp8_e4m3(in[i] / s);
    return 0;
}

void orc_fp8_gemm(const uint8_t* A, const uint8_t* W, float sA, float sW,
                  size_t M, size_t N, size_t K, float* out)
{
    float lut[256];
    for (int c = 0; c < 256; c++) lut[c] = orc_fp8_e4m3_to_float((uint8_t)c);
    for (size_t m = 0; m < M; m++)
        for (size_t n = 0; n < N; n++) {
            float acc = 0.0f;
            for (size_t k = 0; k < K; k++) {
                float p = lut[A[m * K + k]] * lut[W[n * K + k]];
                acc = acc + p;
            }
            out[m * N + n] = acc * sA * sW;
        }
}

/* Build-defined option (no reference counterpart): the per-row int8
 * quantizer of quantize_int8.c:157-177 with ties to even instead of roundf.
 * Scales are the reference's.  Pinned against numpy's rint (half-even) on the
 * same fp32 products x * (1/s). */
int orc_quantize_int8_channel_rne(const float* in, int8_t* out, size_t rows, size_t cols,
                                  float* scales_out)
{
    if (!in || !out || !scales_out || rows == 0 || cols == 0) return -1;
    for (size_t r = 0; r < rows; r++) {
        const float* x = in + r * cols;
        float m = 0.0f;
        for (size_t c = 0; c < cols; c++) {
            float a = fabsf(x[c]);
            if (a > m) m = a;
        }
        float s = (m < FLT_MIN) ? 1.0f : m / 127.0f;
        float inv = 1.0f / s;
        scales_out[r] = s;
        for (size_t c = 0; c < cols; c++) {
            float v = rintf(x[c] * inv);
            int32_t q = (v >= -2147483648.0f && v < 2147483648.0f) ? (int32_t)v : INT32_MIN;
            out[r * cols + c] = (int8_t)clampi(q, -128, 127);
        }
    }
    return 0;
}
