/*
 * oracle_quant.c - CPU restatement of the reference kernel/quantization sources.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Written from the reference's
 * behaviour; every function cites the lines it follows.  Integer results
 * must be bit-identical to the reference; the float outputs of the
 * scale-search and Hessian functions are bit-identical under the pinned
 * flags -O2 -ffp-contract=off.
 *
 * Parity pins (tests/test_oracle_golden.py, tests/test_oracle_ref.py):
 *   - golden fixtures produced by oracle/_ref (the reference sources
 *     compiled unchanged), stored as tests/golden/ npz fixtures;
 *   - known answers: int8 {127,.5,2.5,-2.5} -> 127 1 3 -3; int4
 *     {7,-7,3.5,-3.5,1,0} -> 97 C4 01; e4m3/e5m2 code tables;
 *     fake-quant 1.4->1, -0.6->-1, +-200 clamp (tests/unit/test_fake_quant.c:28-31);
 *   - exhaustive fp8 decode (all 256 codes) and a stratified encode sweep.
 */
#include "oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* (int)roundf(v) as the reference's x86-64 build evaluates it: cvttss2si
 * yields INT32_MIN for NaN and for results outside the int range. */
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

static float absmax(const float* x, size_t n)
{
    float m = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > m) m = a;            /* NaN never wins the comparison */
    }
    return m;
}

/* quantize_int8.c:43-65 */
int orc_quantize_int8_sym(const float* in, int8_t* out, size_t n, float* scale_out)
{
    if (!in || !out || !scale_out || n == 0) return -1;
    float m = absmax(in, n);
    if (m < FLT_MIN) {
        *scale_out = 1.0f;
        memset(out, 0, n);
        return 0;
    }
    float s = m / 127.0f;
    float inv = 1.0f / s;
    *scale_out = s;
    for (size_t i = 0; i < n; i++)
        out[i] = (int8_t)clampi(round_to_i32(in[i] * inv), -128, 127);
    return 0;
}

/* quantize_int8.c:77-85 */
int orc_dequantize_int8_sym(const int8_t* in, float* out, size_t n, float scale)
{
    if (!in || !out || n == 0) return -1;
    for (size_t i = 0; i < n; i++) out[i] = (float)in[i] * scale;
    return 0;
}

/* quantize_int8.c:98-123.  Division by the scale, then + zp in fp32; codes
 * 128..255 are stored through int8_t (two's-complement wrap). */
int orc_quantize_int8_asym(const float* in, int8_t* out, size_t n,
                           float* scale_out, int32_t* zp_out)
{
    if (!in || !out || !scale_out || !zp_out || n == 0) return -1;
    float lo = in[0], hi = in[0];
    for (size_t i = 1; i < n; i++) {
        if (in[i] < lo) lo = in[i];
        if (in[i] > hi) hi = in[i];
    }
    if (hi - lo < FLT_MIN) {
        *scale_out = 1.0f;
        *zp_out = 0;
        memset(out, 0, n);
        return 0;
    }
    float s = (hi - lo) / 255.0f;
    int32_t zp = clampi(round_to_i32(-lo / s), 0, 255);
    *scale_out = s;
    *zp_out = zp;
    for (size_t i = 0; i < n; i++) {
        int32_t q = clampi(round_to_i32(in[i] / s + (float)zp), 0, 255);
        out[i] = (int8_t)(uint8_t)q;
    }
    return 0;
}

/* quantize_int8.c:136-144 */
int orc_dequantize_int8_asym(const int8_t* in, float* out, size_t n,
                             float scale, int32_t zp)
{
    if (!in || !out || n == 0) return -1;
    for (size_t i = 0; i < n; i++)
        out[i] = ((float)(uint8_t)in[i] - (float)zp) * scale;
    return 0;
}

/* quantize_int8.c:157-177 */
int orc_quantize_int8_channel(const float* in, int8_t* out, size_t rows,
                              size_t cols, float* scales_out)
{
    if (!in || !out || !scales_out || rows == 0 || cols == 0) return -1;
    for (size_t r = 0; r < rows; r++) {
        const float* x = in + r * cols;
        float m = absmax(x, cols);
        float s = (m < FLT_MIN) ? 1.0f : m / 127.0f;
        float inv = 1.0f / s;
        scales_out[r] = s;
        for (size_t c = 0; c < cols; c++)
            out[r * cols + c] = (int8_t)clampi(round_to_i32(x[c] * inv), -128, 127);
    }
    return 0;
}

/* quantize_int8.c:189-218.  Element 2i -> low nibble, 2i+1 -> high nibble. */
int orc_quantize_int4_sym(const float* in, uint8_t* out, size_t n, float* scale_out)
{
    if (!in || !out || !scale_out || n == 0) return -1;
    float m = absmax(in, n);
    if (m < FLT_MIN) {
        *scale_out = 1.0f;
        memset(out, 0, (n + 1) / 2);
        return 0;
    }
    float s = m / 7.0f;
    float inv = 1.0f / s;
    *scale_out = s;
    for (size_t i = 0; i < n; i += 2) {
        uint8_t b = (uint8_t)(clampi(round_to_i32(in[i] * inv), -8, 7) & 0xF);
        if (i + 1 < n)
            b |= (uint8_t)((clampi(round_to_i32(in[i + 1] * inv), -8, 7) & 0xF) << 4);
        out[i / 2] = b;
    }
    return 0;
}

/* quantize_int8.c:230-247 */
int orc_dequantize_int4_sym(const uint8_t* in, float* out, size_t n, float scale)
{
    if (!in || !out || n == 0) return -1;
    for (size_t i = 0; i < n; i++) {
        int v = (in[i / 2] >> ((i & 1) * 4)) & 0xF;
        if (v >= 8) v -= 16;
        out[i] = (float)v * scale;
    }
    return 0;
}

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* quantize_fp8.c:41-69.  Mantissa truncated to 3 bits; |x| < 2^-6 -> +-0;
 * exponent above 8, Inf and NaN -> sign|0x78; exponent 8 lands in field 15. */
uint8_t orc_float_to_fp8_e4m3(float v)
{
    uint32_t u = f2u(v);
    uint8_t sign = (uint8_t)((u >> 31) << 7);
    uint32_t ef = (u >> 23) & 0xFFu;
    if (ef == 0xFFu) return sign | 0x78;
    if (ef == 0) return sign;
    int e = (int)ef - 127;
    if (e < -6) return sign;
    if (e > 8) return sign | 0x78;
    return (uint8_t)(sign | ((uint32_t)(e + 7) << 3) | ((u >> 20) & 7u));
}

/* quantize_fp8.c:78-100.  Field 15 -> +-inf (mantissa 0) or +NaN; codes 0x00
 * and 0x80 -> +0.0; every other field-0 code decodes as a normal 2^-7*(1+m/8). */
float orc_fp8_e4m3_to_float(uint8_t c)
{
    uint32_t sign = (uint32_t)(c >> 7);
    uint32_t ef = (c >> 3) & 0xFu, m = c & 7u;
    if (ef == 0xFu) return m ? NAN : (sign ? -INFINITY : INFINITY);
    if (ef == 0 && m == 0) return 0.0f;
    return u2f((sign << 31) | ((ef - 7u + 127u) << 23) | (m << 20));
}

/* quantize_fp8.c:111-136 (n == 0 is accepted) */
int orc_quantize_fp8_e4m3(const float* in, uint8_t* out, size_t n)
{
    if (!in || !out) return -1;
    for (size_t i = 0; i < n; i++) out[i] = orc_float_to_fp8_e4m3(in[i]);
    return 0;
}

int orc_dequantize_fp8_e4m3(const uint8_t* in, float* out, size_t n)
{
    if (!in || !out) return -1;
    for (size_t i = 0; i < n; i++) out[i] = orc_fp8_e4m3_to_float(in[i]);
    return 0;
}

/* quantize_fp8.c:146-172.  Keeps only mantissa bit 22, placed in code bit 0. */
uint8_t orc_float_to_fp8_e5m2(float v)
{
    uint32_t u = f2u(v);
    uint8_t sign = (uint8_t)((u >> 31) << 7);
    uint32_t ef = (u >> 23) & 0xFFu;
    if (ef == 0xFFu) return sign | 0x7C;
    if (ef == 0) return sign;
    int e = (int)ef - 127;
    if (e < -14) return sign;
    if (e > 15) return sign | 0x7C;
    return (uint8_t)(sign | ((uint32_t)(e + 15) << 2) | ((u >> 22) & 1u));
}

/* quantize_fp8.c:181-201 */
float orc_fp8_e5m2_to_float(uint8_t c)
{
    uint32_t sign = (uint32_t)(c >> 7);
    uint32_t ef = (c >> 2) & 0x1Fu, m = c & 3u;
    if (ef == 0x1Fu) return m ? NAN : (sign ? -INFINITY : INFINITY);
    if (ef == 0 && m == 0) return 0.0f;
    return u2f((sign << 31) | ((ef - 15u + 127u) << 23) | (m << 21));
}

int orc_quantize_fp8_e5m2(const float* in, uint8_t* out, size_t n)
{
    if (!in || !out) return -1;
    for (size_t i = 0; i < n; i++) out[i] = orc_float_to_fp8_e5m2(in[i]);
    return 0;
}

int orc_dequantize_fp8_e5m2(const uint8_t* in, float* out, size_t n)
{
    if (!in || !out) return -1;
    for (size_t i = 0; i < n; i++) out[i] = orc_fp8_e5m2_to_float(in[i]);
    return 0;
}

/* awq.c:48-91: grid search of s over [alpha, 1] for column `col` of `row`.
 * The candidate loop accumulates s in fp32; the first strictly smallest
 * loss wins; the group max is only used for the all-zero early exit. */
static float awq_best_scale(const float* row, size_t col, size_t cols,
                            const float* act_scale)
{
    const size_t g = 128;
    size_t lo = (col / g) * g;
    size_t hi = lo + g < cols ? lo + g : cols;
    if (absmax(row + lo, hi - lo) < FLT_MIN) return 1.0f;
    float alpha = act_scale ? (act_scale[col] < 1.0f ? act_scale[col] : 1.0f) : 0.5f;
    float step = (1.0f - alpha) / 20.0f;
    if (step < 0.001f) step = 0.001f;
    float best_s = 1.0f, best_loss = 1e20f;
    for (float s = alpha; s <= 1.0f; s += step) {
        float inv_s = 1.0f / s;
        float mq = 0.0f;
        for (size_t j = lo; j < hi; j++) {
            float a = fabsf(row[j] * s);
            if (a > mq) mq = a;
        }
        float qs = (mq < FLT_MIN) ? 1.0f : mq / 127.0f;
        float loss = 0.0f;
        for (size_t j = lo; j < hi; j++) {
            int32_t q = clampi(round_to_i32(row[j] * s / qs), -128, 127);
            float d = (float)q * qs * inv_s - row[j];
            float sq = d * d;
            loss = loss + sq;
        }
        loss = loss / (float)(hi - lo);
        if (loss < best_loss) {
            best_loss = loss;
            best_s = s;
        }
    }
    return best_s;
}

/* awq.c:111-120: columns in order; each scaled column feeds later searches */
int orc_awq_scale_weights(float* weights, size_t rows, size_t cols,
                          const float* act_scales, float* scale_out)
{
    if (!weights || !act_scales || !scale_out || rows == 0 || cols == 0) return -1;
    for (size_t r = 0; r < rows; r++) {
        float* row = weights + r * cols;
        for (size_t c = 0; c < cols; c++) {
            float s = awq_best_scale(row, c, cols, act_scales);
            scale_out[r * cols + c] = s;
            row[c] *= s;
        }
    }
    return 0;
}

/* awq.c:135-161: per-(row, group) symmetric int8; act_scales is unused. */
int orc_awq_quantize(const float* weights, int8_t* qweight, const float* act_scales,
                     float* scales, size_t rows, size_t cols, int group_size)
{
    (void)act_scales;
    if (!weights || !qweight || !scales || rows == 0 || cols == 0) return -1;
    size_t g = group_size <= 0 ? 128 : (size_t)group_size;
    size_t ng = (cols + g - 1) / g;
    for (size_t r = 0; r < rows; r++) {
        for (size_t j = 0; j < ng; j++) {
            size_t lo = j * g, hi = lo + g < cols ? lo + g : cols;
            const float* x = weights + r * cols;
            float m = absmax(x + lo, hi - lo);
            float s = (m < FLT_MIN) ? 1.0f : m / 127.0f;
            float inv = 1.0f / s;
            scales[r * ng + j] = s;
            for (size_t c = lo; c < hi; c++)
                qweight[r * cols + c] = (int8_t)clampi(round_to_i32(x[c] * inv), -128, 127);
        }
    }
    return 0;
}

/* gptq.c:55-79: upper triangle accumulated sample by sample, mirrored, then
 * reg = 1e-5*H[0][0] (or 1e-5 when that is below 1e-8) on the diagonal. */
int orc_gptq_compute_hessian(float* h, const float* act, size_t n, size_t dim)
{
    if (!h || !act || n == 0 || dim == 0) return -1;
    memset(h, 0, dim * dim * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        const float* a = act + i * dim;
        for (size_t r = 0; r < dim; r++)
            for (size_t c = r; c < dim; c++) {
                float p = a[r] * a[c];
                h[r * dim + c] = h[r * dim + c] + p;
            }
    }
    for (size_t r = 1; r < dim; r++)
        for (size_t c = 0; c < r; c++) h[r * dim + c] = h[c * dim + r];
    float reg = 1e-5f * h[0];
    if (reg < 1e-8f) reg = 1e-5f;
    for (size_t i = 0; i < dim; i++) h[i * dim + i] += reg;
    return 0;
}

/* gptq.c:81-118: Cholesky factor L, then the in-place lower-triangular
 * "inverse" exactly as the reference evaluates it (row-major, in place). */
int orc_cholesky_inv(float* h, size_t dim)
{
    float* L = (float*)calloc(dim * dim, sizeof(float));
    if (!L) return -1;
    for (size_t j = 0; j < dim; j++) {
        float acc = 0.0f;
        for (size_t k = 0; k < j; k++) {
            float p = L[j * dim + k] * L[j * dim + k];
            acc = acc + p;
        }
        float d = h[j * dim + j] - acc;
        if (d < 1e-10f) { free(L); return -1; }
        L[j * dim + j] = sqrtf(d);
        for (size_t i = j + 1; i < dim; i++) {
            float t = 0.0f;
            for (size_t k = 0; k < j; k++) {
                float p = L[i * dim + k] * L[j * dim + k];
                t = t + p;
            }
            L[i * dim + j] = (h[i * dim + j] - t) / L[j * dim + j];
        }
    }
    for (size_t i = 0; i < dim; i++) {
        for (size_t j = 0; j < dim; j++) {
            float v;
            if (j > i) {
                v = 0.0f;
            } else if (j == i) {
                v = 1.0f / L[i * dim + i];
            } else {
                float t = 0.0f;
                for (size_t k = j; k < dim; k++) {
                    float p = L[i * dim + k] * h[k * dim + j];
                    t = t + p;
                }
                v = -t / L[i * dim + i];
            }
            h[i * dim + j] = v;
        }
    }
    free(L);
    return 0;
}

/* gptq.c:134-172: scale = max|w|/qmax, sequential quantize with error
 * feedback w[k] += (-err / h_inv[j][j]) * h_inv[k][j] for k > j. */
int orc_gptq_quantize_block(float* w, float* h_inv, float* qw, float* scale,
                            int32_t* zero, size_t block_size, int bits, int sym)
{
    if (!w || !h_inv || !qw || !scale) return -1;
    int qmax = (1 << (bits - 1)) - 1, qmin = -qmax;
    if (!sym) { qmax = (1 << bits) - 1; qmin = 0; }
    size_t n = block_size;
    float m = absmax(w, n);
    if (m < FLT_MIN) {
        *scale = 1.0f;
        if (zero) *zero = 0;
        memset(qw, 0, n * sizeof(float));
        return 0;
    }
    *scale = m / (float)qmax;
    if (zero) *zero = 0;
    float inv = 1.0f / *scale;
    for (size_t j = 0; j < n; j++) {
        float q = (float)clampi(round_to_i32(w[j] * inv), qmin, qmax) * *scale;
        float err = q - w[j];
        qw[j] = q;
        float hd = h_inv[j * n + j];
        if (fabsf(hd) > 1e-10f) {
            float coef = -err / hd;
            for (size_t k = j + 1; k < n; k++) {
                float p = coef * h_inv[k * n + j];
                w[k] = w[k] + p;
            }
        }
    }
    return 0;
}

/* gptq.c:189-239, literally: per group build I, invert it, run the block. */
int orc_gptq_quantize_literal(float* weights, size_t rows, size_t cols,
                              int group_size, int bits, void* qweight,
                              float* scales, int32_t* zeros, int sym)
{
    if (!weights || !qweight || !scales || rows == 0 || cols == 0) return -1;
    size_t g = group_size <= 0 ? 128 : (size_t)group_size;
    if (bits <= 0 || bits > 16) bits = 8;
    size_t ng = (cols + g - 1) / g;
    for (size_t r = 0; r < rows; r++) {
        for (size_t j = 0; j < ng; j++) {
            size_t lo = j * g, hi = lo + g < cols ? lo + g : cols, gs = hi - lo;
            float* blk = (float*)malloc(gs * sizeof(float));
            float* hinv = (float*)calloc(gs * gs, sizeof(float));
            float* qb = (float*)malloc(gs * sizeof(float));
            if (!blk || !hinv || !qb) { free(blk); free(hinv); free(qb); return -1; }
            memcpy(blk, weights + r * cols + lo, gs * sizeof(float));
            for (size_t i = 0; i < gs; i++) hinv[i * gs + i] = 1.0f;
            if (orc_cholesky_inv(hinv, gs) != 0) {
                memset(hinv, 0, gs * gs * sizeof(float));
                for (size_t i = 0; i < gs; i++) hinv[i * gs + i] = 1.0f;
            }
            float s;
            int32_t z = 0;
            orc_gptq_quantize_block(blk, hinv, qb, &s, &z, gs, bits, sym);
            scales[r * ng + j] = s;
            if (zeros) zeros[r * ng + j] = z;
            if (bits <= 8)
                for (size_t c = 0; c < gs; c++)
                    ((int8_t*)qweight)[r * cols + lo + c] =
                        (int8_t)clampi(round_to_i32(blk[c] / s), -128, 127);
            free(blk); free(hinv); free(qb);
        }
    }
    return 0;
}

/* gptq.c:189-239 in closed form.  With h_inv = cholesky_inv(I) the diagonal
 * is 1 and every entry below it is -0.0f, so the feedback term
 * coef * h_inv[k][j] is a signed zero while coef is finite (codes unchanged:
 * only the sign of a zero weight can flip) and NaN once coef is +-Inf or
 * NaN.  Hence: code[j] = clamp(roundf(w[j] / scale)) until the first column
 * whose error q - w is not finite; every later column of that group reads
 * NaN, i.e. code -128.  scale = max|w|/qmax (1 if max < FLT_MIN, no
 * feedback then); zeros are always 0; bits > 8 stores no codes. */
int orc_gptq_quantize(float* weights, size_t rows, size_t cols, int group_size,
                      int bits, void* qweight, float* scales, int32_t* zeros, int sym)
{
    if (!weights || !qweight || !scales || rows == 0 || cols == 0) return -1;
    size_t g = group_size <= 0 ? 128 : (size_t)group_size;
    if (bits <= 0 || bits > 16) bits = 8;
    int qmax = (1 << (bits - 1)) - 1, qmin = -qmax;
    if (!sym) { qmax = (1 << bits) - 1; qmin = 0; }
    size_t ng = (cols + g - 1) / g;
    int8_t* q8 = (int8_t*)qweight;
    for (size_t r = 0; r < rows; r++) {
        const float* x = weights + r * cols;
        for (size_t j = 0; j < ng; j++) {
            size_t lo = j * g, hi = lo + g < cols ? lo + g : cols;
            float m = absmax(x + lo, hi - lo);
            int degenerate = m < FLT_MIN;
            float s = degenerate ? 1.0f : m / (float)qmax;
            float inv = 1.0f / s;
            scales[r * ng + j] = s;
            if (zeros) zeros[r * ng + j] = 0;
            int poisoned = 0;
            for (size_t c = lo; c < hi; c++) {
                float v = poisoned ? NAN : x[c];
                if (bits <= 8)
                    q8[r * cols + c] = (int8_t)clampi(round_to_i32(v / s), -128, 127);
                if (!degenerate && !poisoned) {
                    float q = (float)clampi(round_to_i32(v * inv), qmin, qmax) * s;
                    float err = q - v;
                    if (!isfinite(err)) poisoned = 1;
                }
            }
        }
    }
    return 0;
}

/* awq.c:171-201 */
int orc_quant_params_create(orc_quant_params* p, int mode)
{
    if (!p) return -1;
    p->scale = 1.0f;
    p->zero_point = 0;
    p->scale_max = 0.0f;
    switch (mode) {
    case ORC_QUANT_INT8_SYM:  p->qmin = -128.0f; p->qmax = 127.0f; break;
    case ORC_QUANT_INT8_ASYM: p->qmin = 0.0f;    p->qmax = 255.0f; break;
    case ORC_QUANT_INT4_SYM:  p->qmin = -8.0f;   p->qmax = 7.0f;   break;
    case ORC_QUANT_FP8_E4M3:
    case ORC_QUANT_FP8_E5M2:  p->qmin = -448.0f; p->qmax = 448.0f; break;
    default:                  p->qmin = -127.0f; p->qmax = 127.0f; break;
    }
    return 0;
}

/* awq.c:210-223 */
const char* orc_quant_mode_name(int mode)
{
    static const char* const names[] = { "none", "int8_sym", "int8_asym", "int4_sym",
                                         "fp8_e4m3", "fp8_e5m2", "awq", "gptq" };
    if (mode < 0 || mode > 7) return "unknown";
    return names[mode];
}

/* tensor.c:2180-2195: floorf(x*inv + 0.5f) (ties toward +inf), clamped to
 * [-2^(b-1), 2^(b-1)-1], times scale. */
int orc_fake_quant(const float* in, float* out, size_t n, float scale, int bits)
{
    if (!in || !out || !(scale > 0.0f) || bits < 2 || bits > 16) return -1;
    float lo = (float)(-(1 << (bits - 1))), hi = (float)((1 << (bits - 1)) - 1);
    float inv = 1.0f / scale;
    for (size_t i = 0; i < n; i++) {
        float t = in[i] * inv;
        float q = floorf(t + 0.5f);
        if (q < lo) q = lo;
        if (q > hi) q = hi;
        out[i] = q * scale;
    }
    return 0;
}

/* algorithms/model_zoo/weights.c:225-252 (weight_tensor_quantize_int8): one
 * multiplier for the tensor, codes by truncation toward zero.  The
 * reference's (int8_t) cast of NaN is undefined in C; on x86-64 gcc emits
 * cvttss2si, whose NaN result 0x80000000 narrows to 0, which is what this
 * states explicitly. */
int orc_quantize_int8_modelzoo(const float* in, int8_t* out, size_t n, float* mult_out)
{
    if (!in || !out || !mult_out || n == 0) return -1;
    float max_val = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float v = fabsf(in[i]);
        if (v > max_val) max_val = v;
    }
    float scale = max_val > 0 ? 127.0f / max_val : 1.0f;
    for (size_t i = 0; i < n; i++) {
        float v = in[i] * scale;
        if (v > 127) v = 127;
        else if (v < -128) v = -128;
        out[i] = v != v ? 0 : (int8_t)v;
    }
    *mult_out = scale;
    return 0;
}

/* tensor.c:1820-1823 (i, j outer; l inner, sequential fp32 from 0.0f) */
void orc_matmul_kn(const float* a, const float* b, float* y, size_t M, size_t K, size_t N)
{
    for (size_t i = 0; i < M; i++)
        for (size_t j = 0; j < N; j++) {
            float acc = 0.0f;
            for (size_t l = 0; l < K; l++) {
                float p = a[i * K + l] * b[l * N + j];
                acc = acc + p;
            }
            y[i * N + j] = acc;
        }
}

void orc_matmul_nk(const float* a, const float* w, float* y, size_t M, size_t K, size_t N)
{
    for (size_t i = 0; i < M; i++)
        for (size_t j = 0; j < N; j++) {
            const float* x = a + i * K;
            const float* r = w + j * K;
            float acc = 0.0f;
            for (size_t l = 0; l < K; l++) {
                float p = x[l] * r[l];
                acc = acc + p;
            }
            y[i * N + j] = acc;
        }
}
