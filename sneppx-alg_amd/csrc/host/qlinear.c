/*
 * qlinear.c - device-pointer entry points (include/sneppx_qlinear.h):
 * argument checks, shape dispatch and workspace, then the HIP launchers.
 * Nothing here touches tensor data; every call is asynchronous on `stream`.
 */
#include <stdint.h>
#include <stdlib.h>

#include "sneppx_qlinear.h"
#include "snx_hip.h"
#include "../snx_internal.h"

/* rows from which W4A16 runs the MFMA GEMM instead of 64-row GEMV slices */
#define SNX_W4_GEMM_MIN_M 256

static int aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

#define REQUIRE(cond, ...)               \
    do {                                 \
        if (!(cond)) {                   \
            snx_set_error(__VA_ARGS__);  \
            return -1;                   \
        }                                \
    } while (0)

int SNEPPX_dev_quantize_int8_channel(const float* in, int8_t* q, float* scales, size_t rows,
                                     size_t cols, SNEPPXStream stream) {
    REQUIRE(in && q && scales, "dev_quantize_int8_channel: NULL pointer");
    REQUIRE(rows && cols, "dev_quantize_int8_channel: empty matrix");
    snx_clear_error();
    return snx_k_quant_int8_rows(in, q, scales, rows, cols, 0, stream);
}

int SNEPPX_dev_quantize_int8_channel_rounding(const float* in, int8_t* q, float* scales,
                                              size_t rows, size_t cols, SNEPPXRounding rounding,
                                              SNEPPXStream stream) {
    REQUIRE(in && q && scales, "dev_quantize_int8_channel_rounding: NULL pointer");
    REQUIRE(rows && cols, "dev_quantize_int8_channel_rounding: empty matrix");
    REQUIRE(rounding == SNEPPX_ROUND_HALF_AWAY || rounding == SNEPPX_ROUND_HALF_EVEN,
            "dev_quantize_int8_channel_rounding: unknown rounding %d", (int)rounding);
    snx_clear_error();
    return snx_k_quant_int8_rows(in, q, scales, rows, cols, rounding == SNEPPX_ROUND_HALF_EVEN,
                                 stream);
}

int SNEPPX_dev_fake_quant(const float* in, float* out, size_t n, float scale, int bits,
                          SNEPPXStream stream) {
    REQUIRE(in && out, "dev_fake_quant: NULL pointer");
    REQUIRE(scale > 0.0f, "dev_fake_quant: scale must be > 0");
    REQUIRE(bits >= 2 && bits <= 16, "dev_fake_quant: bits=%d outside [2, 16]", bits);
    snx_clear_error();
    if (n == 0) return 0;
    return snx_k_fake_quant(in, out, n, scale, bits, stream);
}

int SNEPPX_dev_quantize_w4_awq(const float* w, uint32_t* qweight, uint16_t* scales,
                               uint32_t* qzeros, size_t N, size_t K, int group,
                               SNEPPXStream stream) {
    REQUIRE(w && qweight && scales && qzeros, "dev_quantize_w4_awq: NULL pointer");
    REQUIRE(N && K, "dev_quantize_w4_awq: empty matrix");
    REQUIRE(group > 0 && group % 8 == 0 && K % (size_t)group == 0,
            "dev_quantize_w4_awq: group %d must be a positive multiple of 8 dividing K=%zu",
            group, K);
    snx_clear_error();
    return snx_k_w4_awq_quantize(w, qweight, scales, qzeros, N, K, group, stream);
}

/* g_idx is checked on the host (one small copy) so the kernel's LDS indexing
 * by group stays in bounds. */
int SNEPPX_dev_quantize_w4_gptq(const float* w, const int32_t* g_idx, size_t G,
                                uint32_t* qweight, uint16_t* scales, size_t N, size_t K,
                                SNEPPXStream stream) {
    REQUIRE(w && g_idx && qweight && scales, "dev_quantize_w4_gptq: NULL pointer");
    REQUIRE(N && K && G, "dev_quantize_w4_gptq: empty shape");
    REQUIRE(K % 8 == 0, "dev_quantize_w4_gptq: K=%zu must be a multiple of 8", K);
    snx_clear_error();
    int32_t* h = (int32_t*)malloc(K * sizeof(int32_t));
    REQUIRE(h, "dev_quantize_w4_gptq: out of host memory");
    int rc = snx_hip_memcpy_d2h(h, g_idx, K * sizeof(int32_t), stream);
    if (rc == 0) rc = snx_hip_stream_sync(stream);
    for (size_t k = 0; rc == 0 && k < K; k++)
        if (h[k] < 0 || (size_t)h[k] >= G) {
            snx_set_error("dev_quantize_w4_gptq: g_idx[%zu]=%d outside [0, %zu)", k, h[k], G);
            rc = -1;
        }
    free(h);
    if (rc) return -1;
    return snx_k_w4_gptq_quantize(w, g_idx, G, qweight, scales, N, K, stream);
}

int SNEPPX_dev_quantize_fp8_e4m3_scaled(const float* in, uint8_t* out, float* scale_out,
                                        size_t n, SNEPPXStream stream) {
    REQUIRE(in && out && scale_out, "dev_quantize_fp8_e4m3_scaled: NULL pointer");
    REQUIRE(n, "dev_quantize_fp8_e4m3_scaled: n == 0");
    snx_clear_error();
    int parts = snx_reduce_parts(n);
    float* ws = (float*)snx_workspace(((size_t)parts * 2 + 64) * sizeof(float), 0, stream);
    if (!ws) return -1;
    float* rec = ws + (size_t)parts * 2;
    rec = (float*)(((uintptr_t)rec + 15u) & ~(uintptr_t)15u);
    int rc = snx_k_absmax(in, n, ws, parts, stream);
    if (!rc) rc = snx_k_finalize_scale(ws, parts, SNX_SCALE_FP8_240, in, rec, scale_out, stream);
    if (!rc) rc = snx_k_fp8_encode(in, out, n, 0, rec, stream);
    return rc;
}

int SNEPPX_qlinear_w8_gemv(const float* x, const int8_t* qweight, const float* scales,
                           const float* bias, float* y, size_t M, size_t N, size_t K,
                           SNEPPXStream stream) {
    REQUIRE(x && qweight && scales && y, "qlinear_w8_gemv: NULL pointer");
    REQUIRE(M && N && K, "qlinear_w8_gemv: empty shape");
    REQUIRE(K % 16 != 0 || (aligned16(x) && aligned16(qweight)),
            "qlinear_w8_gemv: x and qweight must be 16-byte aligned");
    snx_clear_error();
    return snx_k_w8_gemv(x, qweight, scales, y, bias, M, N, K, stream);
}

/* Scratch of one W4A16 call: the calling thread's workspace on `stream`, or
 * for the allocation-free entry point the library's static device array
 * (NULL, with the error text set, when the call needs more than it holds). */
static void* w4_scratch(size_t bytes, int noalloc, SNEPPXStream stream) {
    return noalloc ? snx_noalloc_scratch(bytes, "qlinear_w4a16_noalloc")
                   : snx_workspace(bytes, 1, stream);
}

static int w4a16_linear(const char* who, int noalloc, const uint16_t* x, const uint32_t* qweight,
                        const uint16_t* scales, const uint32_t* qzeros, const int32_t* g_idx,
                        size_t G, const float* bias, void* y, SNEPPXDtype y_dtype, size_t M,
                        size_t N, size_t K, int group, SNEPPXStream stream) {
    REQUIRE(x && qweight && scales && y, "%s: NULL pointer", who);
    REQUIRE(M && N && K, "%s: empty shape", who);
    REQUIRE(K % 8 == 0, "%s: K=%zu must be a multiple of 8", who, K);
    REQUIRE(y_dtype == SNEPPX_BFLOAT16 || y_dtype == SNEPPX_FLOAT32,
            "%s: y_dtype must be SNEPPX_BFLOAT16 or SNEPPX_FLOAT32", who);
    int y_f32 = y_dtype == SNEPPX_FLOAT32;
    if (g_idx) {
        REQUIRE(G > 0, "%s: G must be > 0 with g_idx", who);
    } else {
        REQUIRE(group > 0 && K % (size_t)group == 0, "%s: group %d must divide K=%zu", who, group, K);
        G = K / (size_t)group;
    }
    snx_clear_error();
    if (!g_idx && M >= SNX_W4_GEMM_MIN_M && aligned16(x) && aligned16(qweight) &&
        ((uintptr_t)scales & 3u) == 0 && ((uintptr_t)qzeros & 3u) == 0 &&
        snx_w4a16_gemm_ok(M, N, K, group)) {
        /* prefill GEMM: activations prepared once into the call's scratch */
        const size_t Mp = snx_w4_prep_rows(M);
        const size_t xp_bytes = (M * K * sizeof(uint16_t) + 255) & ~(size_t)255;
        char* ws = (char*)w4_scratch(xp_bytes + (K / 128) * Mp * sizeof(float), noalloc, stream);
        if (!ws) return -1;
        uint16_t* xp = (uint16_t*)ws;
        float* xs = (float*)(ws + xp_bytes);
        /* with few tiles, K in spans (partials in a workspace; not for the
         * allocation-free entry point) */
        const int splits = noalloc ? 1 : snx_w4a16_gemm_splits(M, N, K);
        void* part = NULL;
        uint32_t* cnt = NULL;
        if (splits > 1) {
            part = snx_workspace(snx_w4a16_gemm_part_bytes(M, N, splits), 3, stream);
            cnt = (uint32_t*)snx_workspace_zeroed(snx_w4a16_gemm_cnt_bytes(M, N), 4, stream);
            if (!part || !cnt) return -1;
        }
        int rc = snx_k_w4_prep_x(x, xp, xs, M, K, Mp, stream);
        if (!rc) rc = snx_k_w4a16_gemm(xp, xs, qweight, scales, qzeros, y, bias, y_f32, M, N, K,
                                       group, Mp, splits, part, cnt, stream);
        return rc;
    }
    if (!g_idx && snx_w4a16_mt_ok(M, K, group, 0) && aligned16(x) && aligned16(qweight) &&
        ((uintptr_t)scales & 3u) == 0 && ((uintptr_t)qzeros & 3u) == 0) {
        /* 2 <= M <= 16: one persistent workgroup per CU, activations staged once */
        return snx_k_w4a16_gemv_mt(x, qweight, scales, qzeros, NULL, y, bias, y_f32, M, N, K, stream);
    }
    const int kspan = snx_w4a16_splitk_span(M, K, group);
    if (!g_idx && (M > 4 || (M > 1 && !snx_w4a16_small_ok(M, K, group, 0))) && kspan &&
        aligned16(x) && aligned16(qweight)) {
        /* 5 <= M <= 16, and 2 <= M <= 4 where the LDS-staged small-M kernel does
         * not apply (large K): split-K decode + ordered reduction of the partials */
        const size_t S = K / (size_t)kspan;
        float* part = (float*)w4_scratch(S * M * N * sizeof(float), noalloc, stream);
        if (!part) return -1;
        int rc = snx_k_w4a16_splitk(x, qweight, scales, qzeros, part, M, N, K, group, kspan, stream);
        if (!rc) rc = snx_k_w4a16_reduce(part, y, y_f32, (int)S, M * N, N, bias, stream);
        return rc;
    }
    if (!g_idx && M == 1 && aligned16(x) && aligned16(qweight) &&
        snx_w4a16_gemv1_ok(1, K, group, scales, qzeros))
        /* the streaming M = 1 kernel (K a multiple of 256 up to 16384) */
        return snx_k_w4a16_gemv(x, qweight, scales, qzeros, NULL, y, bias, y_f32, 1, N, K, group, stream);
    if (!g_idx && aligned16(x) && aligned16(qweight) &&
        snx_w4a16_gemv_supported(M < 64 ? M : 64, N, K, group)) {
        /* decode GEMV; larger M in 64-row slices that reuse each weight load */
        size_t ob = y_f32 ? 4 : 2;
        for (size_t m0 = 0; m0 < M; m0 += 64) {
            size_t mm = M - m0 < 64 ? M - m0 : 64;
            if (snx_k_w4a16_gemv(x + m0 * K, qweight, scales, qzeros, NULL,
                                 (char*)y + m0 * N * ob, bias, y_f32, mm, N, K, group, stream))
                return -1;
        }
        return 0;
    }
    return snx_k_w4a16_generic(x, qweight, scales, qzeros, g_idx, G, y, bias, y_f32, M, N, K,
                               group, stream);
}

int SNEPPX_qlinear_w4a16(const uint16_t* x, const uint32_t* qweight, const uint16_t* scales,
                         const uint32_t* qzeros, const int32_t* g_idx, size_t G,
                         const float* bias, void* y, SNEPPXDtype y_dtype, size_t M, size_t N,
                         size_t K, int group, SNEPPXStream stream) {
    return w4a16_linear("qlinear_w4a16", 0, x, qweight, scales, qzeros, g_idx, G, bias, y, y_dtype,
                        M, N, K, group, stream);
}

int SNEPPX_qlinear_w4a16_noalloc(const uint16_t* x, const uint32_t* qweight,
                                 const uint16_t* scales, const uint32_t* qzeros,
                                 const int32_t* g_idx, size_t G, const float* bias, void* y,
                                 SNEPPXDtype y_dtype, size_t M, size_t N, size_t K, int group,
                                 SNEPPXStream stream) {
    return w4a16_linear("qlinear_w4a16_noalloc", 1, x, qweight, scales, qzeros, g_idx, G, bias, y,
                        y_dtype, M, N, K, group, stream);
}

/* Stable counting sort of g_idx on the host (one small copy each way). */
int SNEPPX_qlinear_w4_actorder_prepare(const uint32_t* qweight, const int32_t* g_idx, size_t G,
                                       uint32_t* qweight_sorted, uint16_t* perm, size_t N,
                                       size_t K, SNEPPXStream stream) {
    REQUIRE(qweight && g_idx && qweight_sorted && perm, "w4_actorder_prepare: NULL pointer");
    REQUIRE(N && K && G, "w4_actorder_prepare: empty shape");
    REQUIRE(qweight != qweight_sorted, "w4_actorder_prepare: qweight_sorted must not alias qweight");
    REQUIRE(K % 8 == 0 && K <= 65536, "w4_actorder_prepare: K=%zu must be a multiple of 8 and <= 65536", K);
    REQUIRE(K % G == 0, "w4_actorder_prepare: G=%zu must divide K=%zu", G, K);
    snx_clear_error();
    const size_t per = K / G;
    int32_t* h = (int32_t*)malloc(K * sizeof(int32_t));
    uint16_t* hp = (uint16_t*)malloc(K * sizeof(uint16_t));
    size_t* next = (size_t*)calloc(G, sizeof(size_t));
    int rc = (h && hp && next) ? 0 : -1;
    if (rc) snx_set_error("w4_actorder_prepare: out of host memory");
    if (!rc) rc = snx_hip_memcpy_d2h(h, g_idx, K * sizeof(int32_t), stream);
    if (!rc) rc = snx_hip_stream_sync(stream);
    for (size_t k = 0; !rc && k < K; k++) {
        if (h[k] < 0 || (size_t)h[k] >= G) {
            snx_set_error("w4_actorder_prepare: g_idx[%zu]=%d outside [0, %zu)", k, h[k], G);
            rc = -1;
        } else if (next[h[k]]++ == per) {
            snx_set_error("w4_actorder_prepare: group %d holds more than K/G=%zu columns", h[k], per);
            rc = -1;
        }
    }
    /* every group now holds exactly K/G columns: slot g*per + rank in g */
    for (size_t g = 0; !rc && g < G; g++) next[g] = g * per;
    for (size_t k = 0; !rc && k < K; k++) hp[next[h[k]]++] = (uint16_t)k;
    if (!rc) rc = snx_hip_memcpy_h2d(perm, hp, K * sizeof(uint16_t), stream);
    if (!rc) rc = snx_k_w4_permute_cols(qweight, perm, qweight_sorted, N, K, stream);
    if (!rc) rc = snx_hip_stream_sync(stream);
    free(h);
    free(hp);
    free(next);
    return rc ? -1 : 0;
}

int SNEPPX_qlinear_w4a16_actorder(const uint16_t* x, const uint32_t* qweight_sorted,
                                  const uint16_t* scales, const uint32_t* qzeros,
                                  const uint16_t* perm, const float* bias, void* y,
                                  SNEPPXDtype y_dtype, size_t M, size_t N, size_t K, int group,
                                  SNEPPXStream stream) {
    REQUIRE(x && qweight_sorted && scales && perm && y, "qlinear_w4a16_actorder: NULL pointer");
    REQUIRE(M && N && K, "qlinear_w4a16_actorder: empty shape");
    REQUIRE(K % 8 == 0 && K <= 65536, "qlinear_w4a16_actorder: K=%zu must be a multiple of 8 and <= 65536", K);
    REQUIRE(y_dtype == SNEPPX_BFLOAT16 || y_dtype == SNEPPX_FLOAT32,
            "qlinear_w4a16_actorder: y_dtype must be SNEPPX_BFLOAT16 or SNEPPX_FLOAT32");
    REQUIRE(group > 0 && K % (size_t)group == 0,
            "qlinear_w4a16_actorder: group %d must divide K=%zu", group, K);
    snx_clear_error();
    if (aligned16(x) && aligned16(qweight_sorted) && aligned16(perm) && ((uintptr_t)scales & 3u) == 0 &&
        ((uintptr_t)qzeros & 3u) == 0 && snx_w4a16_mt_ok(M, K, group, 1))
        return snx_k_w4a16_gemv_mt(x, qweight_sorted, scales, qzeros, perm, y, bias,
                                   y_dtype == SNEPPX_FLOAT32, M, N, K, stream);
    if (aligned16(x) && aligned16(qweight_sorted) && aligned16(perm) &&
        (snx_w4a16_small_ok(M, K, group, 1) || snx_w4a16_gemv1_ok(M, K, group, scales, qzeros)))
        return snx_k_w4a16_gemv(x, qweight_sorted, scales, qzeros, perm, y, bias,
                                y_dtype == SNEPPX_FLOAT32, M, N, K, group, stream);
    /* other shapes: gather the activation columns once, then the plain path */
    uint16_t* xs = (uint16_t*)snx_workspace(M * K * sizeof(uint16_t), 0, stream);
    if (!xs) return -1;
    int rc = snx_k_gather_cols(x, perm, xs, M, K, stream);
    if (!rc) rc = SNEPPX_qlinear_w4a16(xs, qweight_sorted, scales, qzeros, NULL, 0, bias, y,
                                       y_dtype, M, N, K, group, stream);
    return rc;
}

int SNEPPX_qlinear_w4a16_swiglu(const uint16_t* x, const uint32_t* qweight,
                                const uint16_t* scales, const uint32_t* qzeros, const float* bias,
                                uint16_t* out, size_t M, size_t F, size_t K, int group,
                                SNEPPXStream stream) {
    REQUIRE(x && qweight && scales && out, "qlinear_w4a16_swiglu: NULL pointer");
    REQUIRE(M && F && K, "qlinear_w4a16_swiglu: empty shape");
    REQUIRE(F % 8 == 0 && K % 8 == 0, "qlinear_w4a16_swiglu: F=%zu and K=%zu must be multiples of 8",
            F, K);
    REQUIRE(group > 0 && K % (size_t)group == 0, "qlinear_w4a16_swiglu: group %d must divide K=%zu",
            group, K);
    REQUIRE(aligned16(out), "qlinear_w4a16_swiglu: out must be 16-byte aligned");
    snx_clear_error();
    if (M >= SNX_W4_GEMM_MIN_M && aligned16(x) && aligned16(qweight) &&
        ((uintptr_t)scales & 3u) == 0 && ((uintptr_t)qzeros & 3u) == 0 &&
        snx_w4a16_gemm_ok(M, 2 * F, K, group)) {
        const size_t Mp = snx_w4_prep_rows(M);
        const size_t xp_bytes = (M * K * sizeof(uint16_t) + 255) & ~(size_t)255;
        char* ws = (char*)snx_workspace(xp_bytes + (K / 128) * Mp * sizeof(float), 1, stream);
        if (!ws) return -1;
        uint16_t* xp = (uint16_t*)ws;
        float* xs = (float*)(ws + xp_bytes);
        int rc = snx_k_w4_prep_x(x, xp, xs, M, K, Mp, stream);
        if (!rc) rc = snx_k_w4a16_gemm_swiglu(xp, xs, qweight, scales, qzeros, out, bias, M, F, K,
                                              group, Mp, stream);
        return rc;
    }
    /* one decode row: gate and up rows of an output in one wave, SwiGLU on its total */
    if (M == 1 && aligned16(x) && aligned16(qweight) &&
        snx_w4a16_gemv1_swiglu_ok(F, K, group, scales, qzeros))
        return snx_k_w4a16_gemv1_swiglu(x, qweight, scales, qzeros, bias, out, F, K, group, stream);
    /* other decode rows: the [M][2F] projection in fp32 scratch, then the same rule */
    float* gu = (float*)snx_workspace(M * 2 * F * sizeof(float), 0, stream);
    if (!gu) return -1;
    int rc = SNEPPX_qlinear_w4a16(x, qweight, scales, qzeros, NULL, 0, bias, gu, SNEPPX_FLOAT32, M,
                                  2 * F, K, group, stream);
    if (!rc) rc = snx_k_silu_mul_f32(gu, out, M, F, stream);
    return rc;
}

/* workspace slot of the MLP's SwiGLU rows (prepared or plain) */
#define SLOT_MLP_ACT 6

int SNEPPX_qlinear_w4a16_mlp(const uint16_t* x, const uint32_t* gu_qweight, const uint16_t* gu_scales,
                             const uint32_t* gu_qzeros, const float* gu_bias, const uint32_t* dn_qweight,
                             const uint16_t* dn_scales, const uint32_t* dn_qzeros, const float* dn_bias,
                             void* y, SNEPPXDtype y_dtype, size_t M, size_t H, size_t F, size_t N,
                             int group, SNEPPXStream stream) {
    REQUIRE(x && gu_qweight && gu_scales && dn_qweight && dn_scales && y, "qlinear_w4a16_mlp: NULL pointer");
    REQUIRE(M && H && F && N, "qlinear_w4a16_mlp: empty shape");
    REQUIRE(F % 8 == 0 && H % 8 == 0, "qlinear_w4a16_mlp: F=%zu and H=%zu must be multiples of 8", F, H);
    REQUIRE(group > 0 && H % (size_t)group == 0 && F % (size_t)group == 0,
            "qlinear_w4a16_mlp: group %d must divide H=%zu and F=%zu", group, H, F);
    REQUIRE(y_dtype == SNEPPX_BFLOAT16 || y_dtype == SNEPPX_FLOAT32,
            "qlinear_w4a16_mlp: y_dtype must be SNEPPX_BFLOAT16 or SNEPPX_FLOAT32");
    snx_clear_error();
    const int aligned = aligned16(x) && aligned16(gu_qweight) && aligned16(dn_qweight) &&
                        ((uintptr_t)gu_scales & 3u) == 0 && ((uintptr_t)gu_qzeros & 3u) == 0 &&
                        ((uintptr_t)dn_scales & 3u) == 0 && ((uintptr_t)dn_qzeros & 3u) == 0;
    if (M >= SNX_W4_GEMM_MIN_M && aligned && F % 128 == 0 && snx_w4a16_gemm_ok(M, 2 * F, H, group) &&
        snx_w4a16_gemm_ok(M, N, F, group)) {
        /* x prepared once; the gate/up GEMM's SwiGLU epilogue writes the down
         * GEMM's prepared input (slot order + step sums) */
        const size_t Mp = snx_w4_prep_rows(M);
        const size_t xp_bytes = (M * H * sizeof(uint16_t) + 255) & ~(size_t)255;
        char* ws = (char*)snx_workspace(xp_bytes + (H / 128) * Mp * sizeof(float), 1, stream);
        const size_t ap_bytes = (M * F * sizeof(uint16_t) + 255) & ~(size_t)255;
        char* wa = (char*)snx_workspace(ap_bytes + (F / 128) * Mp * sizeof(float), SLOT_MLP_ACT, stream);
        if (!ws || !wa) return -1;
        uint16_t* xp = (uint16_t*)ws;
        float* xs = (float*)(ws + xp_bytes);
        uint16_t* ap = (uint16_t*)wa;
        float* as = (float*)(wa + ap_bytes);
        const int splits = snx_w4a16_gemm_splits(M, N, F);
        void* part = NULL;
        uint32_t* cnt = NULL;
        if (splits > 1) {
            part = snx_workspace(snx_w4a16_gemm_part_bytes(M, N, splits), 3, stream);
            cnt = (uint32_t*)snx_workspace_zeroed(snx_w4a16_gemm_cnt_bytes(M, N), 4, stream);
            if (!part || !cnt) return -1;
        }
        int rc = snx_k_w4_prep_x(x, xp, xs, M, H, Mp, stream);
        if (!rc) rc = snx_k_w4a16_gemm_swiglu_prep(xp, xs, gu_qweight, gu_scales, gu_qzeros, ap, as, gu_bias,
                                                   M, F, H, group, Mp, stream);
        if (!rc) rc = snx_k_w4a16_gemm(ap, as, dn_qweight, dn_scales, dn_qzeros, y, dn_bias,
                                       y_dtype == SNEPPX_FLOAT32, M, N, F, group, Mp, splits, part, cnt,
                                       stream);
        return rc;
    }
    /* other shapes: the two linears, the SwiGLU rows in a workspace */
    uint16_t* act = (uint16_t*)snx_workspace(M * F * sizeof(uint16_t), SLOT_MLP_ACT, stream);
    if (!act) return -1;
    int rc = SNEPPX_qlinear_w4a16_swiglu(x, gu_qweight, gu_scales, gu_qzeros, gu_bias, act, M, F, H, group,
                                         stream);
    if (!rc) rc = SNEPPX_qlinear_w4a16(act, dn_qweight, dn_scales, dn_qzeros, NULL, 0, dn_bias, y, y_dtype,
                                       M, N, F, group, stream);
    return rc;
}

int SNEPPX_qlinear_silu_mul(const uint16_t* gate_up, uint16_t* out, size_t T, size_t F,
                            SNEPPXStream stream) {
    REQUIRE(gate_up && out, "qlinear_silu_mul: NULL pointer");
    REQUIRE(T && F, "qlinear_silu_mul: empty shape");
    REQUIRE(F % 8 == 0, "qlinear_silu_mul: F=%zu must be a multiple of 8", F);
    REQUIRE(aligned16(gate_up) && aligned16(out), "qlinear_silu_mul: buffers must be 16-byte aligned");
    snx_clear_error();
    return snx_k_silu_mul(gate_up, out, T, F, stream);
}

int SNEPPX_qlinear_silu_mul_quant_int8(const uint16_t* gate_up, int8_t* q, float* scales,
                                       size_t T, size_t F, SNEPPXStream stream) {
    REQUIRE(gate_up && q && scales, "qlinear_silu_mul_quant_int8: NULL pointer");
    REQUIRE(T && F, "qlinear_silu_mul_quant_int8: empty shape");
    REQUIRE(F % 8 == 0 && F <= 32768, "qlinear_silu_mul_quant_int8: F=%zu must be a multiple of 8, <= 32768", F);
    REQUIRE(aligned16(gate_up) && ((uintptr_t)q & 7u) == 0,
            "qlinear_silu_mul_quant_int8: gate_up must be 16-byte and q 8-byte aligned");
    snx_clear_error();
    return snx_k_silu_mul_quant_int8(gate_up, q, scales, T, F, stream);
}

int SNEPPX_dev_quantize_int8_channel_bf16(const uint16_t* in, int8_t* q, float* scales,
                                          size_t rows, size_t cols, SNEPPXStream stream) {
    REQUIRE(in && q && scales, "dev_quantize_int8_channel_bf16: NULL pointer");
    REQUIRE(rows && cols, "dev_quantize_int8_channel_bf16: empty matrix");
    snx_clear_error();
    return snx_k_quant_rows_bf16_fast(in, q, scales, rows, cols, stream);
}

int SNEPPX_qlinear_w8a8_i8(const int8_t* A, const float* sA, const int8_t* W, const float* sW,
                           const float* bias, uint16_t* out, size_t M, size_t N, size_t K,
                           SNEPPXStream stream) {
    REQUIRE(A && sA && W && sW && out, "qlinear_w8a8_i8: NULL pointer");
    REQUIRE(M && N && K, "qlinear_w8a8_i8: empty shape");
    REQUIRE(aligned16(A) && aligned16(W), "qlinear_w8a8_i8: A and W must be 16-byte aligned");
    snx_clear_error();
    return snx_k_i8_gemm(A, W, sA, sW, NULL, out, bias, M, N, K, stream);
}

int SNEPPX_qlinear_i8_gemm_i32(const int8_t* A, const int8_t* W, int32_t* C, size_t M, size_t N,
                               size_t K, SNEPPXStream stream) {
    REQUIRE(A && W && C, "qlinear_i8_gemm_i32: NULL pointer");
    REQUIRE(M && N && K, "qlinear_i8_gemm_i32: empty shape");
    REQUIRE(aligned16(A) && aligned16(W), "qlinear_i8_gemm_i32: A and W must be 16-byte aligned");
    snx_clear_error();
    return snx_k_i8_gemm(A, W, NULL, NULL, C, NULL, NULL, M, N, K, stream);
}

int SNEPPX_qlinear_w8a8_fp8(const uint8_t* A, const float* sA, const uint8_t* W, const float* sW,
                            const float* bias, uint16_t* out, size_t M, size_t N, size_t K,
                            SNEPPXStream stream) {
    REQUIRE(A && sA && W && sW && out, "qlinear_w8a8_fp8: NULL pointer");
    REQUIRE(M && N && K, "qlinear_w8a8_fp8: empty shape");
    REQUIRE(aligned16(A) && aligned16(W), "qlinear_w8a8_fp8: A and W must be 16-byte aligned");
    snx_clear_error();
    return snx_k_fp8_gemm(A, W, sA, sW, out, bias, M, N, K, stream);
}

/* Workspace slot of the dynamically quantized activations (codes, then the
 * per-token scales or the per-tensor scale record at a 256-byte boundary). */
#define SLOT_W8A8_DYN 5

int SNEPPX_qlinear_w8a8_i8_dyn(const uint16_t* A, const int8_t* W, const float* sW,
                               const float* bias, uint16_t* out, size_t M, size_t N, size_t K,
                               SNEPPXStream stream) {
    REQUIRE(A && W && sW && out, "qlinear_w8a8_i8_dyn: NULL pointer");
    REQUIRE(M && N && K, "qlinear_w8a8_i8_dyn: empty shape");
    REQUIRE(aligned16(A) && aligned16(W), "qlinear_w8a8_i8_dyn: A and W must be 16-byte aligned");
    snx_clear_error();
    const size_t qb = (M * K + 255) & ~(size_t)255;
    char* ws = (char*)snx_workspace(qb + M * sizeof(float), SLOT_W8A8_DYN, stream);
    if (!ws) return -1;
    int8_t* aq = (int8_t*)ws;
    float* sa = (float*)(ws + qb);
    int rc = snx_k_quant_rows_bf16_fast(A, aq, sa, M, K, stream);
    if (!rc) rc = snx_k_i8_gemm(aq, W, sa, sW, NULL, out, bias, M, N, K, stream);
    return rc;
}

int SNEPPX_qlinear_w8a8_fp8_dyn(const uint16_t* A, const uint8_t* W, const float* sW,
                                const float* bias, uint16_t* out, size_t M, size_t N, size_t K,
                                SNEPPXStream stream) {
    REQUIRE(A && W && sW && out, "qlinear_w8a8_fp8_dyn: NULL pointer");
    REQUIRE(M && N && K, "qlinear_w8a8_fp8_dyn: empty shape");
    REQUIRE(aligned16(A) && aligned16(W), "qlinear_w8a8_fp8_dyn: A and W must be 16-byte aligned");
    snx_clear_error();
    const size_t n = M * K, qb = (n + 255) & ~(size_t)255;
    const int parts = snx_reduce_parts(n);
    char* ws = (char*)snx_workspace(qb + ((size_t)parts * 2 + 64) * sizeof(float), SLOT_W8A8_DYN, stream);
    if (!ws) return -1;
    uint8_t* aq = (uint8_t*)ws;
    float* part = (float*)(ws + qb);
    float* rec = part + (size_t)parts * 2;
    rec = (float*)(((uintptr_t)rec + 15u) & ~(uintptr_t)15u);
    int rc = snx_k_absmax_bf16(A, n, part, parts, stream);
    /* rec[0] = s_A, the per-tensor scale the GEMM's epilogue multiplies by:
     * the encode kernel reduces the partials itself when it can take the
     * vector path, else a one-block finalize does */
    if (!rc && n % 8 == 0 && ((uintptr_t)aq & 7u) == 0) {
        rc = snx_k_fp8_encode_bf16_pt(A, aq, n, part, parts, rec, stream);
    } else if (!rc) {
        rc = snx_k_finalize_scale(part, parts, SNX_SCALE_FP8_240, NULL, rec, NULL, stream);
        if (!rc) rc = snx_k_fp8_encode_bf16(A, aq, n, rec, stream);
    }
    if (!rc) rc = snx_k_fp8_gemm(aq, W, rec, sW, out, bias, M, N, K, stream);
    return rc;
}
