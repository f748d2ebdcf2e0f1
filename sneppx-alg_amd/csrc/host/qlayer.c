/*
 * qlayer.c - quantized linear layers at the reference's linear call sites
 * (include/sneppx_qlayer.h).  A layer owns its device buffers; creation
 * transposes the reference's [K][N] weight to [N][K] on the device and runs
 * the device quantizers; forward calls the sneppx_qlinear.h entry points.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sneppx_qlayer.h"
#include "snx_hip.h"
#include "../snx_internal.h"

/* workspace slot of this file (qlinear.c uses 0 and 1 inside the linears) */
#define SLOT_X_BF16 2

struct SNEPPXQLayer {
    int format;
    size_t K, N, G;
    int group;            /* W4: columns per group (0: groups given by g_idx) */
    /* W8 */
    int8_t* q8;
    float* s8;
    /* W4 */
    uint32_t* qweight;    /* as stored: column order k */
    uint16_t* scales;
    uint32_t* qzeros;     /* NULL: symmetric, zero 8 */
    int32_t* g_idx;       /* NULL: contiguous groups */
    uint32_t* qsorted;    /* act-order prepared (group-contiguous) codes, or NULL */
    uint16_t* perm;
    float* bias;          /* fp32 [N] or NULL */
};

void SNEPPX_qlayer_destroy(SNEPPXQLayer* L) {
    if (!L) return;
    snx_hip_free(L->q8);
    snx_hip_free(L->s8);
    snx_hip_free(L->qweight);
    snx_hip_free(L->scales);
    snx_hip_free(L->qzeros);
    snx_hip_free(L->g_idx);
    snx_hip_free(L->qsorted);
    snx_hip_free(L->perm);
    snx_hip_free(L->bias);
    free(L);
}

static int set_bias(SNEPPXQLayer* L, const float* b, int on_device, SNEPPXStream stream) {
    if (!L) { snx_set_error("qlayer_set_bias: NULL layer"); return -1; }
    snx_clear_error();
    if (!b) {
        snx_hip_free(L->bias);
        L->bias = NULL;
        return 0;
    }
    if (!L->bias && snx_hip_malloc((void**)&L->bias, L->N * sizeof(float))) return -1;
    int rc = on_device ? snx_hip_memcpy_d2d(L->bias, b, L->N * sizeof(float), stream)
                       : snx_hip_memcpy_h2d(L->bias, b, L->N * sizeof(float), stream);
    if (!rc && !on_device) rc = snx_hip_stream_sync(stream);   /* the host buffer may go away */
    return rc;
}

int SNEPPX_qlayer_set_bias(SNEPPXQLayer* L, const float* bias, SNEPPXStream stream) {
    return set_bias(L, bias, 0, stream);
}

int SNEPPX_qlayer_set_bias_device(SNEPPXQLayer* L, const float* d_bias, SNEPPXStream stream) {
    return set_bias(L, d_bias, 1, stream);
}

/* <prefix>.bias: F32 [N] when present (written by SNEPPX_qlayer_save) */
static int load_bias(SNEPPXQLayer* L, const SNEPPXQStore* st, const char* prefix,
                     SNEPPXStream stream) {
    char key[512];
    snprintf(key, sizeof key, "%s.bias", prefix);
    int dt;
    size_t shape[SNEPPX_QST_MAX_DIMS], nd, nb;
    if (SNEPPX_qstore_info(st, key, &dt, shape, &nd, &nb)) return 0;   /* no bias */
    if (dt != SNEPPX_QST_F32 || nd != 1 || shape[0] != L->N) {
        snx_set_error("qlayer_load: %s must be F32 [%zu]", key, L->N);
        return -1;
    }
    if (snx_hip_malloc((void**)&L->bias, L->N * sizeof(float))) return -1;
    return SNEPPX_qstore_read_device(st, key, L->bias, L->N * sizeof(float), stream);
}

size_t SNEPPX_qlayer_in_features(const SNEPPXQLayer* L) { return L ? L->K : 0; }
size_t SNEPPX_qlayer_out_features(const SNEPPXQLayer* L) { return L ? L->N : 0; }
int SNEPPX_qlayer_format(const SNEPPXQLayer* L) { return L ? L->format : -1; }

static int dalloc(void** p, size_t bytes) { return snx_hip_malloc(p, bytes ? bytes : 1); }

/* device buffers for a layer of the given shape */
static SNEPPXQLayer* alloc_layer(int format, size_t K, size_t N, int group, size_t G, int zeros,
                                 int gidx) {
    SNEPPXQLayer* L = (SNEPPXQLayer*)calloc(1, sizeof *L);
    if (!L) { snx_set_error("qlayer: out of host memory"); return NULL; }
    L->format = format;
    L->K = K;
    L->N = N;
    L->G = G;
    L->group = group;
    int rc = 0;
    if (format == SNEPPX_QLAYER_W8) {
        rc |= dalloc((void**)&L->q8, N * K);
        rc |= dalloc((void**)&L->s8, N * 4);
    } else {
        rc |= dalloc((void**)&L->qweight, N * K / 2);
        rc |= dalloc((void**)&L->scales, N * G * 2);
        if (zeros) rc |= dalloc((void**)&L->qzeros, N * ((G + 7) / 8) * 4);
        if (gidx) rc |= dalloc((void**)&L->g_idx, K * 4);
    }
    if (rc) {
        SNEPPX_qlayer_destroy(L);
        return NULL;
    }
    return L;
}

SNEPPXQLayer* SNEPPX_qlayer_create_kn_device(const float* d_w_kn, size_t K, size_t N,
                                             SNEPPXQLayerFormat format, int group,
                                             SNEPPXStream stream) {
    if (!d_w_kn || !K || !N) { snx_set_error("qlayer_create_kn: empty or NULL weight"); return NULL; }
    if (format != SNEPPX_QLAYER_W8 && format != SNEPPX_QLAYER_W4) {
        snx_set_error("qlayer_create_kn: unknown format %d", (int)format);
        return NULL;
    }
    if (format == SNEPPX_QLAYER_W4 &&
        (group <= 0 || group % 8 || K % (size_t)group)) {
        snx_set_error("qlayer_create_kn: group %d must be a positive multiple of 8 dividing K=%zu",
                      group, K);
        return NULL;
    }
    snx_clear_error();
    const size_t G = format == SNEPPX_QLAYER_W4 ? K / (size_t)group : 0;
    SNEPPXQLayer* L = alloc_layer(format, K, N, format == SNEPPX_QLAYER_W4 ? group : 0, G,
                                  format == SNEPPX_QLAYER_W4, 0);
    if (!L) return NULL;
    float* wt = NULL;
    int rc = dalloc((void**)&wt, N * K * 4);
    if (!rc) rc = snx_k_transpose_f32(d_w_kn, wt, K, N, stream);   /* [K][N] -> [N][K] */
    if (!rc) {
        if (format == SNEPPX_QLAYER_W8)
            rc = SNEPPX_dev_quantize_int8_channel(wt, L->q8, L->s8, N, K, stream);
        else
            rc = SNEPPX_dev_quantize_w4_awq(wt, L->qweight, L->scales, L->qzeros, N, K, group, stream);
    }
    if (!rc) rc = snx_hip_stream_sync(stream);
    if (wt) snx_hip_free(wt);
    if (rc) {
        SNEPPX_qlayer_destroy(L);
        return NULL;
    }
    return L;
}

SNEPPXQLayer* SNEPPX_qlayer_create_kn(const float* w_kn, size_t K, size_t N,
                                      SNEPPXQLayerFormat format, int group, SNEPPXStream stream) {
    if (!w_kn || !K || !N) { snx_set_error("qlayer_create_kn: empty or NULL weight"); return NULL; }
    float* d = NULL;
    if (dalloc((void**)&d, K * N * 4)) return NULL;
    SNEPPXQLayer* L = NULL;
    if (snx_hip_memcpy_h2d(d, w_kn, K * N * 4, stream) == 0)
        L = SNEPPX_qlayer_create_kn_device(d, K, N, format, group, stream);
    snx_hip_stream_sync(stream);
    snx_hip_free(d);
    return L;
}

/* act-order layers: prepare the group-contiguous form when every group has
 * K/G columns; otherwise the layer keeps using g_idx (generic kernel) */
static int try_prepare(SNEPPXQLayer* L, SNEPPXStream stream) {
    if (!L->g_idx || L->K > 65536) return 0;
    if (dalloc((void**)&L->qsorted, L->N * L->K / 2) || dalloc((void**)&L->perm, L->K * 2)) return -1;
    if (SNEPPX_qlinear_w4_actorder_prepare(L->qweight, L->g_idx, L->G, L->qsorted, L->perm, L->N,
                                           L->K, stream) == 0)
        return 0;
    snx_hip_free(L->qsorted);
    snx_hip_free(L->perm);
    L->qsorted = NULL;
    L->perm = NULL;
    snx_clear_error();   /* uneven groups are a valid layer, just not a prepared one */
    return 0;
}

SNEPPXQLayer* SNEPPX_qlayer_load(const SNEPPXQStore* st, const char* prefix, SNEPPXStream stream) {
    if (!st || !prefix) { snx_set_error("qlayer_load: NULL argument"); return NULL; }
    char key[512];
    snprintf(key, sizeof key, "%s.format", prefix);
    const char* fmt = SNEPPX_qstore_metadata(st, key);
    size_t N, K, G;
    if (fmt && strcmp(fmt, "w8") == 0) {
        if (SNEPPX_qstore_query_w8(st, prefix, &N, &K)) return NULL;
        SNEPPXQLayer* L = alloc_layer(SNEPPX_QLAYER_W8, K, N, 0, 0, 0, 0);
        if (!L) return NULL;
        if (SNEPPX_qstore_load_w8(st, prefix, L->q8, L->s8, stream) ||
            load_bias(L, st, prefix, stream)) {
            SNEPPX_qlayer_destroy(L);
            return NULL;
        }
        return L;
    }
    int group, hz, hg;
    if (SNEPPX_qstore_query_w4(st, prefix, &N, &K, &G, &group, &hz, &hg)) {
        if (!fmt && SNEPPX_qstore_query_w8(st, prefix, &N, &K) == 0) {   /* W8 without metadata */
            SNEPPXQLayer* L = alloc_layer(SNEPPX_QLAYER_W8, K, N, 0, 0, 0, 0);
            if (!L) return NULL;
            if (SNEPPX_qstore_load_w8(st, prefix, L->q8, L->s8, stream) ||
                load_bias(L, st, prefix, stream)) {
                SNEPPX_qlayer_destroy(L);
                return NULL;
            }
            return L;
        }
        return NULL;
    }
    if (!hg && (group < 8 || group % 8)) {
        snx_set_error("qlayer_load: %s has groups of %d columns (need a multiple of 8)", prefix, group);
        return NULL;
    }
    SNEPPXQLayer* L = alloc_layer(SNEPPX_QLAYER_W4, K, N, hg ? 0 : group, G, hz, hg);
    if (!L) return NULL;
    if (SNEPPX_qstore_load_w4(st, prefix, L->qweight, L->scales, L->qzeros, L->g_idx, stream) ||
        load_bias(L, st, prefix, stream) || try_prepare(L, stream)) {
        SNEPPX_qlayer_destroy(L);
        return NULL;
    }
    return L;
}

int SNEPPX_qlayer_save(const SNEPPXQLayer* L, SNEPPXQStoreWriter* w, const char* prefix,
                       SNEPPXStream stream) {
    if (!L || !w || !prefix) { snx_set_error("qlayer_save: NULL argument"); return -1; }
    int rc = L->format == SNEPPX_QLAYER_W8
                 ? SNEPPX_qstore_save_w8(w, prefix, L->q8, L->s8, L->N, L->K, stream)
                 : SNEPPX_qstore_save_w4(w, prefix, L->qweight, L->scales, L->qzeros, L->g_idx,
                                         L->N, L->K, L->group, L->G, stream);
    if (!rc && L->bias) {
        char key[512];
        snprintf(key, sizeof key, "%s.bias", prefix);
        const size_t shape[1] = {L->N};
        rc = SNEPPX_qstore_writer_add_device(w, key, SNEPPX_QST_F32, shape, 1, L->bias, stream);
    }
    return rc;
}

/* W4A16 with bf16 activations, output in y_dtype */
static int run_w4(const SNEPPXQLayer* L, const uint16_t* xb, void* y, SNEPPXDtype ydt, size_t M,
                  SNEPPXStream stream) {
    if (L->qsorted)   /* act-order, prepared: groups of K/G sorted columns */
        return SNEPPX_qlinear_w4a16_actorder(xb, L->qsorted, L->scales, L->qzeros, L->perm, L->bias,
                                             y, ydt, M, L->N, L->K, (int)(L->K / L->G), stream);
    return SNEPPX_qlinear_w4a16(xb, L->qweight, L->scales, L->qzeros, L->g_idx, L->G, L->bias, y,
                                ydt, M, L->N, L->K, L->group, stream);
}

int SNEPPX_qlayer_forward_f32(const SNEPPXQLayer* L, const float* d_x, float* d_y, size_t M,
                              SNEPPXStream stream) {
    if (!L || !d_x || !d_y) { snx_set_error("qlayer_forward_f32: NULL argument"); return -1; }
    if (!M) { snx_set_error("qlayer_forward_f32: M = 0"); return -1; }
    snx_clear_error();
    if (L->format == SNEPPX_QLAYER_W8)
        return SNEPPX_qlinear_w8_gemv(d_x, L->q8, L->s8, L->bias, d_y, M, L->N, L->K, stream);
    uint16_t* xb = (uint16_t*)snx_workspace(M * L->K * 2, SLOT_X_BF16, stream);
    if (!xb) return -1;
    if (snx_k_f32_to_bf16(d_x, xb, M * L->K, stream)) return -1;
    return run_w4(L, xb, d_y, SNEPPX_FLOAT32, M, stream);
}

int SNEPPX_qlayer_forward_bf16(const SNEPPXQLayer* L, const uint16_t* d_x, uint16_t* d_y,
                               size_t M, SNEPPXStream stream) {
    if (!L || !d_x || !d_y) { snx_set_error("qlayer_forward_bf16: NULL argument"); return -1; }
    if (!M) { snx_set_error("qlayer_forward_bf16: M = 0"); return -1; }
    if (L->format != SNEPPX_QLAYER_W4) {
        snx_set_error("qlayer_forward_bf16: a W8 layer takes fp32 activations");
        return -1;
    }
    snx_clear_error();
    return run_w4(L, d_x, d_y, SNEPPX_BFLOAT16, M, stream);
}

/* Each call owns its stream and its staging (stream-ordered allocations from
 * the device pool), so concurrent calls share no buffer: the workspaces the
 * linears take inside are keyed by (thread, stream) and this stream is the
 * call's own. */
int SNEPPX_qlayer_matmul_host(const SNEPPXQLayer* L, const float* x, float* y, size_t M) {
    if (!L || !x || !y || !M) { snx_set_error("qlayer_matmul_host: NULL or empty argument"); return -1; }
    const size_t xb = M * L->K * 4, yb = M * L->N * 4;
    void* st = NULL;
    if (snx_hip_stream_create(&st)) return -1;
    float* dx = NULL;
    float* dy = NULL;
    int rc = snx_hip_malloc_async((void**)&dx, xb, st);
    if (!rc) rc = snx_hip_malloc_async((void**)&dy, yb, st);
    if (!rc) rc = snx_hip_memcpy_h2d(dx, x, xb, st);
    if (!rc) rc = SNEPPX_qlayer_forward_f32(L, dx, dy, M, st);
    if (!rc) rc = snx_hip_memcpy_d2h(y, dy, yb, st);
    snx_hip_free_async(dx, st);
    snx_hip_free_async(dy, st);
    const int rs = snx_hip_stream_sync(st);
    snx_release_workspaces(st);
    snx_hip_stream_destroy(st);
    return rc || rs ? -1 : 0;
}
