/*
 * bench_loop.c - back-to-back launch loops used by bench.py.
 *
 * Each function calls one decode entry point of libsneppx_quant.so `steps`
 * times from C, rotating over `copies` weight copies (so every call streams
 * its weights from HBM rather than from the Infinity Cache).  Timing the
 * loop between two events on the launch stream then measures the GPU, not
 * the Python interpreter's per-call cost, which for a ~5 us kernel is of the
 * same order as the kernel.  Not part of the product library.
 */
#include <stddef.h>
#include <stdint.h>

#include "sneppx_qlinear.h"

int snxb_loop_w4a16(int steps, int copies, const uint16_t* x, const uint32_t* const* qw,
                    const uint16_t* const* sc, const uint32_t* const* qz, void* y, int y_dtype,
                    size_t M, size_t N, size_t K, int group, SNEPPXStream stream) {
    for (int i = 0; i < steps; i++) {
        const int c = i % copies;
        if (SNEPPX_qlinear_w4a16(x, qw[c], sc[c], qz ? qz[c] : NULL, NULL, 0, NULL, y,
                                 (SNEPPXDtype)y_dtype, M, N, K, group, stream))
            return -1;
    }
    return 0;
}

int snxb_loop_w4a16_actorder(int steps, int copies, const uint16_t* x, const uint32_t* const* qw,
                             const uint16_t* const* sc, const uint16_t* perm, void* y, int y_dtype,
                             size_t M, size_t N, size_t K, int group, SNEPPXStream stream) {
    for (int i = 0; i < steps; i++) {
        const int c = i % copies;
        if (SNEPPX_qlinear_w4a16_actorder(x, qw[c], sc[c], NULL, perm, NULL, y, (SNEPPXDtype)y_dtype,
                                          M, N, K, group, stream))
            return -1;
    }
    return 0;
}

int snxb_loop_w8_gemv(int steps, int copies, const float* x, const int8_t* const* q,
                      const float* const* s, float* y, size_t M, size_t N, size_t K,
                      SNEPPXStream stream) {
    for (int i = 0; i < steps; i++) {
        const int c = i % copies;
        if (SNEPPX_qlinear_w8_gemv(x, q[c], s[c], NULL, y, M, N, K, stream)) return -1;
    }
    return 0;
}

/* One token (M = 1) through the linears of a decoder layer, or only its
 * gate/up projection with the SwiGLU step (layer == 0).  Copy c of the
 * weights is qw[4 c + j] (j: 0 QKV [QKV][H], 1 O [H][A], 2 stacked gate/up
 * [2F][H], 3 down [H][F]); only j = 2 is read when layer == 0.  A is the
 * attention width the O projection reads (H, or H / tp for one GPU's shard
 * of a tensor-parallel layer, where QKV and F are the shard's widths too).
 * The linears chain as in the layer: x -> qkv, the first A values of qkv
 * stand in for the attention output -> o, o -> h = silu(gate) * up, h -> y.
 * Attention, norms, residual adds and the tensor-parallel reductions are not
 * part of it. */
int snxb_loop_decode(int steps, int copies, int layer, const uint16_t* x,
                     const uint32_t* const* qw, const uint16_t* const* sc,
                     const uint32_t* const* qz, uint16_t* qkv, uint16_t* o, uint16_t* h,
                     uint16_t* y, size_t H, size_t QKV, size_t F, size_t A, SNEPPXStream stream) {
    for (int i = 0; i < steps; i++) {
        const int c = 4 * (i % copies);
        if (!layer) {
            if (SNEPPX_qlinear_w4a16_swiglu(x, qw[c + 2], sc[c + 2], qz[c + 2], NULL, h, 1, F, H, 128,
                                            stream))
                return -1;
            continue;
        }
        if (SNEPPX_qlinear_w4a16(x, qw[c], sc[c], qz[c], NULL, 0, NULL, qkv, SNEPPX_BFLOAT16, 1, QKV, H,
                                 128, stream) ||
            SNEPPX_qlinear_w4a16(qkv, qw[c + 1], sc[c + 1], qz[c + 1], NULL, 0, NULL, o, SNEPPX_BFLOAT16,
                                 1, H, A, 128, stream) ||
            SNEPPX_qlinear_w4a16_swiglu(o, qw[c + 2], sc[c + 2], qz[c + 2], NULL, h, 1, F, H, 128,
                                        stream) ||
            SNEPPX_qlinear_w4a16(h, qw[c + 3], sc[c + 3], qz[c + 3], NULL, 0, NULL, y, SNEPPX_BFLOAT16,
                                 1, H, F, 128, stream))
            return -1;
    }
    return 0;
}
