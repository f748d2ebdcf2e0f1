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
