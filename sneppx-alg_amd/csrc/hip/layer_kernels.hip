// layer_kernels.hip - data movement for the quantized layers of
// include/sneppx_qlayer.h: the [K][N] -> [N][K] weight transpose done once at
// load time, and fp32 -> bf16 activations in front of the W4A16 linears.
// Pure copies and one IEEE rounding; no arithmetic on the values otherwise.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "codec.h"
#include "../snx_internal.h"

using namespace snx;

namespace {

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// 64 x 64 tiles through LDS (row stride 65 floats: the column reads of the
// store phase hit 64 different banks); 256 threads, 16 elements each.
__global__ void __launch_bounds__(256) k_transpose_f32(const float* __restrict__ in,
                                                       float* __restrict__ out, size_t R,
                                                       size_t Cc) {
    __shared__ float t[64][65];
    const size_t r0 = (size_t)blockIdx.y * 64, c0 = (size_t)blockIdx.x * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const size_t r = r0 + ty + 4 * i, c = c0 + tx;
        if (r < R && c < Cc) t[ty + 4 * i][tx] = in[r * Cc + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const size_t c = c0 + ty + 4 * i, r = r0 + tx;
        if (r < R && c < Cc) out[c * R + r] = t[tx][ty + 4 * i];
    }
}

__global__ void __launch_bounds__(256) k_f32_to_bf16(const float* __restrict__ x,
                                                     uint16_t* __restrict__ y, size_t n) {
    for (size_t i = blockIdx.x * (size_t)256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        y[i] = bf16_out(x[i]);
}

}  // namespace

extern "C" {

int snx_k_transpose_f32(const float* in, float* out, size_t rows, size_t cols, void* st) {
    const size_t gx = (cols + 63) / 64, gy = (rows + 63) / 64;
    if (gx > 0x7fffffff || gy > 65535) {
        snx_set_error("transpose: %zu x %zu is too large", rows, cols);
        return -1;
    }
    k_transpose_f32<<<dim3((unsigned)gx, (unsigned)gy), 256, 0, S(st)>>>(in, out, rows, cols);
    return snx_launch_check("k_transpose_f32");
}

int snx_k_f32_to_bf16(const float* x, uint16_t* y, size_t n, void* st) {
    size_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    k_f32_to_bf16<<<(unsigned)(blocks ? blocks : 1), 256, 0, S(st)>>>(x, y, n);
    return snx_launch_check("k_f32_to_bf16");
}

}  // extern "C"
