// gemm_kernels.hip - W8A8 prefill GEMMs for gfx950 (MFMA-bound).
//
//  * int8 x int8 -> int32 on v_mfma_i32_16x16x64_i8 (exact accumulators),
//    epilogue bf16((acc * sA[m]) * sW[n]) or the raw int32 tile.
//  * fp8 e4m3 x e4m3 -> fp32 on v_mfma_f32_16x16x128_f8f6f4, epilogue
//    bf16((acc * sA) * sW) with per-tensor scales read from device memory.
// Both operands are K-contiguous ("TN": A [M][K], W [N][K]).  Each MFMA lane
// reads the K-bytes of its own row for A and of its own column for W at the
// same k offsets, so A and B agree on every k-slot by construction.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "codec.h"
#include "../snx_internal.h"

using namespace snx;

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// 16 bytes of row `r` at column k (zero beyond K; K % 16 == 0 is required).
__device__ __forceinline__ i32x4 frag16(const int8_t* base, int rows, int r, int K, int k) {
    if (r >= rows || k >= K) return i32x4{0, 0, 0, 0};
    return *reinterpret_cast<const i32x4*>(base + (size_t)r * K + k);
}

// Workgroup tile 64x64 (4 waves in 2x2, each 32x32 = 2x2 MFMA tiles).
template <bool RAW>
__global__ void __launch_bounds__(256) k_i8_gemm(const int8_t* __restrict__ A,
                                                 const int8_t* __restrict__ W,
                                                 const float* __restrict__ sA,
                                                 const float* __restrict__ sW,
                                                 int32_t* __restrict__ Craw,
                                                 uint16_t* __restrict__ out, int M, int N, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.y * 64 + (wave >> 1) * 32, n0 = blockIdx.x * 64 + (wave & 1) * 32;
    const int r16 = lane & 15, kq = lane >> 4;
    i32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = i32x4{0, 0, 0, 0};
    for (int k = 0; k < K; k += 64) {
        i32x4 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = frag16(A, M, m0 + i * 16 + r16, K, k + kq * 16);
#pragma unroll
        for (int j = 0; j < 2; j++) b[j] = frag16(W, N, n0 + j * 16 + r16, K, k + kq * 16);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + j * 16 + r16;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + i * 16 + kq * 4 + e;   // C row 4*(lane/16)+e, col lane%16
                if (m >= M) continue;
                if (RAW)
                    Craw[(size_t)m * N + n] = acc[i][j][e];
                else
                    out[(size_t)m * N + n] = f32_to_bf16((float)acc[i][j][e] * sA[m] * sW[n]);
            }
        }
}

__device__ __forceinline__ i32x8 frag32(const uint8_t* base, int rows, int r, int K, int k) {
    if (r >= rows || k >= K) return i32x8{0, 0, 0, 0, 0, 0, 0, 0};
    return *reinterpret_cast<const i32x8*>(base + (size_t)r * K + k);
}

__global__ void __launch_bounds__(256) k_fp8_gemm(const uint8_t* __restrict__ A,
                                                  const uint8_t* __restrict__ W,
                                                  const float* __restrict__ sA,
                                                  const float* __restrict__ sW,
                                                  uint16_t* __restrict__ out, int M, int N, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.y * 64 + (wave >> 1) * 32, n0 = blockIdx.x * 64 + (wave & 1) * 32;
    const int r16 = lane & 15, kq = lane >> 4;
    f32x4 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < K; k += 128) {
        i32x8 a[2], b[2];
#pragma unroll
        for (int i = 0; i < 2; i++) a[i] = frag32(A, M, m0 + i * 16 + r16, K, k + kq * 32);
#pragma unroll
        for (int j = 0; j < 2; j++) b[j] = frag32(W, N, n0 + j * 16 + r16, K, k + kq * 32);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[i], b[j], acc[i][j],
                                                                             0, 0, 0, 0, 0, 0);
    }
    const float sa = sA[0], sw = sW[0];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + j * 16 + r16;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + i * 16 + kq * 4 + e;
                if (m < M) out[(size_t)m * N + n] = f32_to_bf16(acc[i][j][e] * sa * sw);
            }
        }
}

}  // namespace

extern "C" {

int snx_k_i8_gemm(const int8_t* A, const int8_t* W, const float* sA, const float* sW,
                  int32_t* c_i32, uint16_t* out_bf16, size_t M, size_t N, size_t K, void* st) {
    if (K % 16 != 0) {
        snx_set_error("i8 gemm: K=%zu must be a multiple of 16", K);
        return -1;
    }
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (c_i32)
        k_i8_gemm<true><<<grid, 256, 0, S(st)>>>(A, W, sA, sW, c_i32, out_bf16, (int)M, (int)N, (int)K);
    else
        k_i8_gemm<false><<<grid, 256, 0, S(st)>>>(A, W, sA, sW, c_i32, out_bf16, (int)M, (int)N, (int)K);
    return snx_launch_check("k_i8_gemm");
}

int snx_k_fp8_gemm(const uint8_t* A, const uint8_t* W, const float* sA, const float* sW,
                   uint16_t* out_bf16, size_t M, size_t N, size_t K, void* st) {
    if (K % 32 != 0) {
        snx_set_error("fp8 gemm: K=%zu must be a multiple of 32", K);
        return -1;
    }
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    k_fp8_gemm<<<grid, 256, 0, S(st)>>>(A, W, sA, sW, out_bf16, (int)M, (int)N, (int)K);
    return snx_launch_check("k_fp8_gemm");
}

}  // extern "C"
