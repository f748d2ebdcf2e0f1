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
#include <type_traits>

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

// ------------------------------------------------------------ tiled GEMM
// Workgroup tile 256 (M) x 224 (N); 4 waves in 2 x 2, each 128 x 112 =
// 8 x 7 MFMA blocks of 16 x 16.  K advances in 128-byte stages staged in LDS
// (row stride 144 B: 16 rows of one fragment read land on distinct banks),
// double-buffered: global loads for stage t+1 are issued before the MFMAs of
// stage t and written to the other buffer after them, one barrier per stage.
// int8 uses two v_mfma_i32_16x16x64_i8 k-halves per stage, fp8 one
// v_mfma_f32_16x16x128_f8f6f4.  Tiles are mapped so that each XCD (the
// dispatcher deals workgroups to the 8 XCDs round-robin) owns a compact
// 8 x (tiles_n / 8) block and keeps its A and W rows in its own L2.
constexpr int TBM = 256, TBN = 224, TBK = 128, TLDS = 144;
constexpr int TFM = 8, TFN = 7;   // fragments per wave
constexpr int TLDS_A = TBM * TLDS, TLDS_B = TBN * TLDS, TLDS_STAGE = TLDS_A + TLDS_B;

template <bool FP8, bool RAW>
__global__ void __launch_bounds__(256) k_gemm_tiled(const int8_t* __restrict__ A,
                                                    const int8_t* __restrict__ W,
                                                    const float* __restrict__ sA,
                                                    const float* __restrict__ sW,
                                                    int32_t* __restrict__ Craw,
                                                    uint16_t* __restrict__ out, int M, int N, int K,
                                                    int tiles_m, int tiles_n) {
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int r16 = lane & 15, q = lane >> 4;

    // XCD-aware tile order
    const int b = blockIdx.x, nb = gridDim.x;
    int tile;
    if (nb % 8 == 0) {
        const int per = nb / 8;
        tile = (b % 8) * per + b / 8;
    } else {
        tile = b;
    }
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int m0 = tm * TBM, n0 = tn * TBN;

    // global -> LDS staging: A 2048 chunks (8/thread), W 1792 chunks (7/thread);
    // thread t moves chunk (row t/8 + 32 i, 16-byte column t%8).  Global
    // offsets are 32-bit (the launcher checks M*K and N*K fit).
    const int srow = tid >> 3, scol = (tid & 7) * 16;
    uint32_t ga[8], gw[7];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int gr = m0 + srow + 32 * i < M ? m0 + srow + 32 * i : M - 1;
        ga[i] = (uint32_t)gr * (uint32_t)K + scol;
    }
#pragma unroll
    for (int i = 0; i < 7; i++) {
        const int gr = n0 + srow + 32 * i < N ? n0 + srow + 32 * i : N - 1;
        gw[i] = (uint32_t)gr * (uint32_t)K + scol;
    }
    const int lbase = srow * TLDS + scol;

    i32x4 ra[8], rw[7];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 8; i++) ra[i] = *reinterpret_cast<const i32x4*>(A + ga[i] + k0);
#pragma unroll
        for (int i = 0; i < 7; i++) rw[i] = *reinterpret_cast<const i32x4*>(W + gw[i] + k0);
    };
    auto lstore = [&](int buf) {
        int8_t* base = lds + buf * TLDS_STAGE + lbase;
#pragma unroll
        for (int i = 0; i < 8; i++) *reinterpret_cast<i32x4*>(base + i * 32 * TLDS) = ra[i];
#pragma unroll
        for (int i = 0; i < 7; i++) *reinterpret_cast<i32x4*>(base + TLDS_A + i * 32 * TLDS) = rw[i];
    };

    typedef typename std::conditional<FP8, f32x4, i32x4>::type acc_t;
    acc_t acc[TFM][TFN];
#pragma unroll
    for (int i = 0; i < TFM; i++)
#pragma unroll
        for (int j = 0; j < TFN; j++) acc[i][j] = acc_t{0, 0, 0, 0};

    const int a_off = (wm * 128 + r16) * TLDS;
    const int w_off = TLDS_A + (wn * 112 + r16) * TLDS;
    const int nk = K / TBK;

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * TBK);
        const int8_t* base = lds + cur * TLDS_STAGE;
        if (FP8) {
            i32x8 fa[TFM], fw[TFN];
#pragma unroll
            for (int i = 0; i < TFM; i++) {
                const i32x4 lo = *reinterpret_cast<const i32x4*>(base + a_off + i * 16 * TLDS + q * 32);
                const i32x4 hi = *reinterpret_cast<const i32x4*>(base + a_off + i * 16 * TLDS + q * 32 + 16);
                fa[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int j = 0; j < TFN; j++) {
                const i32x4 lo = *reinterpret_cast<const i32x4*>(base + w_off + j * 16 * TLDS + q * 32);
                const i32x4 hi = *reinterpret_cast<const i32x4*>(base + w_off + j * 16 * TLDS + q * 32 + 16);
                fw[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int i = 0; i < TFM; i++)
#pragma unroll
                for (int j = 0; j < TFN; j++)
                    acc[i][j] = (acc_t)__builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        fa[i], fw[j], (f32x4)acc[i][j], 0, 0, 0, 0, 0, 0);
        } else {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                i32x4 fa[TFM], fw[TFN];
#pragma unroll
                for (int i = 0; i < TFM; i++)
                    fa[i] = *reinterpret_cast<const i32x4*>(base + a_off + i * 16 * TLDS + h * 64 + q * 16);
#pragma unroll
                for (int j = 0; j < TFN; j++)
                    fw[j] = *reinterpret_cast<const i32x4*>(base + w_off + j * 16 * TLDS + h * 64 + q * 16);
#pragma unroll
                for (int i = 0; i < TFM; i++)
#pragma unroll
                    for (int j = 0; j < TFN; j++)
                        acc[i][j] = (acc_t)__builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fw[j], (i32x4)acc[i][j], 0, 0, 0);
            }
        }
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

    // epilogue: C row 4*(lane/16)+e, col lane%16 of each 16 x 16 block
    float sa_tile[TFM][4];
    float sw_tile[TFN];
    if (!RAW) {
#pragma unroll
        for (int i = 0; i < TFM; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 128 + i * 16 + q * 4 + e;
                sa_tile[i][e] = FP8 ? sA[0] : sA[m < M ? m : M - 1];
            }
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            const int n = n0 + wn * 112 + j * 16 + r16;
            sw_tile[j] = FP8 ? sW[0] : sW[n < N ? n : N - 1];
        }
    }
#pragma unroll
    for (int i = 0; i < TFM; i++)
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            const int n = n0 + wn * 112 + j * 16 + r16;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 128 + i * 16 + q * 4 + e;
                if (m >= M) continue;
                if (RAW)
                    Craw[(size_t)m * N + n] = ((i32x4)acc[i][j])[e];
                else
                    out[(size_t)m * N + n] = f32_to_bf16((float)acc[i][j][e] * sa_tile[i][e] * sw_tile[j]);
            }
        }
}

template <bool FP8, bool RAW>
int launch_tiled(const int8_t* A, const int8_t* W, const float* sA, const float* sW, int32_t* Craw,
                 uint16_t* out, int M, int N, int K, hipStream_t st) {
    const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
    if ((uint64_t)M * K >= (1ull << 32) || (uint64_t)N * K >= (1ull << 32)) {
        snx_set_error("gemm: operands above 4 GiB are not supported");
        return -1;
    }
    const size_t lds = 2 * (size_t)TLDS_STAGE;
    static bool attr_set = false;   // one-time opt-in to > 64 KB of LDS per workgroup
    if (!attr_set) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemm_tiled<FP8, RAW>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            snx_set_error("gemm: cannot reserve %zu bytes of LDS", lds);
            return -1;
        }
        attr_set = true;
    }
    k_gemm_tiled<FP8, RAW><<<tiles_m * tiles_n, 256, lds, st>>>(A, W, sA, sW, Craw, out, M, N, K,
                                                               tiles_m, tiles_n);
    return snx_launch_check("k_gemm_tiled");
}

}  // namespace

extern "C" {

int snx_k_i8_gemm(const int8_t* A, const int8_t* W, const float* sA, const float* sW,
                  int32_t* c_i32, uint16_t* out_bf16, size_t M, size_t N, size_t K, void* st) {
    if (K % 16 != 0) {
        snx_set_error("i8 gemm: K=%zu must be a multiple of 16", K);
        return -1;
    }
    if (K % TBK == 0 && M >= 128 && N >= 128) {
        if (c_i32)
            return launch_tiled<false, true>(A, W, sA, sW, c_i32, out_bf16, (int)M, (int)N, (int)K, S(st));
        return launch_tiled<false, false>(A, W, sA, sW, c_i32, out_bf16, (int)M, (int)N, (int)K, S(st));
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
    if (K % TBK == 0 && M >= 128 && N >= 128)
        return launch_tiled<true, false>(reinterpret_cast<const int8_t*>(A), reinterpret_cast<const int8_t*>(W),
                                         sA, sW, nullptr, out_bf16, (int)M, (int)N, (int)K, S(st));
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    k_fp8_gemm<<<grid, 256, 0, S(st)>>>(A, W, sA, sW, out_bf16, (int)M, (int)N, (int)K);
    return snx_launch_check("k_fp8_gemm");
}

}  // extern "C"
