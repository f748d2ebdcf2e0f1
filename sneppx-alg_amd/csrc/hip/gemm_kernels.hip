// gemm_kernels.hip - W8A8 prefill GEMMs for gfx950 (MFMA-bound).
//
//  * int8 x int8 -> int32 on v_mfma_i32_16x16x64_i8 (exact accumulators),
//    epilogue bf16((acc * sA[m]) * sW[n]) or the raw int32 tile.
//  * fp8 e4m3 x e4m3 -> fp32 on v_mfma_f32_16x16x128_f8f6f4, epilogue
//    bf16((acc * sA) * sW) with per-tensor scales read from device memory.
//  * MXFP4 x MXFP4 (E2M1 codes, E8M0 block exponents) on the scaled
//    v_mfma_scale_f32_16x16x128_f8f6f4, staged like the fp8 kernel.
// Both operands are K-contiguous ("TN": A [M][K], W [N][K]).  Each MFMA lane
// reads the K-bytes of its own row for A and of its own column for W at the
// same k offsets, so A and B agree on every k-slot by construction.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "codec.h"
#include "launch.h"
#include "../snx_internal.h"

using namespace snx;

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Direct global -> LDS loads go through buffer_load ... lds: those count in
// vmcnt only, while global_load_lds also counts in lgkmcnt and so makes the
// compiler drain every LDS fragment read (lgkmcnt(0)) before each MFMA.
typedef __attribute__((address_space(3))) void* lds_ptr_t;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t brsrc(const void* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, -1, 0x00020000);
}
__device__ __forceinline__ void bload_lds(__amdgpu_buffer_rsrc_t r, void* dst, int bytes, uint32_t voff, uint32_t soff) {
    if (bytes == 16)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 16, voff, soff, 0, 0);
    else if (bytes == 12)   // lane l's 12 bytes land at dst + 16 l (a 16-byte slot, its last 4 bytes untouched)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 12, voff, soff, 0, 0);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)dst, 4, voff, soff, 0, 0);
}

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
                                                 uint16_t* __restrict__ out,
                                                 const float* __restrict__ bias, int M, int N,
                                                 int K) {
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
                    out[(size_t)m * N + n] = f32_to_bf16((float)acc[i][j][e] * sA[m] * sW[n] +
                                                         (bias ? bias[n] : 0.0f));
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
                                                  uint16_t* __restrict__ out,
                                                  const float* __restrict__ bias, int M, int N,
                                                  int K) {
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
            const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + i * 16 + kq * 4 + e;
                if (m < M) out[(size_t)m * N + n] = f32_to_bf16(acc[i][j][e] * sa * sw + bv);
            }
        }
}

// ------------------------------------------------------------ tiled GEMMs
// Workgroup tile 256 (M) x 224 (N), 8 waves.  K advances in 128-byte stages,
// double buffered in LDS (2 x 60 KB).  Operands go global -> LDS directly
// (buffer_load_dwordx4 ... lds: no staging registers, no ds_write): each wave
// instruction fills 8 rows x 128 B.  16-byte chunk c of tile row R sits at
// slot c ^ swz(R), swz(R) = (R & 7) ^ ((R >> 3) & 1): it depends on R mod 16
// only (fragment rows share it), and the 16 rows of a fragment read hit
// distinct bank groups whether LDS serves 8 or 16 lanes a cycle.  Tiles are
// dealt so each XCD (workgroups go to the 8 XCDs round-robin) owns a compact
// 8 x (tiles_n / 8) block.
constexpr int TBM = 256, TBN = 224, TBK = 128;
constexpr int TFN = 7;                                   // 16-column fragments per wave (fp8)
constexpr int TLDS_A = TBM * TBK, TLDS_B = TBN * TBK, TLDS_STAGE = TLDS_A + TLDS_B;

__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

typedef int i32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ i32x4 lds16(const int8_t* p) { return *reinterpret_cast<const i32x4*>(p); }

// fp8 (and the 16x16 int8 form): waves in 4 (M) x 2 (N), each 64 x 112 =
// 4 x 7 MFMA blocks of 16 x 16 (112 accumulators), two waves per SIMD, so one
// wave's LDS latency hides behind the other's MFMAs.
template <bool FP8, bool RAW, bool BIAS>
__global__ void __launch_bounds__(512) k_gemm_8w(const int8_t* __restrict__ A,
                                                 const int8_t* __restrict__ W,
                                                 const float* __restrict__ sA,
                                                 const float* __restrict__ sW,
                                                 int32_t* __restrict__ Craw,
                                                 uint16_t* __restrict__ out,
                                                 const float* __restrict__ bias, int M, int N,
                                                 int K, int tiles_m, int tiles_n) {
    constexpr int FM = 4;
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int r16 = lane & 15, q = lane >> 4;

    const int b = blockIdx.x, nb = gridDim.x;
    const int tile = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int m0 = tm * TBM, n0 = tn * TBN;

    // direct loads: A block 8*w' + ... : wave w, instruction i fills 1 KB block
    // i*8 + w (8 tile rows); A has 32 blocks, W 28
    const int lrow = lane >> 3, lslot = lane & 7;
    uint32_t ga[4], gw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (8 * i + wave) * 8 + lrow;
        const int gr = m0 + row < M ? m0 + row : M - 1;
        ga[i] = (uint32_t)gr * (uint32_t)K + (uint32_t)((lslot ^ swz(row)) * 16);
        const int wr = row < TBN ? row : TBN - 1;
        const int gn = n0 + wr < N ? n0 + wr : N - 1;
        gw[i] = (uint32_t)gn * (uint32_t)K + (uint32_t)((lslot ^ swz(wr)) * 16);
    }
    const __amdgpu_buffer_rsrc_t ra = brsrc(A), rw = brsrc(W);
    auto dload = [&](int buf, int k0) {
        int8_t* base = lds + buf * TLDS_STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) bload_lds(ra, base + (8 * i + wave) * 1024, 16, ga[i], k0);
#pragma unroll
        for (int i = 0; i < 3; i++) bload_lds(rw, base + TLDS_A + (8 * i + wave) * 1024, 16, gw[i], k0);
        if (wave < 4) bload_lds(rw, base + TLDS_A + (24 + wave) * 1024, 16, gw[3], k0);
    };

    typedef typename std::conditional<FP8, f32x4, i32x4>::type acc_t;
    acc_t acc[FM][TFN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < TFN; j++) acc[i][j] = acc_t{0, 0, 0, 0};

    const int sw = swz(r16);
    const int8_t* arow = lds + (wm * 64 + r16) * TBK;
    const int8_t* wrow = lds + TLDS_A + (wn * 112 + r16) * TBK;
    const int nk = K / TBK;

    dload(0, 0);
    // epilogue scales, fetched now so their latency hides under the K loop
    float sa[FM][4], swv[TFN], bv[TFN];
    if (!RAW) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 64 + i * 16 + q * 4 + e;
                sa[i][e] = FP8 ? sA[0] : sA[m < M ? m : M - 1];
            }
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            const int n = n0 + wn * 112 + j * 16 + r16;
            swv[j] = FP8 ? sW[0] : sW[n < N ? n : N - 1];
            bv[j] = BIAS ? bias[n < N ? n : N - 1] : 0.0f;
        }
    }
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        __builtin_amdgcn_s_waitcnt(0x0070);   // this stage landed; earlier LDS reads done
        __syncthreads();
        // loads for stage t+1 into the other buffer (last stage: stage 0 again, unused)
        dload(cur ^ 1, kt + 1 < nk ? (kt + 1) * TBK : 0);
        const int8_t* ab = arow + cur * TLDS_STAGE;
        const int8_t* wb = wrow + cur * TLDS_STAGE;
        if (!FP8) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                i32x4 fa[FM], fw[TFN];
                // k-half h takes chunks 2q + h (the even / odd chunks, the
                // same bank pattern as the fp8 reads; any k order works as
                // long as A and W agree)
#pragma unroll
                for (int i = 0; i < FM; i++) fa[i] = lds16(ab + i * 16 * TBK + (((2 * q + h) ^ sw) << 4));
#pragma unroll
                for (int j = 0; j < TFN; j++) fw[j] = lds16(wb + j * 16 * TBK + (((2 * q + h) ^ sw) << 4));
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < TFN; j++)
                        acc[i][j] = (acc_t)__builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fw[j], (i32x4)acc[i][j], 0, 0, 0);
            }
        } else {
            i32x8 fa[FM], fw[TFN];
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const i32x4 lo = lds16(ab + i * 16 * TBK + (((2 * q) ^ sw) << 4));
                const i32x4 hi = lds16(ab + i * 16 * TBK + (((2 * q + 1) ^ sw) << 4));
                fa[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int j = 0; j < TFN; j++) {
                const i32x4 lo = lds16(wb + j * 16 * TBK + (((2 * q) ^ sw) << 4));
                const i32x4 hi = lds16(wb + j * 16 * TBK + (((2 * q + 1) ^ sw) << 4));
                fw[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < TFN; j++)
                    acc[i][j] = (acc_t)__builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        fa[i], fw[j], (f32x4)acc[i][j], 0, 0, 0, 0, 0, 0);
        }
    }

#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            const int n = n0 + wn * 112 + j * 16 + r16;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 64 + i * 16 + q * 4 + e;
                if (m >= M) continue;
                if (RAW)
                    Craw[(size_t)m * N + n] = ((i32x4)acc[i][j])[e];
                else
                    out[(size_t)m * N + n] = BIAS ? bf16_out((float)acc[i][j][e] * sa[i][e] * swv[j] + bv[j])
                                                  : bf16_out((float)acc[i][j][e] * sa[i][e] * swv[j]);
            }
        }
    }
}

// MXFP4 x MXFP4 (E2M1 codes, one E8M0 exponent per 32 elements) on
// v_mfma_scale_f32_16x16x128_f8f6f4, staged like k_gemm_8w: 256 x 224 tiles,
// 8 waves of 64 x 112, K stages of 128 bytes (256 elements) global -> LDS
// with buffer_load_dwordx4 ... lds, double buffered.  Beside each stage sit the
// stage's 8 scale bytes of every tile row, as 4-byte direct loads (dword h of
// a row: the exponents of its blocks 4h .. 4h + 3), ordered so that each lane
// finds all the exponents of its fragments in 32 (A) + 64 (W) contiguous
// bytes: A dword ((wm * 16 + r16) * 4 + i) * 2 + h holds row wm*64 + 16i + r16,
// W dword ((wn * 16 + r16) * 8 + j) * 2 + h row wn*112 + 16j + r16 (j = 7
// repeats j = 6, never read).  Lane (r16, q) takes 16-byte chunk 2q + h of
// its row for k-step h (A and W alike: a permutation of the stage's k) -
// exactly one 32-element block, whose exponent is the lane's MFMA scale
// operand (int8 s -> E8M0 s + 127).  The lane's two exponents of a stage are
// bytes 2(q % 2), +1 of dword q / 2: one byte permute puts them in bytes 0 and
// 2, one packed 16-bit saturating subtract converts both, and the MFMA's scale
// byte select (op_sel 0 / 2) takes each.  The fp4 products are exact;
// accumulation is fp32.
constexpr int MXS_A = 4 * 16 * 4 * 2 * 4;         // bytes of A exponents per stage
constexpr int MXS_STAGE = TLDS_STAGE + 2 * MXS_A;  // + as many for W (7 of 8 used)

__device__ __forceinline__ int e8m0_of(int8_t s) { return s < -127 ? 0 : (int)s + 127; }
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
// the two exponent bytes of staged dwords {hi, lo} (bytes 4-7, 0-3) that sel
// picks (e.g. 0x0C010C00: bytes 0, 1 of lo; 0x0C050C01: byte 1 of lo and of
// hi) as E8M0 in bytes 0 and 2:
// max(s, -127) + 127 = (s ^ 0x80) - 1, saturating at 0, per 16-bit half
__device__ __forceinline__ int e8m0_pair(int hi, int lo, uint32_t sel) {
    const uint32_t u = __builtin_amdgcn_perm((uint32_t)hi, (uint32_t)lo, sel) ^ 0x00800080u;
    const u16x2 t = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, u), (u16x2){1, 1});
    return __builtin_bit_cast(int, t);
}

// SG picks where the exponents come from:
//  0: one exponent per operand (NVFP4's default): sA[0] + sW[0] split as
//     ceil / floor of its half (each at least -127), as k_mx_expand_scales
//     writes it into every block, passed to every MFMA as a constant;
//  1: staged beside each K stage, in the order above;
//  4: (K a multiple of 1024) every fourth stage loads the next four stages'
//     exponents, 32 bytes per row in two 16-byte direct loads, into one half
//     of a double-buffered 32 KB area after the two stages.  One cache line
//     per row per four stages instead of one per stage: the exponent loads
//     touch as many lines as the code loads otherwise.  Granule (16 bytes:
//     stages 2p, 2p + 1 of a row, dwords (stage, h)) order: A
//     ((wm * 2 + p) * 4 + i) * 16 + r16, W ((wn * 2 + p) * 8 + j) * 16 + r16
//     (j = 7 repeats j = 6, never read): the 16 rows one read instruction
//     takes sit in 256 contiguous bytes, free of bank conflicts.
constexpr int MXG_HALF = 2 * 512 * 16;   // bytes of one group of exponents (A, then W)
template <bool YF32, int SG>
__global__ void __launch_bounds__(512) k_mxfp4_tiled(const uint8_t* __restrict__ A,
                                                     const int8_t* __restrict__ sA,
                                                     const uint8_t* __restrict__ W,
                                                     const int8_t* __restrict__ sW,
                                                     void* __restrict__ out, int M, int N, int K,
                                                     int tiles_m, int tiles_n) {
    constexpr int FM = 4;
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int r16 = lane & 15, q = lane >> 4;

    const int b = blockIdx.x, nb = gridDim.x;
    const int tile = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int m0 = tm * TBM, n0 = tn * TBN;
    const uint32_t KB = (uint32_t)K / 2, KS = (uint32_t)K / 32;   // bytes per row: codes, scales

    const int lrow = lane >> 3, lslot = lane & 7;
    uint32_t ga[4], gw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (8 * i + wave) * 8 + lrow;
        const int gr = m0 + row < M ? m0 + row : M - 1;
        ga[i] = (uint32_t)gr * KB + (uint32_t)((lslot ^ swz(row)) * 16);
        const int wr = row < TBN ? row : TBN - 1;
        const int gn = n0 + wr < N ? n0 + wr : N - 1;
        gw[i] = (uint32_t)gn * KB + (uint32_t)((lslot ^ swz(wr)) * 16);
    }
    // SG 1: exponent dwords of a stage, 512 for A, 512 for W; SG 4: exponent
    // granules of a group, as many; wave w's lanes load items 64 w .. 64 w + 63
    // of each (the orders above)
    uint32_t gs[2] = {0u, 0u};
    if (SG == 1) {
        const int d = 64 * wave + lane, h = d & 1;
        const int ra = (d >> 7) * 64 + ((d >> 1) & 3) * 16 + ((d >> 3) & 15);
        const int gr = m0 + ra < M ? m0 + ra : M - 1;
        gs[0] = (uint32_t)gr * KS + 4 * h;
        const int j = (d >> 1) & 7;
        const int rw = (d >> 8) * 112 + (j < 7 ? j : 6) * 16 + ((d >> 4) & 15);
        const int gn = n0 + rw < N ? n0 + rw : N - 1;
        gs[1] = (uint32_t)gn * KS + 4 * h;
    } else if (SG == 4) {
        const int g = 64 * wave + lane;
        const int ra = (g >> 7) * 64 + ((g >> 4) & 3) * 16 + (g & 15);
        const int gr = m0 + ra < M ? m0 + ra : M - 1;
        gs[0] = (uint32_t)gr * KS + 16 * ((g >> 6) & 1);
        const int j = (g >> 4) & 7;
        const int rw = (g >> 8) * 112 + (j < 7 ? j : 6) * 16 + (g & 15);
        const int gn = n0 + rw < N ? n0 + rw : N - 1;
        gs[1] = (uint32_t)gn * KS + 16 * ((g >> 7) & 1);
    }
    constexpr int STG = SG == 1 ? MXS_STAGE : TLDS_STAGE;   // bytes per K stage
    const __amdgpu_buffer_rsrc_t ra = brsrc(A), rw = brsrc(W), rsa = brsrc(sA), rsw = brsrc(sW);
    auto dload = [&](int buf, int kt) {
        int8_t* base = lds + buf * STG;
        const uint32_t k0 = (uint32_t)kt * TBK;
#pragma unroll
        for (int i = 0; i < 4; i++) bload_lds(ra, base + (8 * i + wave) * 1024, 16, ga[i], k0);
#pragma unroll
        for (int i = 0; i < 3; i++) bload_lds(rw, base + TLDS_A + (8 * i + wave) * 1024, 16, gw[i], k0);
        if (wave < 4) bload_lds(rw, base + TLDS_A + (24 + wave) * 1024, 16, gw[3], k0);
        if (SG == 1) {
            bload_lds(rsa, base + TLDS_STAGE + wave * 256, 4, gs[0], kt * 8);
            bload_lds(rsw, base + TLDS_STAGE + MXS_A + wave * 256, 4, gs[1], kt * 8);
        }
    };
    auto gload = [&](int grp) {   // SG 4: exponents of stages 4 grp .. 4 grp + 3
        int8_t* base = lds + 2 * TLDS_STAGE + (grp & 1) * MXG_HALF;
        bload_lds(rsa, base + wave * 1024, 16, gs[0], grp * 32);
        bload_lds(rsw, base + MXG_HALF / 2 + wave * 1024, 16, gs[1], grp * 32);
    };
    int pta = 0, ptw = 0;
    if (SG == 0) {
        const int t = (int)sA[0] + (int)sW[0];
        pta = e8m0_of((int8_t)max(t - (t >> 1), -127)) * 0x10001;   // in bytes 0 and 2
        ptw = e8m0_of((int8_t)max(t >> 1, -127)) * 0x10001;
    }

    f32x4 acc[FM][TFN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < TFN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int sw = swz(r16);
    const int8_t* arow = lds + (wm * 64 + r16) * TBK;
    const int8_t* wrow = lds + TLDS_A + (wn * 112 + r16) * TBK;
    // this lane's exponent dword (q / 2) of its first A / W row in a stage
    const int8_t* srow_a = (SG == 1 ? lds + TLDS_STAGE + (wm * 16 + r16) * 32
                                    : lds + 2 * TLDS_STAGE + wm * 2048 + r16 * 16) + 4 * (q >> 1);
    const int8_t* srow_w = (SG == 1 ? lds + TLDS_STAGE + MXS_A + (wn * 16 + r16) * 64
                                    : lds + 2 * TLDS_STAGE + MXG_HALF / 2 + wn * 4096 + r16 * 16) + 4 * (q >> 1);
    const uint32_t psel = (q & 1) ? 0x0C030C02u : 0x0C010C00u;
    const int nk = K / (2 * TBK);

    dload(0, 0);
    if (SG == 4) gload(0);
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        __builtin_amdgcn_s_waitcnt(0x0070);   // this stage landed; earlier LDS reads done
        __syncthreads();
        dload(cur ^ 1, kt + 1 < nk ? kt + 1 : 0);   // last stage: stage 0 again, unused
        // the other half was last read in the previous group, before the barrier above
        if (SG == 4 && (kt & 3) == 0 && kt + 4 < nk) gload((kt >> 2) + 1);
        const int8_t* ab = arow + cur * STG;
        const int8_t* wb = wrow + cur * STG;
        // per fragment row, this lane's two exponents of the stage as E8M0 in bytes 0, 2
        int ea[FM], ew[TFN];
        if (SG == 0) {
#pragma unroll
            for (int i = 0; i < FM; i++) ea[i] = pta;
#pragma unroll
            for (int j = 0; j < TFN; j++) ew[j] = ptw;
        } else {
            // SG 4: group half, granule pair (kt / 2) % 2, stage kt % 2 within it
            const int8_t* xa = SG == 4 ? srow_a + ((kt >> 2) & 1) * MXG_HALF + ((kt >> 1) & 1) * 1024 + (kt & 1) * 8
                                       : srow_a + cur * STG;
            const int8_t* xw = SG == 4 ? srow_w + ((kt >> 2) & 1) * MXG_HALF + ((kt >> 1) & 1) * 2048 + (kt & 1) * 8
                                       : srow_w + cur * STG;
#pragma unroll
            for (int i = 0; i < FM; i++)
                ea[i] = e8m0_pair(0, *reinterpret_cast<const int*>(xa + (SG == 4 ? 256 : 8) * i), psel);
#pragma unroll
            for (int j = 0; j < TFN; j++)
                ew[j] = e8m0_pair(0, *reinterpret_cast<const int*>(xw + (SG == 4 ? 256 : 8) * j), psel);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = 2 * q + h;
            i32x8 fa[FM], fw[TFN];
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const i32x4 v = lds16(ab + i * 16 * TBK + ((c ^ sw) << 4));
                fa[i] = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
            }
#pragma unroll
            for (int j = 0; j < TFN; j++) {
                const i32x4 v = lds16(wb + j * 16 * TBK + ((c ^ sw) << 4));
                fw[j] = i32x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < TFN; j++)
                    acc[i][j] = h == 0 ? __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                             fa[i], fw[j], acc[i][j], 4, 4, 0, ea[i], 0, ew[j])
                                       : __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                                             fa[i], fw[j], acc[i][j], 4, 4, 2, ea[i], 2, ew[j]);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070);   // the last (unused) loads drain before exit

#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            const int n = n0 + wn * 112 + j * 16 + r16;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 64 + i * 16 + q * 4 + e;
                if (m >= M) continue;
                if (YF32)
                    reinterpret_cast<float*>(out)[(size_t)m * N + n] = acc[i][j][e];
                else
                    reinterpret_cast<uint16_t*>(out)[(size_t)m * N + n] = bf16_out(acc[i][j][e]);
            }
        }
    }
}

// MXFP8 / MXFP6 x the same format (block 32 along K, one E8M0 exponent per
// block) on v_mfma_scale_f32_16x16x128_f8f6f4: the fp8 kernel's 256 x 224
// tiles and 8 waves of 64 x 112, K stages of 128 elements (one MFMA step),
// double buffered, with each stage's scale bytes of every tile row (4 per
// row) staged beside it.  MF is the matrix cores' element format (0 e4m3,
// 1 e5m2, 2 e2m3, 3 e3m2), EB its bits.  A row of a stage is 128 * EB / 8
// bytes (8 or 6 chunks of 16 B); its chunks go to the XOR-swizzled slots of a
// 128-byte LDS row, and the two padding slots of an fp6 row load a chunk the
// same instruction loads anyway (no extra memory traffic; never read).
// Lane (r16, q) carries the exponent of block q of the stage (elements
// [32 q, +32)) as its MFMA scale.  Its operand registers hold, for fp6, that
// block (24 bytes, packed little-endian as the reference writes them); for
// fp8, elements [16 q, +16) in registers 0-3 and [64 + 16 q, +16) in 4-7 --
// the matrix cores' 8-bit k order, in which register half h of lane group q
// is scaled by the exponent of lane group 2 h + q / 2.  fp8 codes must be decodable by the
// matrix cores (no all-ones exponents: see k_mx_to_mfma).
constexpr int MX8_SCALES = 512;                          // scale dwords per stage (480 used)
constexpr int MX8_STAGE = TLDS_STAGE + MX8_SCALES * 4;

template <int MF, int EB, bool YF32>
__global__ void __launch_bounds__(512) k_mx8_tiled(const uint8_t* __restrict__ A,
                                                   const int8_t* __restrict__ sA,
                                                   const uint8_t* __restrict__ W,
                                                   const int8_t* __restrict__ sW,
                                                   void* __restrict__ out, int M, int N, int K,
                                                   int tiles_m, int tiles_n) {
    constexpr int FM = 4;
    constexpr int RB = 128 * EB / 8;                     // bytes of a row per stage
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int r16 = lane & 15, q = lane >> 4;

    const int b = blockIdx.x, nb = gridDim.x;
    const int tile = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int m0 = tm * TBM, n0 = tn * TBN;
    const uint32_t KB = (uint32_t)K * EB / 8, KS = (uint32_t)K / 32;   // code and scale bytes per row

    // LDS slot lslot (16 bytes) of row r holds piece lslot ^ swz(r) of the
    // row's stage bytes: 16-byte chunks of an fp8 row, 12-byte pieces of an
    // fp6 row (8 x 12 = its 96 bytes; a 12-byte load fills the first 12
    // bytes of each lane's 16-byte slot), so the stage streams exactly the
    // rows' bytes
    constexpr uint32_t PB = EB == 8 ? 16u : 12u;         // bytes per piece
    const int lrow = lane >> 3, lslot = lane & 7;
    uint32_t ga[4], gw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (8 * i + wave) * 8 + lrow;
        const int gr = m0 + row < M ? m0 + row : M - 1;
        ga[i] = (uint32_t)gr * KB + (uint32_t)(lslot ^ swz(row)) * PB;
        const int wr = row < TBN ? row : TBN - 1;
        const int gn = n0 + wr < N ? n0 + wr : N - 1;
        gw[i] = (uint32_t)gn * KB + (uint32_t)(lslot ^ swz(wr)) * PB;
    }
    // scale dword of tile row d = 64 wave + lane (A rows, then W rows; d >= 480 repeats row 479)
    uint32_t gs;
    bool s_is_a;
    {
        const int d = 64 * wave + lane < TBM + TBN ? 64 * wave + lane : TBM + TBN - 1;
        s_is_a = d < TBM;
        if (s_is_a) {
            const int gr = m0 + d < M ? m0 + d : M - 1;
            gs = (uint32_t)gr * KS;
        } else {
            const int gn = n0 + (d - TBM) < N ? n0 + (d - TBM) : N - 1;
            gs = (uint32_t)gn * KS;
        }
    }
    const __amdgpu_buffer_rsrc_t ra = brsrc(A), rw = brsrc(W), rsa = brsrc(sA), rsw = brsrc(sW);
    auto dload = [&](int buf, int kt) {
        int8_t* base = lds + buf * MX8_STAGE;
        const uint32_t k0 = (uint32_t)kt * RB;
#pragma unroll
        for (int i = 0; i < 4; i++) bload_lds(ra, base + (8 * i + wave) * 1024, PB, ga[i], k0);
#pragma unroll
        for (int i = 0; i < 3; i++) bload_lds(rw, base + TLDS_A + (8 * i + wave) * 1024, PB, gw[i], k0);
        if (wave < 4) bload_lds(rw, base + TLDS_A + (24 + wave) * 1024, PB, gw[3], k0);
        // wave-uniform operand choice (waves 0-3 hold A rows, 4-7 W rows)
        if (wave < 4)
            bload_lds(rsa, base + TLDS_STAGE + wave * 256, 4, gs, 4u * (uint32_t)kt);
        else
            bload_lds(rsw, base + TLDS_STAGE + wave * 256, 4, gs, 4u * (uint32_t)kt);
    };

    f32x4 acc[FM][TFN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < TFN; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int sw = swz(r16);
    const int8_t* arow = lds + (wm * 64 + r16) * TBK;
    const int8_t* wrow = lds + TLDS_A + (wn * 112 + r16) * TBK;
    const int8_t* srow_a = lds + TLDS_STAGE + (wm * 64 + r16) * 4 + q;
    const int8_t* srow_w = lds + TLDS_STAGE + (TBM + wn * 112 + r16) * 4 + q;
    const int nk = K / 128;

    // lane group q's operand: fp8 chunks q and q + 4 of the row; fp6 block q
    // (bytes [24 q, 24 q + 24) of the row = its pieces 2 q and 2 q + 1)
    auto frag = [&](const int8_t* row) -> i32x8 {
        if (EB == 8) {
            const i32x4 lo = lds16(row + ((q ^ sw) << 4));
            const i32x4 hi = lds16(row + (((q + 4) ^ sw) << 4));
            return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        } else {
            typedef int i32x3 __attribute__((ext_vector_type(3)));
            const i32x3 lo = *reinterpret_cast<const i32x3*>(row + (((2 * q) ^ sw) << 4));
            const i32x3 hi = *reinterpret_cast<const i32x3*>(row + (((2 * q + 1) ^ sw) << 4));
            return i32x8{lo[0], lo[1], lo[2], hi[0], hi[1], hi[2], 0, 0};
        }
    };

    dload(0, 0);
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        __builtin_amdgcn_s_waitcnt(0x0070);   // this stage landed; earlier LDS reads done
        __syncthreads();
        dload(cur ^ 1, kt + 1 < nk ? kt + 1 : 0);   // last stage: stage 0 again, unused
        const int8_t* ab = arow + cur * MX8_STAGE;
        const int8_t* wb = wrow + cur * MX8_STAGE;
        i32x8 fa[FM], fw[TFN];
        int sca[FM], scw[TFN];
#pragma unroll
        for (int i = 0; i < FM; i++) {
            fa[i] = frag(ab + i * 16 * TBK);
            sca[i] = e8m0_of(srow_a[cur * MX8_STAGE + i * 16 * 4]);
        }
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            fw[j] = frag(wb + j * 16 * TBK);
            scw[j] = e8m0_of(srow_w[cur * MX8_STAGE + j * 16 * 4]);
        }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < TFN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                    fa[i], fw[j], acc[i][j], MF, MF, 0, sca[i], 0, scw[j]);
    }
    __builtin_amdgcn_s_waitcnt(0x0070);   // the last (unused) loads drain before exit

#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            const int n = n0 + wn * 112 + j * 16 + r16;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = m0 + wm * 64 + i * 16 + q * 4 + e;
                if (m >= M) continue;
                if (YF32)
                    reinterpret_cast<float*>(out)[(size_t)m * N + n] = acc[i][j][e];
                else
                    reinterpret_cast<uint16_t*>(out)[(size_t)m * N + n] = bf16_out(acc[i][j][e]);
            }
        }
    }
}

template <int MF, int EB, bool YF32>
int launch_mx8_tiled(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                     void* out, int M, int N, int K, hipStream_t st) {
    const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
    const size_t lds = 2 * (size_t)MX8_STAGE;
    static std::atomic<uint64_t> lds_done{0};   // > 64 KB of LDS per workgroup, per device
    const void* kfn = reinterpret_cast<const void*>(&k_mx8_tiled<MF, EB, YF32>);
    if (snx::lds_optin(kfn, (int)lds, lds_done) != hipSuccess) {
        snx_set_error("mx gemm: cannot reserve %zu bytes of LDS", lds);
        return -1;
    }
    k_mx8_tiled<MF, EB, YF32><<<tiles_m * tiles_n, 512, lds, st>>>(A, sA, W, sW, out, M, N, K, tiles_m,
                                                                    tiles_n);
    return snx_launch_check("k_mx8_tiled");
}

template <bool YF32, int SG>
int launch_mxfp4_tiled(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                       void* out, int M, int N, int K, hipStream_t st) {
    const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
    const size_t lds = SG == 1 ? 2 * (size_t)MXS_STAGE
                               : 2 * (size_t)TLDS_STAGE + (SG == 4 ? 2 * MXG_HALF : 0);
    static std::atomic<uint64_t> lds_done{0};   // > 64 KB of LDS per workgroup, per device
    const void* kfn = reinterpret_cast<const void*>(&k_mxfp4_tiled<YF32, SG>);
    if (snx::lds_optin(kfn, (int)lds, lds_done) != hipSuccess) {
        snx_set_error("mxfp4 gemm: cannot reserve %zu bytes of LDS", lds);
        return -1;
    }
    k_mxfp4_tiled<YF32, SG><<<tiles_m * tiles_n, 512, lds, st>>>(A, sA, W, sW, out, M, N, K, tiles_m, tiles_n);
    return snx_launch_check("k_mxfp4_tiled");
}

// int8 on the 32x32 shape: same tile, LDS layout and direct loads as
// k_gemm_8w, but the 8 waves split the tile along M only (wave w owns rows
// [32 w, +32) and all 224 columns = 7 blocks of 32x32), so a stage issues
// 28 v_mfma_i32_32x32x32_i8 per wave -- half the instructions of the 16x16
// shape for the same work.  Operand lane l: row (A) / column (W) l % 32,
// k-bytes [16 (l/32), +16) of each 32-byte k-step.
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
constexpr int XCROW = 232;   // u16 per staged output row: 224 + 8 pad
static_assert(8 * 32 * XCROW * 2 <= 2 * TLDS_STAGE, "output staging fits in the LDS ring");

template <bool FP8, bool RAW, bool BIAS>
__global__ void __launch_bounds__(512) k_gemm_x32(const int8_t* __restrict__ A,
                                                    const int8_t* __restrict__ W,
                                                    const float* __restrict__ sA,
                                                    const float* __restrict__ sW,
                                                    int32_t* __restrict__ Craw,
                                                    uint16_t* __restrict__ out,
                                                    const float* __restrict__ bias, int M, int N,
                                                    int K, int tiles_m, int tiles_n) {
    constexpr int FN = TBN / 32;                 // 7 blocks per wave
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r32 = lane & 31, h = lane >> 5;

    const int b = blockIdx.x, nb = gridDim.x;
    const int tile = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int m0 = tm * TBM, n0 = tn * TBN;

    const int lrow = lane >> 3, lslot = lane & 7;
    uint32_t ga[4], gw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (8 * i + wave) * 8 + lrow;
        const int gr = m0 + row < M ? m0 + row : M - 1;
        ga[i] = (uint32_t)gr * (uint32_t)K + (uint32_t)((lslot ^ swz(row)) * 16);
        const int wr = row < TBN ? row : TBN - 1;
        const int gn = n0 + wr < N ? n0 + wr : N - 1;
        gw[i] = (uint32_t)gn * (uint32_t)K + (uint32_t)((lslot ^ swz(wr)) * 16);
    }
    const __amdgpu_buffer_rsrc_t ra = brsrc(A), rw = brsrc(W);
    auto dload = [&](int buf, int k0) {
        int8_t* base = lds + buf * TLDS_STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++) bload_lds(ra, base + (8 * i + wave) * 1024, 16, ga[i], k0);
#pragma unroll
        for (int i = 0; i < 3; i++) bload_lds(rw, base + TLDS_A + (8 * i + wave) * 1024, 16, gw[i], k0);
        if (wave < 4) bload_lds(rw, base + TLDS_A + (24 + wave) * 1024, 16, gw[3], k0);
    };

    typedef typename std::conditional<FP8, f32x16, i32x16>::type acc_t;
    acc_t acc[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) acc[j] = acc_t{};

    const int sw = swz(r32);
    const int8_t* arow = lds + (wave * 32 + r32) * TBK;
    const int8_t* wrow = lds + TLDS_A + r32 * TBK;
    const int nk = K / TBK;

    dload(0, 0);
    float sa[16], swv[FN], bv[FN];
    if (!RAW) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = m0 + wave * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            sa[v] = FP8 ? sA[0] : sA[m < M ? m : M - 1];
        }
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = n0 + j * 32 + r32;
            swv[j] = FP8 ? sW[0] : sW[n < N ? n : N - 1];
            bv[j] = BIAS ? bias[n < N ? n : N - 1] : 0.0f;
        }
    }
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        __builtin_amdgcn_s_waitcnt(0x0070);   // this stage landed; earlier LDS reads done
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        dload(cur ^ 1, kt + 1 < nk ? (kt + 1) * TBK : 0);
        const int8_t* ab = arow + cur * TLDS_STAGE;
        const int8_t* wb = wrow + cur * TLDS_STAGE;
        if (!FP8) {
#pragma unroll
            for (int s = 0; s < 4; s++) {          // k-steps of 32 bytes: chunk 2 s + h
                const int off = ((2 * s + h) ^ sw) << 4;
                const i32x4 fa = lds16(ab + off);
                i32x4 fw[FN];
#pragma unroll
                for (int j = 0; j < FN; j++) fw[j] = lds16(wb + j * 32 * TBK + off);
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[j] = (acc_t)__builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fw[j], (i32x16)acc[j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int s = 0; s < 2; s++) {          // k-steps of 64 bytes: chunks 4 s + 2 h, +1
                const int o0 = ((4 * s + 2 * h) ^ sw) << 4, o1 = ((4 * s + 2 * h + 1) ^ sw) << 4;
                const i32x4 alo = lds16(ab + o0), ahi = lds16(ab + o1);
                const i32x8 fa = i32x8{alo[0], alo[1], alo[2], alo[3], ahi[0], ahi[1], ahi[2], ahi[3]};
                i32x8 fw[FN];
#pragma unroll
                for (int j = 0; j < FN; j++) {
                    const i32x4 lo = lds16(wb + j * 32 * TBK + o0), hi = lds16(wb + j * 32 * TBK + o1);
                    fw[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[j] = (acc_t)__builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fa, fw[j], (f32x16)acc[j], 0, 0, 0, 0, 0, 0);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070);   // the last (unused) loads drain before exit

    if (RAW) {   // int32 accumulators (bit-exactness checks): direct stores
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = n0 + j * 32 + r32;
            if (n >= N) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {    // 32x32 C layout: row 8 (v/4) + 4 (l/32) + v%4
                const int m = m0 + wave * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m < M) Craw[(size_t)m * N + n] = ((i32x16)acc[j])[v];
            }
        }
        return;
    }
    // bf16 tile through LDS: each wave writes its 32 x 224 block row-major
    // (rows padded to 464 B: the two lane halves, 4 rows apart, use different
    // banks), then stores 16-byte pieces, 448 contiguous bytes per row.
    __syncthreads();                      // every wave is done with the ring
    uint16_t* ct = reinterpret_cast<uint16_t*>(lds) + wave * (32 * XCROW);
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
        for (int v = 0; v < 16; v++)
            ct[(8 * (v >> 2) + 4 * h + (v & 3)) * XCROW + j * 32 + r32] =
                BIAS ? bf16_out((float)acc[j][v] * sa[v] * swv[j] + bv[j])
                     : bf16_out((float)acc[j][v] * sa[v] * swv[j]);
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
#pragma unroll
    for (int t = 0; t < 14; t++) {        // 32 rows x 28 pieces = 896 = 14 x 64
        const int qd = t * 64 + lane;
        const int row = qd / 28, c = qd - row * 28;
        const int m = m0 + wave * 32 + row, n = n0 + c * 8;
        if (m >= M || n >= N) continue;
        const i32x4 val = *reinterpret_cast<const i32x4*>(ct + row * XCROW + c * 8);
        uint16_t* dst = out + (size_t)m * N + n;
        if (vec && n + 8 <= N) {
            *reinterpret_cast<i32x4*>(dst) = val;
        } else {
            const uint16_t* e = reinterpret_cast<const uint16_t*>(&val);
            for (int i = 0; i < 8 && n + i < N; i++) dst[i] = e[i];
        }
    }
}

constexpr uint32_t BUF_DROP = 0x7ffffff0u;   // store offset outside every output buffer

// Persistent form of k_gemm_8w (the C4 kernel for int8 and fp8 e4m3): the
// same 256 x 224 tile, 4 (M) x 2 (N) waves of 64 x 112 in 16 x 16 MFMA
// blocks, LDS ring, swizzle and fragment reads, with
//  * one workgroup per CU walking tiles b, b + nb, ... (nb a multiple of 8:
//    every tile of a workgroup stays on its XCD);
//  * each k-step's wait and barrier at its end, after its MFMAs, so the last
//    k-step of a tile loads the next tile's stage 0 and the next tile starts
//    computing at once;
//  * an epilogue that stages each wave's bf16 rows through its own slice of
//    the buffer the last k-step freed (two passes of 32 rows x 112 columns)
//    and writes 224-byte row pieces with 16-byte buffer stores (rows or
//    columns outside the matrix get an out-of-range offset and are dropped),
//    so tile i's output drains while tile i + 1 computes.  A wave reads back
//    only what it wrote, so no barrier sits between staging and stores.
// Requires N % 8 == 0 (a 16-byte piece never straddles a row end), a 16-byte
// aligned output below 2 GiB and operands below 2 GiB.
// SPLIT > 1 (shapes with too few tiles to fill the CUs, such as one GPU's
// column shard of a tensor-parallel layer): a work unit is (tile, K span s)
// with spans of K / SPLIT; unit v covers tile v % ntiles, span v / ntiles.
// After its K loop each wave stores its accumulators to its slot of `part`
// (lane-major, 1 KB per store instruction) with the system-coherent cache
// policy (written through the XCD's L2), waits until they are written, and
// counts itself in cnt[tile][wave].  The wave that arrives last adds the
// SPLIT slots of its (tile, wave) in span order (0, 1, ...: the same fp32
// sums whichever wave is last), returns the counter to 0 for the next call
// and runs the epilogue; the others skip it.  The last wave reads the slots
// with the same policy, so no copy an L2 holds is used, and no fence has to
// write back or drop whole caches.  No wave waits for another, so
// the result does not depend on which units are resident together.
constexpr int PCROW = 120;             // u16 per staged output row of a wave: 112 + 8 pad
constexpr int kSysCoherent = 1 | 16;   // buffer cache policy sc0 sc1: system-coherent access
static_assert(8 * 32 * PCROW * 2 <= TLDS_STAGE, "a pass of every wave fits in one stage buffer");
// A tile's int8 row / column scales and its bias wait in LDS beside the ring
// (256 floats each, loaded straight from global memory when the tile starts)
// instead of in registers across the K loop.
constexpr int PSCALES = 2 * TLDS_STAGE;
constexpr int PLDS = PSCALES + 3 * 256 * 4;

template <bool FP8, bool RAW, bool BIAS, int SPLIT = 1>
__global__ void __launch_bounds__(512) k_gemm_8wp(const int8_t* __restrict__ A,
                                                  const int8_t* __restrict__ W,
                                                  const float* __restrict__ sA,
                                                  const float* __restrict__ sW,
                                                  int32_t* __restrict__ Craw,
                                                  uint16_t* __restrict__ out,
                                                  const float* __restrict__ bias, int M, int N,
                                                  int K, int tiles_m, int tiles_n,
                                                  i32x4* __restrict__ part, uint32_t* __restrict__ cnt) {
    constexpr int FM = 4;
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int r16 = lane & 15, q = lane >> 4;
    const int b = blockIdx.x, nb = gridDim.x;
    const int ntiles = tiles_m * tiles_n, nunits = ntiles * SPLIT;
    const int lrow = lane >> 3, lslot = lane & 7;
    // unit of walk position t (each XCD a compact block of units), its tile and K span
    auto unit_of = [&](int t) { return (nunits % 8 == 0) ? (t % 8) * (nunits / 8) + t / 8 : t; };
    auto tile_of = [&](int t) { return SPLIT == 1 ? unit_of(t) : unit_of(t) % ntiles; };
    auto addr = [&](int t, uint32_t* ga, uint32_t* gw) {
        const int tl = tile_of(t);
        const int m0 = (tl % tiles_m) * TBM, n0 = (tl / tiles_m) * TBN;
        const uint32_t kb = SPLIT == 1 ? 0u : (uint32_t)(unit_of(t) / ntiles) * (uint32_t)(K / SPLIT);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = (8 * i + wave) * 8 + lrow;
            const int gr = m0 + row < M ? m0 + row : M - 1;
            ga[i] = (uint32_t)gr * (uint32_t)K + kb + (uint32_t)((lslot ^ swz(row)) * 16);
            const int wr = row < TBN ? row : TBN - 1;
            const int gn = n0 + wr < N ? n0 + wr : N - 1;
            gw[i] = (uint32_t)gn * (uint32_t)K + kb + (uint32_t)((lslot ^ swz(wr)) * 16);
        }
    };
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, M * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, N * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc((void*)out, (short)0, BUF_DROP, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc((void*)sA, (short)0, FP8 ? 4 : M * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsw = __builtin_amdgcn_make_buffer_rsrc((void*)sW, (short)0, FP8 ? 4 : N * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rbi = __builtin_amdgcn_make_buffer_rsrc((void*)bias, (short)0, BIAS ? N * 4 : 0, 0x00020000);
    auto dload = [&](int buf, const uint32_t* ga, const uint32_t* gw, int k0) {
        int8_t* base = lds + buf * TLDS_STAGE;
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(base + (8 * i + wave) * 1024), 16, ga[i], k0, 0, 0);
#pragma unroll
        for (int i = 0; i < 3; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(base + TLDS_A + (8 * i + wave) * 1024), 16, gw[i], k0, 0, 0);
        if (wave < 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(base + TLDS_A + (24 + wave) * 1024), 16, gw[3], k0, 0, 0);
    };
    typedef typename std::conditional<FP8, f32x4, i32x4>::type acc_t;
    acc_t acc[FM][TFN];
    const int sw = swz(r16);
    const int8_t* arow = lds + (wm * 64 + r16) * TBK;
    const int8_t* wrow = lds + TLDS_A + (wn * 112 + r16) * TBK;
    const int nk = K / SPLIT / TBK;

    // int8: each k-step is two halves h (the even / odd 16-byte chunks, the
    // same bank pattern as the fp8 reads; any k order works as long as A and
    // W agree).  The second half's fragments are read while the first half's
    // MFMAs run, and the next k-step's first half right after the barrier,
    // while this k-step's second half runs.
    i32x4 h0a[FM], h0w[TFN], h1a[FM], h1w[TFN];
    auto rdh = [&](i32x4* fa, i32x4* fw, int bufi, int h) {
        const int off = bufi * TLDS_STAGE + (((2 * q + h) ^ sw) << 4);
#pragma unroll
        for (int i = 0; i < FM; i++) fa[i] = lds16(arow + off + i * 16 * TBK);
#pragma unroll
        for (int j = 0; j < TFN; j++) fw[j] = lds16(wrow + off + j * 16 * TBK);
    };
    auto mmh = [&](const i32x4* fa, const i32x4* fw) {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < TFN; j++)
                acc[i][j] = (acc_t)__builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fw[j], (i32x4)acc[i][j], 0, 0, 0);
    };

    int t = b;
    if (t >= nunits) return;
    const float sa8 = FP8 ? sA[0] : 0.0f, sw8 = FP8 ? sW[0] : 0.0f;   // fp8: per-tensor scales
    uint32_t ga[4], gw[4];
    addr(t, ga, gw);
    dload(0, ga, gw, 0);
    __builtin_amdgcn_s_waitcnt(0x0070);        // vmcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    int buf = 0;
    if (!FP8) rdh(h0a, h0w, 0, 0);
    for (;;) {
        const int tl = tile_of(t);
        const int m0 = (tl % tiles_m) * TBM, n0 = (tl / tiles_m) * TBN;
        const int tnext = t + nb;
        const bool has_next = tnext < nunits;
        // this tile's scales / bias into LDS (landed by the first k-step's wait)
        {
            const int e = 64 * (wave & 3) + lane;
            if (!FP8 && !RAW && wave < 4) {
                const int m = m0 + e < M ? m0 + e : M - 1;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsa, (lds_ptr_t)(lds + PSCALES + 256 * wave), 4,
                                                         (uint32_t)m * 4u, 0, 0, 0);
            }
            const int n = n0 + e < N ? n0 + e : N - 1;
            if (!FP8 && !RAW && wave >= 4)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_ptr_t)(lds + PSCALES + 1024 + 256 * (wave - 4)), 4,
                                                         (uint32_t)n * 4u, 0, 0, 0);
            if (BIAS && wave < 4)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rbi, (lds_ptr_t)(lds + PSCALES + 2048 + 256 * wave), 4,
                                                         (uint32_t)n * 4u, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < TFN; j++) acc[i][j] = acc_t{0, 0, 0, 0};
        for (int kt = 0; kt < nk; kt++) {
            const int cur = buf;
            if (kt + 1 < nk) {
                dload(cur ^ 1, ga, gw, (kt + 1) * TBK);
            } else {       // the next tile's stage 0 (this tile's again if there is none)
                if (has_next) addr(tnext, ga, gw);
                dload(cur ^ 1, ga, gw, 0);
            }
            if (!FP8) {
                rdh(h1a, h1w, cur, 1);
                mmh(h0a, h0w);
                // the next stage landed and every wave's reads of this one are done
                __builtin_amdgcn_s_waitcnt(0x0070);
                __builtin_amdgcn_s_barrier();
                rdh(h0a, h0w, cur ^ 1, 0);
                mmh(h1a, h1w);
            } else {
                const int8_t* ab = arow + cur * TLDS_STAGE;
                const int8_t* wb = wrow + cur * TLDS_STAGE;
                // lane group q takes 16-byte chunks q and q + 4 of the row (the
                // k order of the 8-bit operands of the f8f6f4 instruction)
                i32x8 fa[FM], fw[TFN];
#pragma unroll
                for (int i = 0; i < FM; i++) {
                    const i32x4 lo = lds16(ab + i * 16 * TBK + (((2 * q) ^ sw) << 4));
                    const i32x4 hi = lds16(ab + i * 16 * TBK + (((2 * q + 1) ^ sw) << 4));
                    fa[i] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int j = 0; j < TFN; j++) {
                    const i32x4 lo = lds16(wb + j * 16 * TBK + (((2 * q) ^ sw) << 4));
                    const i32x4 hi = lds16(wb + j * 16 * TBK + (((2 * q + 1) ^ sw) << 4));
                    fw[j] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < TFN; j++)
                        acc[i][j] = (acc_t)__builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                            fa[i], fw[j], (f32x4)acc[i][j], 0, 0, 0, 0, 0, 0);
                // the next stage landed and every wave's reads of this one are done
                __builtin_amdgcn_s_waitcnt(0x0070);
                __builtin_amdgcn_s_barrier();
            }
            buf = cur ^ 1;
        }
        // buffer buf holds the next tile's stage 0; buffer buf ^ 1 is free
        bool last = true;
        if (SPLIT > 1) {
            // slot (unit, wave): FM x TFN x 64 lanes x 16 B, lane-major; buffer
            // accesses with the wave-uniform part of the address in soffset
            constexpr int SLOTB = FM * TFN * 64 * 16;
            const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
                (void*)part, (short)0, nunits * 8 * SLOTB, 0x00020000);
            const int sp = unit_of(t) / ntiles;
            const uint32_t mine = (uint32_t)((sp * ntiles + tl) * 8 + wave) * SLOTB;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < TFN; j++)
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, acc[i][j]), rp, lane * 16,
                                                           mine + (i * TFN + j) * 1024, kSysCoherent);
            // the slot is written before it is counted; and nothing may write
            // the accumulator registers before the stores have read them (a
            // 16-byte store reads its data after issue): the scheduler may not
            // move the next instructions above this wait
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_waitcnt(0x0f70);           // vmcnt(0)
            __builtin_amdgcn_sched_barrier(0);
            uint32_t c = 0;
            if (lane == 0) c = atomicAdd(&cnt[tl * 8 + wave], 1u);
            last = __builtin_amdgcn_readfirstlane(c) == SPLIT - 1;
            if (last) {
                const uint32_t first = (uint32_t)(tl * 8 + wave) * SLOTB, sstride = (uint32_t)ntiles * 8 * SLOTB;
                // in chunks of 4 fragments x SPLIT spans: the loads of a chunk in
                // flight together, and each chunk's offsets carry a zero that the
                // previous chunk's sums produce (an opaque dependency), so that
                // the compiler cannot hoist every load and spill the sums
                constexpr int JC = 4;
                uint32_t dep = 0;
#pragma unroll
                for (int i = 0; i < FM; i++) {
#pragma unroll
                    for (int j0 = 0; j0 < TFN; j0 += JC) {
                        i32x4 v[SPLIT][JC];
#pragma unroll
                        for (int s2 = 0; s2 < SPLIT; s2++)
#pragma unroll
                            for (int jj = 0; jj < JC; jj++)
                                if (j0 + jj < TFN)
                                    v[s2][jj] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                        rp, lane * 16, first + dep + s2 * sstride + (i * TFN + j0 + jj) * 1024,
                                        kSysCoherent));
#pragma unroll
                        for (int jj = 0; jj < JC; jj++) {
                            if (j0 + jj >= TFN) break;
                            acc_t r = __builtin_bit_cast(acc_t, v[0][jj]);
#pragma unroll
                            for (int s2 = 1; s2 < SPLIT; s2++) r += __builtin_bit_cast(acc_t, v[s2][jj]);
                            acc[i][j0 + jj] = r;
                        }
                        if (j0 + JC <= TFN)
                            asm volatile("s_mov_b32 %0, 0"
                                         : "=s"(dep)
                                         : "v"(acc[i][j0]), "v"(acc[i][j0 + 1]), "v"(acc[i][j0 + 2]),
                                           "v"(acc[i][j0 + 3]));
                        else
                            asm volatile("s_mov_b32 %0, 0"
                                         : "=s"(dep)
                                         : "v"(acc[i][j0]), "v"(acc[i][j0 + 1 < TFN ? j0 + 1 : j0]),
                                           "v"(acc[i][j0 + 2 < TFN ? j0 + 2 : j0]));
                    }
                }
                if (lane == 0) atomicExch(&cnt[tl * 8 + wave], 0u);   // ready for the next call
            }
        }
        if (RAW) {   // int32 accumulators (bit-exactness checks): direct stores
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < TFN; j++) {
                    const int n = n0 + wn * 112 + j * 16 + r16;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int m = m0 + wm * 64 + i * 16 + q * 4 + e;
                        if (last && m < M && n < N) Craw[(size_t)m * N + n] = ((i32x4)acc[i][j])[e];
                    }
                }
            if (!has_next) break;
            t = tnext;
            continue;
        }
        uint16_t* ct = reinterpret_cast<uint16_t*>(lds + (buf ^ 1) * TLDS_STAGE) + wave * (32 * PCROW);
        const float* lsc = reinterpret_cast<const float*>(lds + PSCALES);
        float swv[TFN], bv[TFN];
#pragma unroll
        for (int j = 0; j < TFN; j++) {
            const int c = wn * 112 + j * 16 + r16;
            swv[j] = FP8 ? sw8 : lsc[256 + c];
            bv[j] = BIAS ? lsc[512 + c] : 0.0f;
        }
#pragma unroll
        for (int p = 0; p < 2; p++) {         // fragment rows 2p, 2p + 1: wave rows 32 p .. 32 p + 31
            if (!last) break;
#pragma unroll
            for (int i = 2 * p; i < 2 * p + 2; i++) {
                const f32x4 sa = FP8 ? f32x4{sa8, sa8, sa8, sa8}
                                     : *reinterpret_cast<const f32x4*>(lsc + wm * 64 + i * 16 + q * 4);
#pragma unroll
                for (int j = 0; j < TFN; j++)
#pragma unroll
                    for (int e = 0; e < 4; e += 2) {   // rows e, e + 1 in one conversion
                        float v0 = (float)acc[i][j][e] * sa[e] * swv[j];
                        float v1 = (float)acc[i][j][e + 1] * sa[e + 1] * swv[j];
                        if (BIAS) v0 += bv[j], v1 += bv[j];
                        const uint32_t pk = bf16x2_out(v0, v1);
                        uint16_t* c0 = ct + ((i - 2 * p) * 16 + q * 4 + e) * PCROW + j * 16 + r16;
                        c0[0] = (uint16_t)pk;
                        c0[PCROW] = (uint16_t)(pk >> 16);
                    }
            }
#pragma unroll
            for (int c = 0; c < 7; c++) {     // 32 rows x 14 pieces of 16 B = 7 x 64
                const int qd = c * 64 + lane;
                const int row = qd / 14, pc = qd - row * 14;
                const int m = m0 + wm * 64 + 32 * p + row, n = n0 + wn * 112 + pc * 8;
                const i32x4 val = *reinterpret_cast<const i32x4*>(ct + row * PCROW + pc * 8);
                const uint32_t off = (m < M && n < N) ? ((uint32_t)m * (uint32_t)N + (uint32_t)n) * 2u : BUF_DROP;
                __builtin_amdgcn_raw_buffer_store_b128(val, ro, off, 0, 0);
            }
        }
        // staging reads done (lgkmcnt(0)) before the next tile loads into this buffer
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_s_barrier();
        if (!has_next) break;
        t = tnext;
    }
    __builtin_amdgcn_s_waitcnt(0x0070);       // the spare stage-0 loads land before exit
}

// K spans of the persistent kernel for M x N x K: 2 when the tiles fill at
// most a quarter of the one-workgroup-per-CU grid and K splits into whole
// 128-byte stages, else 1.  Measured (fp8, K = 4096, 256 CUs): 10, 32 and 64
// tiles run 17-22 % faster in two spans; 128 tiles run 10 % slower, the
// partials' traffic costing more than the CUs the spans bring in; four spans
// were slower than two at 64 tiles (the last wave of a (tile, wave) reads
// three 28 KB partial slots in round trips of one 16-load chunk).
int w8a8_splits(int M, int N, int K) {
    const int ntiles = ((M + TBM - 1) / TBM) * ((N + TBN - 1) / TBN);
    const int ncu = snx::cu_count();
    const int grid = ncu >= 8 ? ncu - ncu % 8 : ncu;
    if (ntiles * 4 <= grid && K % (2 * TBK) == 0) return 2;
    return 1;
}

template <bool FP8, bool RAW, bool BIAS, int SPLIT>
int launch_8wp_s(const int8_t* A, const int8_t* W, const float* sA, const float* sW, int32_t* Craw,
                 uint16_t* out, const float* bias, int M, int N, int K, int tiles_m, int tiles_n, int grid,
                 i32x4* part, uint32_t* cnt, hipStream_t st) {
    const size_t lds = PLDS;
    static std::atomic<uint64_t> lds_done{0};   // > 64 KB of LDS per workgroup, per device
    const void* kfn = reinterpret_cast<const void*>(&k_gemm_8wp<FP8, RAW, BIAS, SPLIT>);
    if (snx::lds_optin(kfn, (int)lds, lds_done) != hipSuccess) {
        snx_set_error("gemm: cannot reserve %zu bytes of LDS", lds);
        return -1;
    }
    k_gemm_8wp<FP8, RAW, BIAS, SPLIT><<<grid, 512, lds, st>>>(A, W, sA, sW, Craw, out, bias, M, N, K, tiles_m,
                                                              tiles_n, part, cnt);
    return snx_launch_check("k_gemm_8wp");
}

template <bool FP8, bool RAW, bool BIAS>
int launch_8wp(const int8_t* A, const int8_t* W, const float* sA, const float* sW, int32_t* Craw,
               uint16_t* out, const float* bias, int M, int N, int K, hipStream_t st) {
    const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
    const int ntiles = tiles_m * tiles_n;
    const int ncu = snx::cu_count();
    const int split = w8a8_splits(M, N, K);
    // one workgroup per CU (rounded down to a multiple of 8: units keep their XCD)
    int grid = ncu >= 8 ? ncu - ncu % 8 : ncu;
    if (grid > ntiles * split) grid = ntiles * split;
    if (split == 1)
        return launch_8wp_s<FP8, RAW, BIAS, 1>(A, W, sA, sW, Craw, out, bias, M, N, K, tiles_m, tiles_n, grid,
                                              nullptr, nullptr, st);
    // the span partials (one 229,376-byte slot per unit and wave group) and
    // the arrival counters of the (tile, wave) pairs, which the kernel leaves at 0
    const size_t slots = (size_t)ntiles * split * 8 * (4 * TFN * 64);
    i32x4* part = static_cast<i32x4*>(snx_workspace(slots * sizeof(i32x4), 3, st));
    uint32_t* cnt = static_cast<uint32_t*>(snx_workspace_zeroed((size_t)ntiles * 8 * sizeof(uint32_t), 4, st));
    if (!part || !cnt) return -1;
    return launch_8wp_s<FP8, RAW, BIAS, 2>(A, W, sA, sW, Craw, out, bias, M, N, K, tiles_m, tiles_n, grid, part,
                                          cnt, st);
}

template <bool FP8, bool RAW, bool BIAS>
int launch_x32(const int8_t* A, const int8_t* W, const float* sA, const float* sW,
                 int32_t* Craw, uint16_t* out, const float* bias, int M, int N, int K, hipStream_t st) {
    const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
    if ((uint64_t)M * K >= (1ull << 32) || (uint64_t)N * K >= (1ull << 32)) {
        snx_set_error("gemm: operands above 4 GiB are not supported");
        return -1;
    }
    const size_t lds = 2 * (size_t)TLDS_STAGE;
    static std::atomic<uint64_t> lds_done{0};   // > 64 KB of LDS per workgroup, per device
    const void* kfn = reinterpret_cast<const void*>(&k_gemm_x32<FP8, RAW, BIAS>);
    if (snx::lds_optin(kfn, (int)lds, lds_done) != hipSuccess) {
        snx_set_error("gemm: cannot reserve %zu bytes of LDS", lds);
        return -1;
    }
    k_gemm_x32<FP8, RAW, BIAS><<<tiles_m * tiles_n, 512, lds, st>>>(A, W, sA, sW, Craw, out, bias, M, N,
                                                              K, tiles_m, tiles_n);
    return snx_launch_check("k_gemm_x32");
}

template <bool FP8, bool RAW, bool BIAS>
int launch_tiled(const int8_t* A, const int8_t* W, const float* sA, const float* sW, int32_t* Craw,
                 uint16_t* out, const float* bias, int M, int N, int K, hipStream_t st) {
    const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
    if ((uint64_t)M * K >= (1ull << 32) || (uint64_t)N * K >= (1ull << 32)) {
        snx_set_error("gemm: operands above 4 GiB are not supported");
        return -1;
    }
    const size_t lds = 2 * (size_t)TLDS_STAGE;
    static std::atomic<uint64_t> lds_done{0};   // > 64 KB of LDS per workgroup, per device
    const void* kfn = reinterpret_cast<const void*>(&k_gemm_8w<FP8, RAW, BIAS>);
    if (snx::lds_optin(kfn, (int)lds, lds_done) != hipSuccess) {
        snx_set_error("gemm: cannot reserve %zu bytes of LDS", lds);
        return -1;
    }
    k_gemm_8w<FP8, RAW, BIAS><<<tiles_m * tiles_n, 512, lds, st>>>(A, W, sA, sW, Craw, out, bias, M, N,
                                                            K, tiles_m, tiles_n);
    return snx_launch_check("k_gemm_8w");
}

}  // namespace

extern "C" {

int snx_k_i8_gemm(const int8_t* A, const int8_t* W, const float* sA, const float* sW,
                  int32_t* c_i32, uint16_t* out_bf16, const float* bias, size_t M, size_t N,
                  size_t K, void* st) {
    if (K % 16 != 0) {
        snx_set_error("i8 gemm: K=%zu must be a multiple of 16", K);
        return -1;
    }
    if (K % TBK == 0 && M >= 128 && N >= 128) {
        // the persistent kernel addresses operands with 31-bit buffer offsets
        // and writes bf16 output in 16-byte row pieces
        const bool fits = (uint64_t)M * K < (1ull << 31) && (uint64_t)N * K < (1ull << 31);
        if (c_i32)
            return fits ? launch_8wp<false, true, false>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K, S(st))
                        : launch_x32<false, true, false>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K, S(st));
        if (fits && N % 8 == 0 && (reinterpret_cast<uintptr_t>(out_bf16) & 15) == 0 && (uint64_t)M * N * 2 < BUF_DROP)
            return bias ? launch_8wp<false, false, true>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K, S(st))
                        : launch_8wp<false, false, false>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K, S(st));
        return bias ? launch_x32<false, false, true>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K, S(st))
                    : launch_x32<false, false, false>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K, S(st));
    }
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (c_i32)
        k_i8_gemm<true><<<grid, 256, 0, S(st)>>>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K);
    else
        k_i8_gemm<false><<<grid, 256, 0, S(st)>>>(A, W, sA, sW, c_i32, out_bf16, bias, (int)M, (int)N, (int)K);
    return snx_launch_check("k_i8_gemm");
}

int snx_k_mxfp4_gemm_tiled(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                           void* out, int y_f32, size_t M, size_t N, size_t K, void* st) {
    if (K % 256 != 0 || (uint64_t)M * (K / 2) >= (1ull << 32) || (uint64_t)N * (K / 2) >= (1ull << 32)) {
        snx_set_error("mxfp4 gemm: tiled kernel needs K %% 256 == 0 and operands below 4 GiB");
        return -1;
    }
    if (K % 1024 == 0) {
        if (y_f32) return launch_mxfp4_tiled<true, 4>(A, sA, W, sW, out, (int)M, (int)N, (int)K, S(st));
        return launch_mxfp4_tiled<false, 4>(A, sA, W, sW, out, (int)M, (int)N, (int)K, S(st));
    }
    if (y_f32) return launch_mxfp4_tiled<true, 1>(A, sA, W, sW, out, (int)M, (int)N, (int)K, S(st));
    return launch_mxfp4_tiled<false, 1>(A, sA, W, sW, out, (int)M, (int)N, (int)K, S(st));
}

// the same kernel on E2M1 operands with one exponent each (sA[0], sW[0])
int snx_k_mxfp4_gemm_tiled_pt(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                              void* out, int y_f32, size_t M, size_t N, size_t K, void* st) {
    if (K % 256 != 0 || (uint64_t)M * (K / 2) >= (1ull << 32) || (uint64_t)N * (K / 2) >= (1ull << 32)) {
        snx_set_error("mxfp4 gemm: tiled kernel needs K %% 256 == 0 and operands below 4 GiB");
        return -1;
    }
    if (y_f32) return launch_mxfp4_tiled<true, 0>(A, sA, W, sW, out, (int)M, (int)N, (int)K, S(st));
    return launch_mxfp4_tiled<false, 0>(A, sA, W, sW, out, (int)M, (int)N, (int)K, S(st));
}

int snx_k_mx8_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                   void* out, int y_f32, int mf, size_t M, size_t N, size_t K, void* st) {
    const int eb = mf < 2 ? 8 : 6;
    if (K % 128 != 0 || (uint64_t)M * K * eb / 8 >= (1ull << 32) || (uint64_t)N * K * eb / 8 >= (1ull << 32)) {
        snx_set_error("mx gemm: K %% 128 == 0 and operands below 4 GiB are required");
        return -1;
    }
    const int m = (int)M, n = (int)N, k = (int)K;
#define SNX_MX8(F, B)                                                                       \
    return y_f32 ? launch_mx8_tiled<F, B, true>(A, sA, W, sW, out, m, n, k, S(st))          \
                 : launch_mx8_tiled<F, B, false>(A, sA, W, sW, out, m, n, k, S(st))
    switch (mf) {
        case 0: SNX_MX8(0, 8);
        case 1: SNX_MX8(1, 8);
        case 2: SNX_MX8(2, 6);
        default: SNX_MX8(3, 6);
    }
#undef SNX_MX8
}

int snx_k_fp8_gemm(const uint8_t* A, const uint8_t* W, const float* sA, const float* sW,
                   uint16_t* out_bf16, const float* bias, size_t M, size_t N, size_t K, void* st) {
    if (K % 32 != 0) {
        snx_set_error("fp8 gemm: K=%zu must be a multiple of 32", K);
        return -1;
    }
    if (K % TBK == 0 && M >= 128 && N >= 128) {
        const int8_t* a8 = reinterpret_cast<const int8_t*>(A);
        const int8_t* w8 = reinterpret_cast<const int8_t*>(W);
        if (N % 8 == 0 && (reinterpret_cast<uintptr_t>(out_bf16) & 15) == 0 && (uint64_t)M * N * 2 < BUF_DROP &&
            (uint64_t)M * K < (1ull << 31) && (uint64_t)N * K < (1ull << 31))
            return bias ? launch_8wp<true, false, true>(a8, w8, sA, sW, nullptr, out_bf16, bias, (int)M, (int)N, (int)K, S(st))
                        : launch_8wp<true, false, false>(a8, w8, sA, sW, nullptr, out_bf16, bias, (int)M, (int)N, (int)K, S(st));
        if (bias)
            return launch_tiled<true, false, true>(a8, w8, sA, sW, nullptr, out_bf16, bias, (int)M, (int)N,
                                                   (int)K, S(st));
        return launch_tiled<true, false, false>(a8, w8, sA, sW, nullptr, out_bf16, bias, (int)M, (int)N,
                                                (int)K, S(st));
    }
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    k_fp8_gemm<<<grid, 256, 0, S(st)>>>(A, W, sA, sW, out_bf16, bias, (int)M, (int)N, (int)K);
    return snx_launch_check("k_fp8_gemm");
}

}  // extern "C"
