// gemv_kernels.hip - decode GEMVs for gfx950 (HBM-bound).
//
//  * W8 weight-only (C1): int8 [N][K] x fp32 activations; 16-byte loads per
//    lane, bytes converted in registers, per-channel scale applied once.
//  * W4A16 (C2/C3/C5 decode): packed uint4 [N][K/8] x bf16 activations.
//    Nibbles become bf16 (128 + q) with one and-or per pair; the bias and
//    zero point come off exactly in fp32 and the fp16 group scale is applied
//    once per group.  M = 1 runs on the diagonal of
//    v_mfma_f32_4x4x4bf16_1k (k_w4a16_gemv1), larger M on
//    v_mfma_f32_16x16x32_bf16.
//  * A generic W4A16 kernel (any group size, any g_idx, any M) as fallback.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "codec.h"
#include "launch.h"
#include "../snx_internal.h"

using namespace snx;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Barrier for LDS hand-offs only: waits for this wave's LDS operations, not
// for its global loads (a __syncthreads() fence would drain those too).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}

__device__ __forceinline__ u32x4 load16(const void* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// Buffer loads: an offset at or past a buffer's record count returns zeros
// and touches no memory; kNontemporal is the cache policy of a nontemporal
// access (the "nt" bit).
constexpr uint32_t kNoRecord = 0x7ffffff0u;
constexpr int kNontemporal = 2;

// ----------------------------------------------------------------- W8 GEMV
// One wave per R rows; lane l covers bytes [16 l, 16 l + 16) of every
// 1024-column slice, so a wave load instruction reads 1 KB contiguous.
template <int R>
__global__ void __launch_bounds__(256) k_w8_gemv(const float* __restrict__ x,
                                                 const int8_t* __restrict__ q,
                                                 const float* __restrict__ s,
                                                 float* __restrict__ y,
                                                 const float* __restrict__ bias, int M, int N,
                                                 int K) {
    const int lane = threadIdx.x & 63;
    const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (n0 >= N) return;
    for (int m = 0; m < M; m++) {
        const float* xm = x + (size_t)m * K;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        for (int k = lane * 16; k < K; k += 1024) {
            float xv[16];
#pragma unroll
            for (int t = 0; t < 16; t += 4) {
                float4 v = *reinterpret_cast<const float4*>(xm + k + t);
                xv[t] = v.x; xv[t + 1] = v.y; xv[t + 2] = v.z; xv[t + 3] = v.w;
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                int n = n0 + r < N ? n0 + r : N - 1;
                u32x4 w = load16(q + (size_t)n * K + k);
#pragma unroll
                for (int t = 0; t < 16; t++) {
                    int b = (int)(int8_t)(w[t >> 2] >> (8 * (t & 3)));
                    acc[r] += xv[t] * (float)b;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = wave_sum(acc[r]);
            if (lane == 0 && n0 + r < N) {
                float o = s[n0 + r] * v;
                if (bias) o += bias[n0 + r];
                y[(size_t)m * N + n0 + r] = o;
            }
        }
    }
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_mv(float a) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, a), CTRL,
                                                                 ROW_MASK, 0xF, false));
}

// Full-wave sum with DPP moves (no LDS traffic); the total lands in lane 63.
__device__ __forceinline__ float dpp_sum_to_lane63(float v) {
    v += dpp_mv<0xB1, 0xF>(v);    // quad_perm [1,0,3,2]
    v += dpp_mv<0x4E, 0xF>(v);    // quad_perm [2,3,0,1]
    v += dpp_mv<0x141, 0xF>(v);   // row_half_mirror
    v += dpp_mv<0x140, 0xF>(v);   // row_mirror: every lane of a 16-lane row holds the row sum
    v += dpp_mv<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp_mv<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
    return v;
}

// M = 1, K = 1024 SL: a workgroup of 16 waves (one output row each) stages
// x (fp32) once in LDS; lane l of a wave loads bytes [16 l, +16) of every
// 1 KB slice of its row (nontemporal 16-byte loads, all SL in flight before
// the first FMA).  Bytes are read as unsigned (b ^ 0x80 = b + 128) with
// v_cvt_f32_ubyte*, and 128 * sum(x) comes off per 16-column slot:
// sum x*b = sum over slots of (sum x*(b + 128) - 128 * sum x), so the
// partial sums stay the size of the result even for activations far from
// zero mean.  The lane's 16 activations of a slot sit at
// (slice * 64 + lane) * 80 bytes, so the 16-byte LDS reads of a wave are free
// of bank conflicts; the slot's sum of x, computed once per workgroup at
// staging, sits in the 16 bytes of padding after them.
template <int SL>
__global__ void __launch_bounds__(1024) k_w8_gemv1(const float* __restrict__ x,
                                                   const int8_t* __restrict__ q,
                                                   const float* __restrict__ s,
                                                   float* __restrict__ y,
                                                   const float* __restrict__ bias, int N) {
    constexpr int K = 1024 * SL, NIT = K / 4, NTHR = 1024, XPT = (NIT + NTHR - 1) / NTHR;
    extern __shared__ __attribute__((aligned(16))) float xl[];   // [SL * 64][16 x + sum + pad]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * 16 + wave;
    const int n = n0 < N ? n0 : N - 1;

    float4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        int it = tid + i * NTHR;
        it = it < NIT ? it : NIT - 1;
        xr[i] = reinterpret_cast<const float4*>(x)[it];
    }
    // every wave's activation loads go out before any weight load of the
    // workgroup: a CU returns its loads in issue order
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    u32x4 w[SL];
#pragma unroll
    for (int sl = 0; sl < SL; sl++)
        w[sl] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(q + (size_t)n * K + sl * 1024 + lane * 16));
    asm volatile("" ::: "memory");
    // item it holds columns 4 it .. 4 it + 3 of slot it / 4; the four items
    // of a slot sit in four consecutive lanes (NTHR % 4 == 0)
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int it = tid + i * NTHR;
        float part = (xr[i].x + xr[i].y) + (xr[i].z + xr[i].w);
        part += dpp_mv<0xB1, 0xF>(part);   // quad_perm [1,0,3,2]
        part += dpp_mv<0x4E, 0xF>(part);   // quad_perm [2,3,0,1]
        if (it < NIT) {
            reinterpret_cast<float4*>(xl)[(it >> 2) * 5 + (it & 3)] = xr[i];
            if ((it & 3) == 0) xl[(it >> 2) * 20 + 16] = part;
        }
    }
    __syncthreads();

    float acc = 0.0f;
#pragma unroll
    for (int sl = 0; sl < SL; sl++) {
        float xv[16];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float4 v = reinterpret_cast<const float4*>(xl)[(sl * 64 + lane) * 5 + t];
            xv[4 * t] = v.x; xv[4 * t + 1] = v.y; xv[4 * t + 2] = v.z; xv[4 * t + 3] = v.w;
        }
        float a = -128.0f * xl[(sl * 64 + lane) * 20 + 16];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t u = w[sl][e] ^ 0x80808080u;
            // (float)(byte j of u) compiles to one v_cvt_f32_ubyte<j>
            a += xv[4 * e] * (float)(u & 0xFFu);
            a += xv[4 * e + 1] * (float)((u >> 8) & 0xFFu);
            a += xv[4 * e + 2] * (float)((u >> 16) & 0xFFu);
            a += xv[4 * e + 3] * (float)(u >> 24);
        }
        acc += a;
    }
    acc = dpp_sum_to_lane63(acc);
    if (lane == 63 && n0 < N) {
        float o = s[n0] * acc;
        if (bias) o += bias[n0];
        y[n0] = o;
    }
}

// Any K: one wave per row, scalar tail.
__global__ void __launch_bounds__(256) k_w8_gemv_any(const float* __restrict__ x,
                                                     const int8_t* __restrict__ q,
                                                     const float* __restrict__ s,
                                                     float* __restrict__ y,
                                                     const float* __restrict__ bias, int M, int N,
                                                     int K) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    for (int m = 0; m < M; m++) {
        float acc = 0.0f;
        for (int k = lane; k < K; k += 64) acc += x[(size_t)m * K + k] * (float)q[(size_t)n * K + k];
        acc = wave_sum(acc);
        if (lane == 0) y[(size_t)m * N + n] = bias ? s[n] * acc + bias[n] : s[n] * acc;
    }
}

// -------------------------------------------------------------- W4A16 GEMV
// Work: a workgroup owns 16 output columns n and all of K; its 4 waves take
// one quarter of K each and meet in LDS.  Per 128-column step a lane loads
// the 16 bytes (32 nibbles) of row n0 + lane%16 at column 32*(lane/16), which
// feed 4 MFMAs (one packed word each).  MFMA k-slot t of lane group g is
// column 32 g + 8 j + {0,4,1,5,2,6,3,7}[t] for MFMA j; the activations are
// permuted the same way with v_perm_b32, so A and B agree on every k.
template <int MT, bool ZEROS, bool YF32>
__global__ void __launch_bounds__(256) k_w4a16_gemv(const uint16_t* __restrict__ x,
                                                    const uint32_t* __restrict__ qw,
                                                    const uint16_t* __restrict__ scales,
                                                    const uint32_t* __restrict__ qz,
                                                    void* __restrict__ y,
                                                    const float* __restrict__ bias, int M, int N,
                                                    int K, int G, int group) {
    constexpr int CH = 8;                       // steps whose loads are in flight together
    __shared__ f32x4 red[4][MT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nl = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int n = n0 + nl < N ? n0 + nl : N - 1;
    const int kw = K >> 3, zw = (G + 7) >> 3;
    const int steps = K >> 9;                   // 128-column steps per wave (K % 512 == 0)
    const int s0 = wave * steps;
    const uint32_t* wrow = qw + (size_t)n * kw + kq * 4;

    f32x4 yacc[MT];
#pragma unroll
    for (int t = 0; t < MT; t++) yacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int sc = 0; sc < steps; sc += CH) {
        u32x4 wv[CH];
#pragma unroll
        for (int c = 0; c < CH; c++)
            if (sc + c < steps) wv[c] = load16(wrow + (s0 + sc + c) * 16);
#pragma unroll
        for (int c = 0; c < CH; c++) {
            if (sc + c >= steps) break;
            const int kbase = (s0 + sc + c) * 128;
            const int g = kbase / group;
            const float sf = f16_dev(scales[(size_t)n * G + g]);
            uint32_t z = 8;
            if (ZEROS) z = (qz[(size_t)n * zw + (g >> 3)] >> (4 * (g & 7))) & 15u;
            const uint32_t negc = (0xC300u | z) * 0x00010001u;   // bf16 -(128 + z), twice
            const u32x4 bneg = {negc, negc, negc, negc};
            f32x4 acc[MT];
#pragma unroll
            for (int t = 0; t < MT; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t w = wv[c][j];
                u32x4 b;
                b[0] = (w & 0x000F000Fu) | 0x43004300u;
                b[1] = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
                b[2] = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
                b[3] = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
                const bf16x8 bq = __builtin_bit_cast(bf16x8, b);
                const bf16x8 bz = __builtin_bit_cast(bf16x8, bneg);
#pragma unroll
                for (int t = 0; t < MT; t++) {
                    const int m = t * 16 + nl;
                    u32x4 a = {0u, 0u, 0u, 0u};
                    if (m < M) {
                        const u32x4 xv = load16(x + (size_t)m * K + kbase + kq * 32 + j * 8);
                        a[0] = __builtin_amdgcn_perm(xv[2], xv[0], 0x05040100u);
                        a[1] = __builtin_amdgcn_perm(xv[2], xv[0], 0x07060302u);
                        a[2] = __builtin_amdgcn_perm(xv[3], xv[1], 0x05040100u);
                        a[3] = __builtin_amdgcn_perm(xv[3], xv[1], 0x07060302u);
                    }
                    const bf16x8 av = __builtin_bit_cast(bf16x8, a);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bq, acc[t], 0, 0, 0);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bz, acc[t], 0, 0, 0);
                }
            }
#pragma unroll
            for (int t = 0; t < MT; t++) yacc[t] += sf * acc[t];
        }
    }
#pragma unroll
    for (int t = 0; t < MT; t++) red[wave][t][lane] = yacc[t];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < MT; t++) {
        f32x4 v = red[0][t][lane] + red[1][t][lane] + red[2][t][lane] + red[3][t][lane];
        if (n0 + nl >= N) continue;
        if (bias) v += bias[n0 + nl];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = t * 16 + kq * 4 + i;   // MFMA C layout: row 4*(lane/16)+i, col lane%16
            if (m >= M) continue;
            if (YF32)
                reinterpret_cast<float*>(y)[(size_t)m * N + n0 + nl] = v[i];
            else
                reinterpret_cast<uint16_t*>(y)[(size_t)m * N + n0 + nl] = f32_to_bf16(v[i]);
        }
    }
}

// Small-M W4A16 (M <= 4): same work split and k-slot order as k_w4a16_gemv,
// but the activations are staged once per workgroup in LDS, already in the
// MFMA k-slot order, with their sums X[t][m] over every 128-column step t.
// Each MFMA then accumulates sum x*(128+q) and the step epilogue subtracts
// (128+z)*X in fp32, so only one MFMA per packed word is issued.
// Load order matters because vmcnt retires in issue order: the activation
// loads go first, then scales/zeros, then the weights, all unconditional
// (clamped addresses), so staging x never waits for the weight stream.
// XPT = 16-byte activation items per thread (>= M*K/8/256); MM >= M is the
// number of output rows the epilogue keeps; the group size is 1 << gshift.
// PERM: the weight columns are stored in the order perm (uint16 [K]; column
// k' of qw is column perm[k'] of the layer), so the activations are gathered
// the same way: raw x and perm go to LDS first, then each item is rebuilt
// from LDS as x[m][perm[k']] before the slot-order staging.  No global load
// depends on another, so the weight stream is issued exactly as without it.
template <int XPT, int MM, bool ZEROS, bool YF32, bool VS, bool PERM>
__global__ void __launch_bounds__(256) k_w4a16_gemv_small(const uint16_t* __restrict__ x,
                                                          const uint32_t* __restrict__ qw,
                                                          const uint16_t* __restrict__ scales,
                                                          const uint32_t* __restrict__ qz,
                                                          const uint16_t* __restrict__ perm,
                                                          void* __restrict__ y,
                                                          const float* __restrict__ bias, int M,
                                                          int N, int K, int G, int gshift) {
    constexpr int CH = 8;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int xrow = K * 2 + 16;                               // bytes per staged row (+pad)
    float* xsum = reinterpret_cast<float*>(smem + M * xrow);   // [K/128][4]
    f32x4* red = reinterpret_cast<f32x4*>(xsum + (K >> 7) * 4);  // [4 waves][64 lanes]
    uint16_t* xraw = reinterpret_cast<uint16_t*>(red + 256);   // PERM: [M][K] source order
    uint16_t* pl = xraw + M * K;                               // PERM: [K]

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar math
    const int nl = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * 16;
    const int n = n0 + nl < N ? n0 + nl : N - 1;
    const int k8n = K >> 3, zw = (G + 7) >> 3;
    const int steps = K >> 9;
    const int s0 = wave * steps;
    const uint32_t* wrow = qw + (size_t)n * k8n + kq * 4;
    const int nitems = M * k8n;

    // 1. activation items (L2-resident after the first workgroups)
    u32x4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        int it = threadIdx.x + i * 256;
        it = it < nitems ? it : nitems - 1;
        const int m = it / k8n;
        xr[i] = load16(x + (size_t)m * K + (size_t)(it - m * k8n) * 8);
    }
    u32x4 pr[PERM ? XPT : 1];
    if (PERM) {   // perm items: K/8 <= nitems, same item grid
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            int it = threadIdx.x + i * 256;
            it = it < k8n ? it : k8n - 1;
            pr[i] = load16(perm + (size_t)it * 8);
        }
    }
    // keep the activation loads ahead of everything below
    asm volatile("" ::: "memory");
    // 2. scales / zeros, 3. weights of the first chunk
    uint32_t sreg[CH], zreg[CH];
    u32x4 wv[CH];
    if (VS) {   // group 128, chunk aligned to 8 groups: one vector load each
        const u32x4 sv = load16(scales + (size_t)n * G + s0);
#pragma unroll
        for (int c = 0; c < CH; c++) sreg[c] = (sv[c >> 1] >> (16 * (c & 1))) & 0xFFFFu;
        const uint32_t zv = ZEROS ? qz[(size_t)n * zw + (s0 >> 3)] : 0u;
#pragma unroll
        for (int c = 0; c < CH; c++) zreg[c] = zv;
    } else {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int st = s0 + (c < steps ? c : steps - 1);
            const int g = (st << 7) >> gshift;
            sreg[c] = scales[(size_t)n * G + g];
            zreg[c] = ZEROS ? qz[(size_t)n * zw + (g >> 3)] : 0u;
        }
    }
#pragma unroll
    for (int c = 0; c < CH; c++) wv[c] = load16(wrow + (s0 + (c < steps ? c : steps - 1)) * 16);
    asm volatile("" ::: "memory");

    if (PERM) {
        // raw activations and perm to LDS (clamped items rewrite the last
        // item with its own value), then gather each item in perm order
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            int it = threadIdx.x + i * 256;
            it = it < nitems ? it : nitems - 1;
            *reinterpret_cast<u32x4*>(xraw + (size_t)it * 8) = xr[i];
            int ip = threadIdx.x + i * 256;
            ip = ip < k8n ? ip : k8n - 1;
            *reinterpret_cast<u32x4*>(pl + (size_t)ip * 8) = pr[i];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            int it = threadIdx.x + i * 256;
            it = it < nitems ? it : nitems - 1;
            const int m = it / k8n;
            const int k8 = it - m * k8n;
            const u32x4 pv = *reinterpret_cast<const u32x4*>(pl + k8 * 8);
            const uint16_t* xm = xraw + m * K;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                uint32_t lo = pv[e] & 0xFFFFu, hi = pv[e] >> 16;
                lo = lo < (uint32_t)K ? lo : (uint32_t)K - 1u;   // caller's perm stays in LDS bounds
                hi = hi < (uint32_t)K ? hi : (uint32_t)K - 1u;
                xr[i][e] = (uint32_t)xm[lo] | (uint32_t)xm[hi] << 16;
            }
        }
    }

    // stage x in slot order 0,4,1,5,2,6,3,7 per 8 columns (items past the end
    // go to a dummy slot so the stores stay unconditional), and sum every 16
    // consecutive items (one 128-column step) with a 16-lane reduction
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int it = threadIdx.x + i * 256;
        const bool live = it < nitems;
        const int m = (live ? it : nitems - 1) / k8n;
        const int k8 = (live ? it : nitems - 1) - m * k8n;
        const int off = live ? m * xrow + k8 * 16 : M * xrow - 16;
        u32x4 p;
        p[0] = __builtin_amdgcn_perm(xr[i][2], xr[i][0], 0x05040100u);
        p[1] = __builtin_amdgcn_perm(xr[i][2], xr[i][0], 0x07060302u);
        p[2] = __builtin_amdgcn_perm(xr[i][3], xr[i][1], 0x05040100u);
        p[3] = __builtin_amdgcn_perm(xr[i][3], xr[i][1], 0x07060302u);
        *reinterpret_cast<u32x4*>(smem + off) = p;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++)
            sum += __builtin_bit_cast(float, xr[i][e] << 16) + __builtin_bit_cast(float, xr[i][e] & 0xFFFF0000u);
        sum += __shfl_xor(sum, 8);
        sum += __shfl_xor(sum, 4);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 1);
        if (live && (k8 & 15) == 0) xsum[(k8 >> 4) * 4 + m] = sum;
    }
    __syncthreads();

    // constants for v_and_or_b32: gfx9 VOP3 takes no literals, so they live in registers
    uint32_t nib_mask, bf_bias;
    asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(bf_bias));

    const bool arow = nl < M;
    const uint8_t* abase = smem + (arow ? nl : 0) * xrow + kq * 64;
    f32x4 yacc = {0.f, 0.f, 0.f, 0.f};
    for (int sc = 0; sc < steps; sc += CH) {
        if (sc > 0) {
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const int st = s0 + (sc + c < steps ? sc + c : steps - 1);
                const int g = (st << 7) >> gshift;
                sreg[c] = scales[(size_t)n * G + g];
                zreg[c] = ZEROS ? qz[(size_t)n * zw + (g >> 3)] : 0u;
            }
#pragma unroll
            for (int c = 0; c < CH; c++)
                wv[c] = load16(wrow + (s0 + (sc + c < steps ? sc + c : steps - 1)) * 16);
        }
#pragma unroll
        for (int c = 0; c < CH; c++) {
            if (sc + c >= steps) break;
            const int st = s0 + sc + c;
            const int g = (st << 7) >> gshift;
            u32x4 a[4];
#pragma unroll
            for (int j = 0; j < 4; j++) a[j] = u32x4{0u, 0u, 0u, 0u};
            if (arow) {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    a[j] = *reinterpret_cast<const u32x4*>(abase + st * 256 + j * 16);
            }
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t w = wv[c][j];
                u32x4 b;
                b[0] = (w & nib_mask) | bf_bias;
                b[1] = ((w >> 4) & nib_mask) | bf_bias;
                b[2] = ((w >> 8) & nib_mask) | bf_bias;
                b[3] = ((w >> 12) & nib_mask) | bf_bias;
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[j]),
                                                              __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
            }
            const float sf = (float)__builtin_bit_cast(_Float16, (uint16_t)sreg[c]);
            const uint32_t z = ZEROS ? (zreg[c] >> (4 * (g & 7))) & 15u : 8u;
            const float corr = sf * (float)(128u + z);
            const f32x4 xs = *reinterpret_cast<const f32x4*>(xsum + st * 4);
#pragma unroll
            for (int i = 0; i < MM; i++) yacc[i] += sf * acc[i] - corr * xs[i];
        }
    }
    red[wave * 64 + lane] = yacc;
    __syncthreads();
    if (wave != 0 || kq != 0 || n0 + nl >= N) return;
    f32x4 v = red[lane] + red[64 + lane] + red[128 + lane] + red[192 + lane];
    if (bias) v += bias[n0 + nl];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (i >= M) break;
        if (YF32)
            reinterpret_cast<float*>(y)[(size_t)i * N + n0 + nl] = v[i];
        else
            reinterpret_cast<uint16_t*>(y)[(size_t)i * N + n0 + nl] = f32_to_bf16(v[i]);
    }
}

// M = 1 decode GEMV, group 128, K = 2048 T.  A workgroup (8 waves) owns an
// even share of the N output rows (at most 16), each wave up to 2 of them; lane l of a wave covers the 32-column
// chunks c = 64 t + l (16 bytes of a row, one 16-byte load), so a wave load
// instruction reads 1 KB of one row and the lane's columns are the same for
// both rows.  The product runs on v_mfma_f32_4x4x4bf16_1k with only its
// diagonal used: block b = lanes 4b..4b+3, A = the lane's unpacked weights,
// B = the lane's own activations, so D[b][j][j] (lane 4b+j, element j) is
// the lane's partial dot product - a quarter of the outputs of an
// instruction that does a sixteenth of the work of a 16x16x32 one.
// Activations are staged once per workgroup in LDS in MFMA k-slot order with
// their 32-column sums; scales and zero words of the 16 rows are staged raw
// beside them.  Every activation, scale and zero load is issued before any
// weight load of the workgroup (s_barrier between them), because a CU
// returns its loads in issue order; the weight loads are nontemporal.
// PERM: the columns of qw are stored in the order perm (uint16 [K]), so the
// activations are gathered x[perm[k']] from LDS before staging.
// GLU: qw / scales / qzeros hold a stacked gate/up projection [2N][K] (gate
// rows first) and y is bf16 [N] = silu(gate) * up: wave w of a workgroup
// owning output rows [wg0, rend) (at most 8) computes gate row n = wg0 + w and
// up row N + n as its two rows, and lane 63 applies the SwiGLU rule.
// KR (ragged K): K = Kr, a multiple of 256 in (2048 (T - 1), 2048 T); the
// layout is the one of K = 2048 T, with the columns past K as padding: their
// weight loads read zeros without a memory access, and their activations,
// chunk sums and group scales are staged as zeros, so they add exactly 0.
// Scales and zero words are then staged one 4-byte word per thread (rows of
// K / 128 scales need not be 16-byte aligned).
template <int T, bool ZEROS, bool YF32, bool PERM, bool GLU = false, bool KR = false>
__global__ void __launch_bounds__(512) k_w4a16_gemv1(const uint16_t* __restrict__ x,
                                                     const uint32_t* __restrict__ qw,
                                                     const uint16_t* __restrict__ scales,
                                                     const uint32_t* __restrict__ qz,
                                                     const uint16_t* __restrict__ perm,
                                                     void* __restrict__ y,
                                                     const float* __restrict__ bias, int N,
                                                     int rows_q, int rows_rem, int Kr) {
    static_assert(!(GLU && KR), "the GLU form takes K = 2048 T only");
    constexpr int KM = 2048 * T, GM = 16 * T, NCHM = KM / 32, NITM = KM / 8;
    constexpr int RW = 2, WROWS = 16, NTHR = 512;
    constexpr int XPT = (NITM + NTHR - 1) / NTHR;
    constexpr int SPR = 2 * T, ZPRM = 2 * T;                 // 16 B scale pieces, zero words per row (LDS)
    const int K = KR ? Kr : KM, G = KR ? Kr >> 7 : GM, KW = K / 8, NIT = K / 8;
    const int ZPR = KR ? (G + 7) >> 3 : ZPRM;                // zero words per row in memory
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* xsum = reinterpret_cast<float*>(smem + NCHM * 80);            // [NCHM]
    uint32_t* ssc = reinterpret_cast<uint32_t*>(xsum + NCHM);            // [16 rows][GM/2 words]
    uint32_t* szr = ssc + WROWS * (GM / 2);                              // [16 rows][2T words]
    uint16_t* xraw = reinterpret_cast<uint16_t*>(szr + WROWS * ZPRM);    // PERM: [KM]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // rows [wg0, rend) of this workgroup: an even share of N (rows_q or
    // rows_q + 1 <= WROWS; rows_q = N / grid, rows_rem = N % grid), so every
    // CU gets the same number of rows when the grid is a multiple of the CU
    // count
    const int b = blockIdx.x;
    const int wg0 = b * rows_q + (b < rows_rem ? b : rows_rem);
    const int rend = wg0 + rows_q + (b < rows_rem ? 1 : 0);
    const int n0 = GLU ? wg0 + wave : wg0 + wave * RW;

    // 1. activations (and perm), then the raw scales / zero words of the 16 rows
    u32x4 xr[XPT], pr[PERM ? XPT : 1];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        int it = tid + i * NTHR;
        it = it < NIT ? it : NIT - 1;
        xr[i] = load16(x + (size_t)it * 8);
        if (PERM) pr[i] = load16(perm + (size_t)it * 8);
    }
    u32x4 sv = {0u, 0u, 0u, 0u};
    uint32_t zv = 0u;
    const bool sload = tid < WROWS * SPR;
    const bool zload = ZEROS && tid >= WROWS * SPR && tid < WROWS * (SPR + ZPR);
    // staged row j = 2 wave + r: row n0 + r, or (GLU) gate / up row of n0
    auto staged_row = [&](int j) {
        int row = GLU ? wg0 + (j >> 1) : wg0 + j;
        row = row < rend ? row : rend - 1;
        return GLU && (j & 1) ? row + N : row;
    };
    // KR: word u of the [16][GM/2] scale block (row u / (GM/2), scale pair
    // u % (GM/2)) and of the [16][2T] zero block; pairs past G/2 and words
    // past ZPR stay 0
    constexpr int KRS = KR ? (WROWS * (GM / 2) + NTHR - 1) / NTHR : 1;
    constexpr int KRZ = KR && ZEROS ? (WROWS * ZPRM + NTHR - 1) / NTHR : 1;
    uint32_t ksv[KRS], kzv[KRZ];
    if (KR) {
#pragma unroll
        for (int i = 0; i < KRS; i++) {
            const int u = tid + i * NTHR, row = u / (GM / 2), w = u % (GM / 2);
            ksv[i] = u < WROWS * (GM / 2) && w < (G >> 1)
                         ? *reinterpret_cast<const uint32_t*>(scales + (size_t)staged_row(row) * G + 2 * w)
                         : 0u;
        }
#pragma unroll
        for (int i = 0; i < KRZ; i++) {
            const int u = tid + i * NTHR, row = u / ZPRM, w = u % ZPRM;
            kzv[i] = ZEROS && u < WROWS * ZPRM && w < ZPR ? qz[(size_t)staged_row(row) * ZPR + w] : 0u;
        }
    } else {
        if (sload) sv = load16(scales + (size_t)staged_row(tid / SPR) * G + (tid % SPR) * 8);
        if (zload) {
            const int j = tid - WROWS * SPR;
            zv = qz[(size_t)staged_row(j / ZPR) * ZPR + j % ZPR];
        }
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // 2. weights: RW rows x T chunks, all in flight (nontemporal).  A row past
    // the workgroup's share reads zeros without a memory access: its offset
    // lies beyond the buffer's record count.
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(qw), (short)0, (GLU ? 2 : 1) * N * KW * 4, 0x00020000);
    u32x4 wv[RW][T];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        const bool live = GLU ? n0 < rend : n0 + r < rend;
        const uint32_t wrow = GLU ? (uint32_t)(n0 + r * N) : (uint32_t)(n0 + r);
#pragma unroll
        for (int t = 0; t < T; t++) {
            const bool in_k = !KR || 32 * (64 * t + lane) < K;
            const uint32_t off = live && in_k ? wrow * (KW * 4) + (uint32_t)(64 * t + lane) * 16u : kNoRecord;
            wv[r][t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rq, off, 0, kNontemporal));
        }
    }
    asm volatile("" ::: "memory");

    // 3. staging
    if (KR) {
#pragma unroll
        for (int i = 0; i < KRS; i++)
            if (tid + i * NTHR < WROWS * (GM / 2)) ssc[tid + i * NTHR] = ksv[i];
#pragma unroll
        for (int i = 0; i < KRZ; i++)
            if (ZEROS && tid + i * NTHR < WROWS * ZPRM) szr[tid + i * NTHR] = kzv[i];
    } else {
        if (sload) *reinterpret_cast<u32x4*>(ssc + tid * 4) = sv;
        if (zload) szr[tid - WROWS * SPR] = zv;
    }
    if (PERM) {
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const int it = tid + i * NTHR;
            if (it < NIT) *reinterpret_cast<u32x4*>(xraw + it * 8) = xr[i];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < XPT; i++) {
            const u32x4 pv = pr[i];   // the thread's own perm piece (of its clamped item)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                uint32_t lo = pv[e] & 0xFFFFu, hi = pv[e] >> 16;
                lo = lo < (uint32_t)K ? lo : (uint32_t)K - 1u;   // the caller's perm stays in LDS bounds
                hi = hi < (uint32_t)K ? hi : (uint32_t)K - 1u;
                xr[i][e] = (uint32_t)xraw[lo] | (uint32_t)xraw[hi] << 16;
            }
        }
    }
    // k-slot order {0,4,1,5 | 2,6,3,7} per 8 columns; chunk c (4 items) at c * 80 bytes;
    // chunk sums over the 4 items held by 4 consecutive lanes.  KR: the items
    // past K (up to 2048 T) are staged as zeros.
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int it0 = tid + i * NTHR;
        const bool live = it0 < (KR ? NITM : NIT);
        const int it = live ? it0 : NIT - 1;
        if (KR && it0 >= NIT) xr[i] = u32x4{0u, 0u, 0u, 0u};
        u32x4 p;
        p[0] = __builtin_amdgcn_perm(xr[i][2], xr[i][0], 0x05040100u);
        p[1] = __builtin_amdgcn_perm(xr[i][2], xr[i][0], 0x07060302u);
        p[2] = __builtin_amdgcn_perm(xr[i][3], xr[i][1], 0x05040100u);
        p[3] = __builtin_amdgcn_perm(xr[i][3], xr[i][1], 0x07060302u);
        if (live) *reinterpret_cast<u32x4*>(smem + (it >> 2) * 80 + (it & 3) * 16) = p;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++)
            sum += __builtin_bit_cast(float, xr[i][e] << 16) + __builtin_bit_cast(float, xr[i][e] & 0xFFFF0000u);
        sum += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, sum), 0xB1, 0xF, 0xF, false));
        sum += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, sum), 0x4E, 0xF, 0xF, false));
        if (live && (it & 3) == 0) xsum[it >> 2] = sum;
    }
    __syncthreads();

    // 4. this lane's activations, chunk sums, scales and zero-point correction
    // JIT (K > 8192): each chunk's activations are read from LDS where the
    // chunk is used (once per row) instead of being held for both rows: 16
    // registers instead of 16 T, so two workgroups fit on a CU.
    constexpr bool JIT = T >= 5;
    uint32_t xb[JIT ? 1 : T][16];
    float X[T];
#pragma unroll
    for (int t = 0; t < T; t++) {
        const int c = 64 * t + lane;
        if (!JIT) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(smem + c * 80 + q * 16);
                xb[JIT ? 0 : t][4 * q] = v[0];
                xb[JIT ? 0 : t][4 * q + 1] = v[1];
                xb[JIT ? 0 : t][4 * q + 2] = v[2];
                xb[JIT ? 0 : t][4 * q + 3] = v[3];
            }
        }
        X[t] = xsum[c];
    }
    float sc[RW][T], corr[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        corr[r] = 0.0f;
        const int wr = wave * RW + r;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int g = 16 * t + (lane >> 2);                 // group of chunk 64 t + lane
            const uint32_t sw = ssc[wr * (GM / 2) + (g >> 1)];
            const float s = f16_dev((uint16_t)((g & 1) ? (sw >> 16) : (sw & 0xFFFFu)));
            const uint32_t z = ZEROS ? (szr[wr * ZPRM + (g >> 3)] >> (4 * (g & 7))) & 15u : 8u;
            sc[r][t] = s;
            corr[r] = fmaf(s * (float)(128u + z), X[t], corr[r]);
        }
    }

    // 5. nibbles -> bf16 (128 + q), one and-or per pair; diagonal 4x4x4 MFMAs.
    // The weight loads are consumed in issue order (row 0's chunks, then row
    // 1's), each chunk's products fenced from the next by a scheduling
    // barrier, and row 0 is summed across the wave before row 1's loads are
    // waited for: after the last load lands only one chunk's products, one
    // wave sum and the stores remain.  The stores stay at the end: a store
    // issued earlier counts in vmcnt and would make the waits for row 1's
    // loads cover both of them.
    uint32_t nib_mask, bf_bias;
    asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(bf_bias));
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const int dg = lane & 3;
    float out[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) {
        f32x4 y4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < T; t++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            uint32_t xc[16];
            if constexpr (JIT) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u32x4 v = *reinterpret_cast<const u32x4*>(smem + (64 * t + lane) * 80 + q * 16);
                    xc[4 * q] = v[0];
                    xc[4 * q + 1] = v[1];
                    xc[4 * q + 2] = v[2];
                    xc[4 * q + 3] = v[3];
                }
            } else {
#pragma unroll
                for (int q = 0; q < 16; q++) xc[q] = xb[JIT ? 0 : t][q];
            }
#pragma unroll
            for (int d = 0; d < 4; d++) {
                const uint32_t w = wv[r][t][d];
                const u32x2 a0 = {(w & nib_mask) | bf_bias, ((w >> 4) & nib_mask) | bf_bias};
                const u32x2 a1 = {((w >> 8) & nib_mask) | bf_bias, ((w >> 12) & nib_mask) | bf_bias};
                const u32x2 b0 = {xc[4 * d], xc[4 * d + 1]};
                const u32x2 b1 = {xc[4 * d + 2], xc[4 * d + 3]};
                acc = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, a0),
                                                             __builtin_bit_cast(s16x4, b0), acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, a1),
                                                             __builtin_bit_cast(s16x4, b1), acc, 0, 0, 0);
            }
            y4 += sc[r][t] * acc;
            __builtin_amdgcn_sched_barrier(0);
        }
        // 6. the lane's diagonal element, wave sum to lane 63
        const float d = dg == 0 ? y4[0] : dg == 1 ? y4[1] : dg == 2 ? y4[2] : y4[3];
        out[r] = dpp_sum_to_lane63(d - corr[r]);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (lane == 63 && GLU) {
        if (n0 < rend) {
            const float g = bias ? out[0] + bias[n0] : out[0];
            const float u = bias ? out[1] + bias[N + n0] : out[1];
            reinterpret_cast<uint16_t*>(y)[n0] = bf16_out(silu_mul_fast(g, u));
        }
    } else if (lane == 63) {
#pragma unroll
        for (int r = 0; r < RW; r++) {
            if (n0 + r >= rend) break;
            if (bias) out[r] += bias[n0 + r];
            if (YF32)
                reinterpret_cast<float*>(y)[n0 + r] = out[r];
            else
                reinterpret_cast<uint16_t*>(y)[n0 + r] = f32_to_bf16(out[r]);
        }
    }
}

// Split-K W4A16 for 5 <= M <= 16: workgroup (bx, s) owns output rows
// [64 bx, +64) (16 per wave) and the K span [s kspan, +kspan).  It stages
// only that span of the M activation rows in LDS (slot order, per-step
// sums), so the four waves share one copy, and every wave streams its 16
// weight rows across the span with all of its loads in flight at once.
// MFMA rows beyond M read zeros.  Partial sums go to part[s][M][N] (fp32);
// k_w4a16_reduce adds the S partials in a fixed order.
template <bool ZEROS>
__global__ void __launch_bounds__(256) k_w4a16_splitk(const uint16_t* __restrict__ x,
                                                      const uint32_t* __restrict__ qw,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint32_t* __restrict__ qz,
                                                      float* __restrict__ part, int M, int N,
                                                      int K, int G, int gshift, int kspan) {
    constexpr int CH = 8;                                       // steps per wave (kspan <= 1024)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int xrow = kspan * 2 + 16;                            // bytes per staged row (+pad)
    float* xsum = reinterpret_cast<float*>(smem + 16 * xrow);   // [steps][16]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nl = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * 64 + wave * 16;
    const int n = n0 + nl < N ? n0 + nl : N - 1;
    const int s = blockIdx.y, kb = s * kspan;
    const int steps = kspan >> 7;
    const int k8n = K >> 3, zw = (G + 7) >> 3;
    const int span8 = kspan >> 3, nitems = M * span8;           // <= 8 items per thread

    // 1. activation items of the span (L2-resident after the first workgroups)
    u32x4 xr[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        int it = tid + i * 256;
        it = it < nitems ? it : nitems - 1;
        const int m = it / span8;
        xr[i] = load16(x + (size_t)m * K + kb + (it - m * span8) * 8);
    }
    asm volatile("" ::: "memory");
    // 2. scales / zeros, 3. weights: every step of the span in flight
    uint32_t sreg[CH], zreg[CH];
    u32x4 wv[CH];
    const uint32_t* wrow = qw + (size_t)n * k8n + (kb >> 3) + kq * 4;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int st = c < steps ? c : steps - 1;
        const int g = (kb + st * 128) >> gshift;
        sreg[c] = scales[(size_t)n * G + g];
        zreg[c] = ZEROS ? qz[(size_t)n * zw + (g >> 3)] : 0u;
    }
#pragma unroll
    for (int c = 0; c < CH; c++) wv[c] = load16(wrow + (c < steps ? c : steps - 1) * 16);
    asm volatile("" ::: "memory");

    // stage the span in slot order 0,4,1,5,2,6,3,7 and sum every 128 columns
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int it = tid + i * 256;
        const bool live = it < nitems;
        const int itc = live ? it : nitems - 1;
        const int m = itc / span8;
        const int k8 = itc - m * span8;
        const int off = live ? m * xrow + k8 * 16 : 16 * xrow - 16;   // dead items: pad slot
        u32x4 p;
        p[0] = __builtin_amdgcn_perm(xr[i][2], xr[i][0], 0x05040100u);
        p[1] = __builtin_amdgcn_perm(xr[i][2], xr[i][0], 0x07060302u);
        p[2] = __builtin_amdgcn_perm(xr[i][3], xr[i][1], 0x05040100u);
        p[3] = __builtin_amdgcn_perm(xr[i][3], xr[i][1], 0x07060302u);
        *reinterpret_cast<u32x4*>(smem + off) = p;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++)
            sum += __builtin_bit_cast(float, xr[i][e] << 16) + __builtin_bit_cast(float, xr[i][e] & 0xFFFF0000u);
        sum += __shfl_xor(sum, 8);
        sum += __shfl_xor(sum, 4);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 1);
        if (live && (k8 & 15) == 0) xsum[(k8 >> 4) * 16 + m] = sum;
    }
    __syncthreads();

    uint32_t nib_mask, bf_bias;
    asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(bf_bias));

    const bool arow = nl < M;
    const uint8_t* abase = smem + (arow ? nl : 0) * xrow + kq * 64;
    f32x4 yacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CH; c++) {
        if (c >= steps) break;
        const int g = (kb + c * 128) >> gshift;
        u32x4 a[4];
#pragma unroll
        for (int j = 0; j < 4; j++) a[j] = u32x4{0u, 0u, 0u, 0u};
        if (arow) {
#pragma unroll
            for (int j = 0; j < 4; j++) a[j] = *reinterpret_cast<const u32x4*>(abase + c * 256 + j * 16);
        }
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t w = wv[c][j];
            u32x4 b;
            b[0] = (w & nib_mask) | bf_bias;
            b[1] = ((w >> 4) & nib_mask) | bf_bias;
            b[2] = ((w >> 8) & nib_mask) | bf_bias;
            b[3] = ((w >> 12) & nib_mask) | bf_bias;
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[j]),
                                                          __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
        }
        const float sf = (float)__builtin_bit_cast(_Float16, (uint16_t)sreg[c]);
        const uint32_t z = ZEROS ? (zreg[c] >> (4 * (g & 7))) & 15u : 8u;
        const float corr = sf * (float)(128u + z);
        const f32x4 xs = *reinterpret_cast<const f32x4*>(xsum + c * 16 + kq * 4);
#pragma unroll
        for (int i = 0; i < 4; i++) yacc[i] += sf * acc[i] - corr * xs[i];
    }
    if (n0 + nl >= N) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {   // MFMA C layout: row 4 (lane/16) + i, column lane % 16
        const int m = kq * 4 + i;
        if (m < M) part[((size_t)s * M + m) * N + n0 + nl] = yacc[i];
    }
}

// y[m][n] = sum over s of part[s][m][n], s ascending
__global__ void __launch_bounds__(256) k_w4a16_reduce(const float* __restrict__ part,
                                                      void* __restrict__ y, int y_f32, int S,
                                                      size_t MN, int N,
                                                      const float* __restrict__ bias) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= MN) return;
    float v = 0.0f;
    for (int s = 0; s < S; s++) v += part[(size_t)s * MN + i];
    if (bias) v += bias[i % (size_t)N];
    if (y_f32)
        reinterpret_cast<float*>(y)[i] = v;
    else
        reinterpret_cast<uint16_t*>(y)[i] = f32_to_bf16(v);
}

struct W4Launch {
    const uint16_t* x;
    const uint32_t* qw;
    const uint16_t* scales;
    const uint32_t* qz;
    const uint16_t* perm;
    void* y;
    const float* bias;
    int y_f32, M, N, K, G, group;
    size_t lds;
    hipStream_t s;
};

template <int XPT, int MM, bool VS, bool PERM>
int launch_small_vs(const W4Launch& a) {
    dim3 grid((unsigned)((a.N + 15) / 16)), block(256);
    const int gshift = __builtin_ctz((unsigned)a.group);
#define SNX_SMALL(Z, F)                                                                         \
    k_w4a16_gemv_small<XPT, MM, Z, F, VS, PERM><<<grid, block, a.lds, a.s>>>(                   \
        a.x, a.qw, a.scales, a.qz, a.perm, a.y, a.bias, a.M, a.N, a.K, a.G, gshift)
    if (a.qz) {
        if (a.y_f32) SNX_SMALL(true, true);
        else SNX_SMALL(true, false);
    } else {
        if (a.y_f32) SNX_SMALL(false, true);
        else SNX_SMALL(false, false);
    }
#undef SNX_SMALL
    return snx_launch_check("k_w4a16_gemv_small");
}

template <int XPT, int MM, bool PERM>
int launch_small_m(const W4Launch& a) {
    // vector scale/zero loads: group 128 and each wave's steps exactly 8
    const int steps = a.K >> 9;
    if (a.group == 128 && steps == 8 && (a.G & 7) == 0) return launch_small_vs<XPT, MM, true, PERM>(a);
    return launch_small_vs<XPT, MM, false, PERM>(a);
}

// LDS of k_w4a16_gemv1 for K = 2048 T (the ragged form takes that of the
// next multiple of 2048).
size_t gemv1_lds(size_t K, bool perm) {
    const size_t nch = K / 32, g = K / 128;
    return nch * 80 + nch * 4 + 16 * (g / 2) * 4 + 16 * (g / 8) * 4 + (perm ? 2 * K : 0);
}

// Workgroups of the M = 1 kernel: enough for at most `per` rows each (16, or
// 8 output rows of the GLU form), rounded up to a multiple of the CU count
// once there is more than one per CU, so each workgroup takes an even share
// of the rows and every CU the same number.
unsigned gemv1_grid(int N, int per = 16) {
    const int ncu = snx::cu_count();
    int nwg = (N + per - 1) / per;
    if (nwg > ncu) nwg = (nwg + ncu - 1) / ncu * ncu;
    return (unsigned)(nwg < N ? nwg : N);
}

template <int T, bool PERM, bool KR>
int launch_gemv1_t(const W4Launch& a) {
    dim3 grid(gemv1_grid(a.N)), block(512);
    const size_t lds = gemv1_lds((size_t)(2048 * T), PERM);
    if (lds > 64 * 1024) {   // PERM at K > 12288: the staged copy of x
        static std::atomic<uint64_t> lds_done[4];   // (zeros, f32 out) variants, per device
        const void* kfn[4] = {reinterpret_cast<const void*>(&k_w4a16_gemv1<T, false, false, PERM, false, KR>),
                              reinterpret_cast<const void*>(&k_w4a16_gemv1<T, false, true, PERM, false, KR>),
                              reinterpret_cast<const void*>(&k_w4a16_gemv1<T, true, false, PERM, false, KR>),
                              reinterpret_cast<const void*>(&k_w4a16_gemv1<T, true, true, PERM, false, KR>)};
        const int v = (a.qz ? 2 : 0) + (a.y_f32 ? 1 : 0);
        if (snx::lds_optin(kfn[v], (int)lds, lds_done[v]) != hipSuccess) {
            snx_set_error("w4a16 gemv: cannot reserve %zu bytes of LDS", lds);
            return -1;
        }
    }
#define SNX_G1(Z, F)                                                                      \
    k_w4a16_gemv1<T, Z, F, PERM, false, KR><<<grid, block, lds, a.s>>>(                           \
        a.x, a.qw, a.scales, a.qz, a.perm, a.y, a.bias, a.N, a.N / (int)grid.x, a.N % (int)grid.x, a.K)
    if (a.qz) {
        if (a.y_f32) SNX_G1(true, true);
        else SNX_G1(true, false);
    } else {
        if (a.y_f32) SNX_G1(false, true);
        else SNX_G1(false, false);
    }
#undef SNX_G1
    return snx_launch_check("k_w4a16_gemv1");
}

// k_w4a16_gemv1 applies: M = 1, group 128, K a multiple of 256 up to 16384;
// K = 2048 T takes 16-byte aligned scales, the ragged form (other K) 4-byte
// aligned ones; 4-byte aligned zero words; weight offsets below the buffer
// limit.
bool gemv1_ok(const W4Launch& a) {
    const uintptr_t salign = a.K % 2048 == 0 ? 15u : 3u;
    return a.M == 1 && a.group == 128 && a.K % 256 == 0 && a.K >= 256 && a.K <= 16384 &&
           ((uintptr_t)a.scales & salign) == 0 && ((uintptr_t)a.qz & 3u) == 0 &&
           (uint64_t)a.N * (uint64_t)a.K / 2 < kNoRecord;   // buffer offsets of the weights
}

template <bool PERM, bool KR>
int launch_gemv1_k(const W4Launch& a) {
    switch ((a.K + 2047) / 2048) {
        case 1: return launch_gemv1_t<1, PERM, KR>(a);
        case 2: return launch_gemv1_t<2, PERM, KR>(a);
        case 3: return launch_gemv1_t<3, PERM, KR>(a);
        case 4: return launch_gemv1_t<4, PERM, KR>(a);
        case 5: return launch_gemv1_t<5, PERM, KR>(a);
        case 6: return launch_gemv1_t<6, PERM, KR>(a);
        case 7: return launch_gemv1_t<7, PERM, KR>(a);
        default: return launch_gemv1_t<8, PERM, KR>(a);
    }
}

template <bool PERM>
int launch_gemv1(const W4Launch& a) {
    return a.K % 2048 == 0 ? launch_gemv1_k<PERM, false>(a) : launch_gemv1_k<PERM, true>(a);
}

template <int T>
int launch_gemv1_glu_t(const W4Launch& a) {
    dim3 grid(gemv1_grid(a.N, 8)), block(512);
    const size_t lds = gemv1_lds((size_t)a.K, false);
#define SNX_G1(Z)                                                                                 \
    k_w4a16_gemv1<T, Z, false, false, true><<<grid, block, lds, a.s>>>(                           \
        a.x, a.qw, a.scales, a.qz, nullptr, a.y, a.bias, a.N, a.N / (int)grid.x, a.N % (int)grid.x, a.K)
    if (a.qz) SNX_G1(true);
    else SNX_G1(false);
#undef SNX_G1
    return snx_launch_check("k_w4a16_gemv1<glu>");
}

template <int XPT, bool PERM>
int launch_small(const W4Launch& a) {
    if (gemv1_ok(a)) return launch_gemv1<PERM>(a);
    if (a.M == 1) return launch_small_m<XPT, 1, PERM>(a);
    if (a.M == 2) return launch_small_m<XPT, 2, PERM>(a);
    return launch_small_m<XPT, 4, PERM>(a);
}

// Decode GEMV for 2 <= M <= 16 activation rows: group 128, K = 1024 NC
// (NC <= 4), on v_mfma_f32_16x16x32_bf16 with the activations as the A
// operand (16 rows, rows >= M zero) and 16 weight rows as B.
// Persistent: one workgroup (8 waves) per CU copies the M activation rows
// once into LDS, then walks the 16-row groups rg = b, b + nb, ...  Wave w
// owns columns [K w / 8, K (w + 1) / 8) of every group.  Its A fragments are
// read from LDS once, put in the nibble unpack's column order
// {0,4,1,5,2,6,3,7} (v_perm) and kept in registers; the 128-column sums X of
// its activation rows come from the same fragments times a ones operand on
// the matrix cores.  Per group each lane (row n = l % 16, quarter
// q = l / 16) loads NC 16-byte pieces of its row (words 16 c + 4 q .. +3 of
// the wave's part; chunk c is quantization group w NC + c); MFMA (c, e) takes
// word e of every lane's piece c, so A and B lanes with the same quarter
// hold the same eight columns.  Per group c:
// y += s (sum of the 4 MFMAs) - s (128 + z) X, which removes the 128 bias of
// the unpacked nibbles and the zero point exactly.  The 8 waves' partial
// 16 x 16 tiles are added in LDS in wave order (deterministic).  The first
// three groups' loads go out at the start, after every activation load of the
// workgroup (a CU returns its loads in issue order).  PERM: qw's columns are
// stored in the order perm (uint16 [K]); the A fragments gather
// x[m][perm[k']] from the LDS copy.
template <int NC, bool ZEROS, bool YF32, bool PERM, int EARLY>
__global__ void __launch_bounds__(512) k_w4a16_gemv_mt(const uint16_t* __restrict__ x,
                                                       const uint32_t* __restrict__ qw,
                                                       const uint16_t* __restrict__ scales,
                                                       const uint32_t* __restrict__ qz,
                                                       const uint16_t* __restrict__ perm,
                                                       void* __restrict__ y,
                                                       const float* __restrict__ bias, int M,
                                                       int N) {
    constexpr int K = 1024 * NC, KW = K / 8, G = K / 128, ZW = (G + 7) / 8;
    constexpr int RS = K * 2 + 16;            // LDS row stride in bytes (16 B pad: no bank conflicts)
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* xs = smem;                                                  // [M][RS]
    f32x4* red = reinterpret_cast<f32x4*>(smem + (size_t)M * RS);       // [2][8][64]
    uint16_t* pl = reinterpret_cast<uint16_t*>(red + 2 * 8 * 64);       // PERM: [K]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, q4 = lane >> 4;
    const int ngroups = (N + 15) >> 4, nb = gridDim.x;
    const int kw0 = wave * NC * 16;           // first packed word of the wave's columns

    // weight pieces of group rg (rows clamped into the matrix), scales (packed
    // fp16 pairs, kept packed so nothing waits on them before use), zero words
    // (groups wave NC .. wave NC + NC - 1 span two words only for NC = 3)
    constexpr int NS = (NC + 1) / 2;
    constexpr int NZ = NC == 3 ? 2 : 1;
    // Groups past the end load the workgroup's first group again (cached, never
    // used): every path issues the same loads, so each wait stays exact.
    auto wload = [&](int rg, u32x4 (&wv)[NC], uint32_t (&sc)[NS], uint32_t (&zw)[NZ]) {
        int n = (rg < ngroups ? rg : (int)blockIdx.x) * 16 + l16;
        n = n < N ? n : N - 1;
        const uint32_t* row = qw + (size_t)n * KW + kw0 + 4 * q4;
#pragma unroll
        for (int c = 0; c < NC; c++)
            wv[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + 16 * c));
        const uint16_t* srow = scales + (size_t)n * G + wave * NC;
        if (NC % 2 == 0) {          // 4-byte aligned: G and wave NC are even
#pragma unroll
            for (int j = 0; j < NS; j++) sc[j] = reinterpret_cast<const uint32_t*>(srow)[j];
        } else {
#pragma unroll
            for (int j = 0; j < NS; j++)
                sc[j] = (uint32_t)srow[2 * j] | (2 * j + 1 < NC ? (uint32_t)srow[2 * j + 1] << 16 : 0u);
        }
#pragma unroll
        for (int j = 0; j < NZ; j++) {
            const int gz = (wave * NC + j * (NC - 1)) >> 3;
            zw[j] = ZEROS ? qz[(size_t)n * ZW + gz] : 0u;
        }
    };
    int rg = blockIdx.x;
    if (rg >= ngroups) return;
    u32x4 wa[NC], wb[NC], wc[NC];
    uint32_t sa[NS], sb[NS], sc3[NS], za[NZ], zb[NZ], zc[NZ];

    // 1. the activation rows (and perm) copied into LDS as they are
    const int items = M * KW;
    constexpr int XPT = (16 * KW + 511) / 512;
    u32x4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int it = tid + 512 * i;
        if (it < items) xr[i] = load16(x + (size_t)it * 8);
    }
    constexpr int PPT = PERM ? (KW + 511) / 512 : 1;
    u32x4 pr[PPT];
    if (PERM) {
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int it = tid + 512 * i;
            if (it < KW) pr[i] = load16(perm + (size_t)it * 8);
        }
    }
    // the first EARLY groups' weights go out right behind the activation (and
    // perm) loads: the CU returns loads in issue order, so the copy below
    // waits only for the activations while those weights stream.  More
    // groups issued this early fill the CU's queue of outstanding loads and
    // hold up the copy (EARLY = 2 pays from M = 12 on, where the copy itself
    // is long; all three groups this early is slower at every M).
    static_assert(EARLY == 1 || EARLY == 2, "one or two groups ahead of the copy");
    wload(rg, wa, sa, za);
    if constexpr (EARLY == 2) wload(rg + nb, wb, sb, zb);
#pragma unroll
    for (int i = 0; i < XPT; i++) {
        const int it = tid + 512 * i;
        if (it < items) {
            const int m = it / KW, w = it - m * KW;
            *reinterpret_cast<u32x4*>(xs + (size_t)m * RS + (size_t)w * 16) = xr[i];
        }
    }
    if (PERM) {
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int it = tid + 512 * i;
            if (it < KW) *reinterpret_cast<u32x4*>(pl + (size_t)it * 8) = pr[i];
        }
    }
    lds_barrier();
    // the remaining of the first three groups once the activations are in LDS
    if constexpr (EARLY == 1) wload(rg + nb, wb, sb, zb);
    wload(rg + 2 * nb, wc, sc3, zc);

    // 2. the wave's A fragments: row l16 (zero beyond M), words
    //    kw0 + 16 c + 4 q4 + e, columns put in the order {0,4,1,5,2,6,3,7}
    bf16x8 af[NC][4];
    {
        const bool mlive = l16 < M;
        const int mrow = mlive ? l16 : 0;
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int wd = kw0 + 16 * c + 4 * q4 + e;
                u32x4 v;
                if (PERM) {      // columns perm[8 wd + j] of the original order
                    const u32x4 pv = *reinterpret_cast<const u32x4*>(pl + (size_t)wd * 8);
                    const uint16_t* xrow = reinterpret_cast<const uint16_t*>(xs + (size_t)mrow * RS);
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        uint32_t lo = pv[j] & 0xFFFFu, hi = pv[j] >> 16;
                        lo = lo < (uint32_t)K ? lo : (uint32_t)K - 1u;   // the caller's perm stays in LDS bounds
                        hi = hi < (uint32_t)K ? hi : (uint32_t)K - 1u;
                        v[j] = (uint32_t)xrow[lo] | (uint32_t)xrow[hi] << 16;
                    }
                } else {
                    v = *reinterpret_cast<const u32x4*>(xs + (size_t)mrow * RS + (size_t)wd * 16);
                }
                u32x4 p;
                p[0] = __builtin_amdgcn_perm(v[2], v[0], 0x05040100u);
                p[1] = __builtin_amdgcn_perm(v[2], v[0], 0x07060302u);
                p[2] = __builtin_amdgcn_perm(v[3], v[1], 0x05040100u);
                p[3] = __builtin_amdgcn_perm(v[3], v[1], 0x07060302u);
                af[c][e] = __builtin_bit_cast(bf16x8, mlive ? p : u32x4{0u, 0u, 0u, 0u});
            }
    }
    // 128-column sums of the wave's groups: rows 4 q4 + i of lane l's column
    f32x4 xsum[NC];
    {
        const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};   // bf16 1.0
#pragma unroll
        for (int c = 0; c < NC; c++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; e++)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[c][e], __builtin_bit_cast(bf16x8, ones), acc, 0, 0, 0);
            xsum[c] = acc;
        }
    }

    uint32_t nib_mask, bf_bias;
    asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(bf_bias));

    // 3. groups
    int rb = 0;
    auto group = [&](int g, u32x4 (&wv)[NC], uint32_t (&sc)[NS], uint32_t (&zw)[NZ]) {
        f32x4 y4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NC; c++) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t w = wv[c][e];
                u32x4 b;
                b[0] = (w & nib_mask) | bf_bias;
                b[1] = ((w >> 4) & nib_mask) | bf_bias;
                b[2] = ((w >> 8) & nib_mask) | bf_bias;
                b[3] = ((w >> 12) & nib_mask) | bf_bias;
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[c][e], __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
            }
            const int gq = wave * NC + c;
            const float s = f16_dev((uint16_t)(sc[c >> 1] >> (16 * (c & 1))));
            const uint32_t zword = (NZ == 2 && (gq >> 3) != ((wave * NC) >> 3)) ? zw[NZ - 1] : zw[0];
            const uint32_t z = ZEROS ? (zword >> (4 * (gq & 7))) & 15u : 8u;
            const float cs = s * (float)(128u + z);
#pragma unroll
            for (int i = 0; i < 4; i++) y4[i] = fmaf(s, acc[i], fmaf(-cs, xsum[c][i], y4[i]));
        }
        red[(rb * 8 + wave) * 64 + lane] = y4;
        lds_barrier();
        if (tid < 256) {           // output (m, n) = (4 (l / 16) + i, l % 16) of lane l = tid / 4
            const int l = tid >> 2, i = tid & 3;
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < 8; w++) v += red[(rb * 8 + w) * 64 + l][i];
            const int m = 4 * (l >> 4) + i, n = g * 16 + (l & 15);
            if (m < M && n < N) {
                if (bias) v += bias[n];
                if (YF32)
                    reinterpret_cast<float*>(y)[(size_t)m * N + n] = v;
                else
                    reinterpret_cast<uint16_t*>(y)[(size_t)m * N + n] = f32_to_bf16(v);
            }
        }
        rb ^= 1;                   // the other reduction buffer: no second barrier
    };
    // up to three groups per workgroup (N <= 48 x CUs) run from the loads
    // issued at the start, in straight-line code so each wait covers only its
    // own group; any further groups load one at a time
    group(rg, wa, sa, za);
    if (rg + nb < ngroups) group(rg + nb, wb, sb, zb);
    if (rg + 2 * nb < ngroups) group(rg + 2 * nb, wc, sc3, zc);
    for (int g = rg + 3 * nb; g < ngroups; g += nb) {
        wload(g, wa, sa, za);
        group(g, wa, sa, za);
    }
}

template <int NC, bool Z, bool F, bool PERM, int EARLY>
int launch_gemv_mt_e(const uint16_t* x, const uint32_t* qw, const uint16_t* scales, const uint32_t* qz,
                     const uint16_t* perm, void* y, const float* bias, int M, int N, size_t lds, int grid,
                     hipStream_t st) {
    // the LDS size depends on M: opt in to the most any call may ask for
    static std::atomic<uint64_t> lds_done{0};   // > 64 KB of LDS per workgroup, per device
    const void* kfn = reinterpret_cast<const void*>(&k_w4a16_gemv_mt<NC, Z, F, PERM, EARLY>);
    if (snx::lds_optin(kfn, 160 * 1024, lds_done) != hipSuccess) {
        snx_set_error("w4a16 gemv: cannot reserve %zu bytes of LDS", lds);
        return -1;
    }
    k_w4a16_gemv_mt<NC, Z, F, PERM, EARLY><<<grid, 512, lds, st>>>(x, qw, scales, qz, perm, y, bias, M, N);
    return snx_launch_check("k_w4a16_gemv_mt");
}

// Measured at N = 11008, K = 4096: one group's weights ahead of the
// activation copy is fastest up to M = 10 (8.1-8.5 against 8.5-8.8 us with
// two), two from M = 12 (8.8-9.2 against 9.0-9.6 us).
template <int NC, bool Z, bool F, bool PERM>
int launch_gemv_mt(const uint16_t* x, const uint32_t* qw, const uint16_t* scales, const uint32_t* qz,
                   const uint16_t* perm, void* y, const float* bias, int M, int N, size_t lds, int grid,
                   hipStream_t st) {
    if (M > 10)
        return launch_gemv_mt_e<NC, Z, F, PERM, 2>(x, qw, scales, qz, perm, y, bias, M, N, lds, grid, st);
    return launch_gemv_mt_e<NC, Z, F, PERM, 1>(x, qw, scales, qz, perm, y, bias, M, N, lds, grid, st);
}

template <int NC, bool PERM>
int launch_gemv_mt_nc(const uint16_t* x, const uint32_t* qw, const uint16_t* scales, const uint32_t* qz,
                      const uint16_t* perm, void* y, const float* bias, int y_f32, int M, int N,
                      size_t lds, int grid, hipStream_t st) {
    if (qz) {
        if (y_f32) return launch_gemv_mt<NC, true, true, PERM>(x, qw, scales, qz, perm, y, bias, M, N, lds, grid, st);
        return launch_gemv_mt<NC, true, false, PERM>(x, qw, scales, qz, perm, y, bias, M, N, lds, grid, st);
    }
    if (y_f32) return launch_gemv_mt<NC, false, true, PERM>(x, qw, scales, qz, perm, y, bias, M, N, lds, grid, st);
    return launch_gemv_mt<NC, false, false, PERM>(x, qw, scales, qz, perm, y, bias, M, N, lds, grid, st);
}

template <bool PERM>
int launch_gemv_mt_k(const uint16_t* x, const uint32_t* qw, const uint16_t* scales, const uint32_t* qz,
                     const uint16_t* perm, void* y, const float* bias, int y_f32, int M, int N, int K,
                     size_t lds, int grid, hipStream_t st) {
    switch (K / 1024) {
        case 1: return launch_gemv_mt_nc<1, PERM>(x, qw, scales, qz, perm, y, bias, y_f32, M, N, lds, grid, st);
        case 2: return launch_gemv_mt_nc<2, PERM>(x, qw, scales, qz, perm, y, bias, y_f32, M, N, lds, grid, st);
        case 3: return launch_gemv_mt_nc<3, PERM>(x, qw, scales, qz, perm, y, bias, y_f32, M, N, lds, grid, st);
        default: return launch_gemv_mt_nc<4, PERM>(x, qw, scales, qz, perm, y, bias, y_f32, M, N, lds, grid, st);
    }
}

// Generic W4A16: one wave per output column n, any group layout and M.
__global__ void __launch_bounds__(256) k_w4a16_generic(const uint16_t* __restrict__ x,
                                                       const uint32_t* __restrict__ qw,
                                                       const uint16_t* __restrict__ scales,
                                                       const uint32_t* __restrict__ qz,
                                                       const int32_t* __restrict__ g_idx,
                                                       void* __restrict__ y,
                                                       const float* __restrict__ bias, int y_f32,
                                                       int M, int N, int K, int G, int group) {
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    const int kw = K >> 3, zw = (G + 7) >> 3;
    for (int m = 0; m < M; m++) {
        float acc = 0.0f;
        for (int wd = lane; wd < kw; wd += 64) {
            const uint32_t w = qw[(size_t)n * kw + wd];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int k = wd * 8 + t;
                int g = g_idx ? g_idx[k] : k / group;
                g = g < 0 ? 0 : (g >= G ? G - 1 : g);   // out-of-range g_idx stays in bounds
                const int z = qz ? (int)((qz[(size_t)n * zw + (g >> 3)] >> (4 * (g & 7))) & 15u) : 8;
                const float deq = (float)((int)((w >> (4 * t)) & 15u) - z) *
                                  f16_dev(scales[(size_t)n * G + g]);
                acc += bf16_to_f32(x[(size_t)m * K + k]) * deq;
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            if (bias) acc += bias[n];
            if (y_f32)
                reinterpret_cast<float*>(y)[(size_t)m * N + n] = acc;
            else
                reinterpret_cast<uint16_t*>(y)[(size_t)m * N + n] = f32_to_bf16(acc);
        }
    }
}

template <int MT>
int launch_w4a16(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                 const uint32_t* qz, void* y, const float* bias, int y_f32, int M, int N, int K,
                 int G, int group, hipStream_t st) {
    dim3 grid((N + 15) / 16), block(256);
#define SNX_W4(Z, F) \
    k_w4a16_gemv<MT, Z, F><<<grid, block, 0, st>>>(x, qw, scales, qz, y, bias, M, N, K, G, group)
    if (qz) {
        if (y_f32) SNX_W4(true, true);
        else SNX_W4(true, false);
    } else {
        if (y_f32) SNX_W4(false, true);
        else SNX_W4(false, false);
    }
#undef SNX_W4
    return snx_launch_check("k_w4a16_gemv");
}

// Column gather of the activations: xs[m][k'] = x[m][perm[k']].
__global__ void __launch_bounds__(256) k_gather_cols(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ perm,
                                                     uint16_t* __restrict__ xs, int K, size_t total) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const size_t m = i / (size_t)K;
    const int k = (int)(i - m * (size_t)K);
    int src = perm[k];
    src = src < K ? src : K - 1;
    xs[i] = x[m * K + src];
}

// Packed uint4 column permutation: one output word (8 columns) per thread.
__global__ void __launch_bounds__(256) k_w4_permute_cols(const uint32_t* __restrict__ qw,
                                                         const uint16_t* __restrict__ perm,
                                                         uint32_t* __restrict__ qs, int K,
                                                         size_t words) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= words) return;
    const int k8n = K >> 3;
    const size_t n = i / (size_t)k8n;
    const int w = (int)(i - n * (size_t)k8n);
    const uint32_t* row = qw + n * (size_t)k8n;
    uint32_t out = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        int src = perm[w * 8 + e];
        src = src < K ? src : K - 1;
        out |= ((row[src >> 3] >> (4 * (src & 7))) & 15u) << (4 * e);
    }
    qs[i] = out;
}

// k_w8_gemv1 at K = 1024 SL: the activations staged in LDS (SL * 5 KB; above
// 64 KB from SL = 13 on, which needs the one-time opt-in)
template <int SL>
int launch_w8_gemv1(const float* x, const int8_t* q, const float* s, float* y, const float* bias,
                    size_t N, hipStream_t st) {
    const size_t lds = (size_t)SL * 64 * 20 * sizeof(float);
    if (lds > 64 * 1024) {
        static std::atomic<uint64_t> lds_done{0};
        if (snx::lds_optin(reinterpret_cast<const void*>(&k_w8_gemv1<SL>), (int)lds, lds_done) != hipSuccess) {
            snx_set_error("w8 gemv: cannot reserve %zu bytes of LDS", lds);
            return -1;
        }
    }
    k_w8_gemv1<SL><<<(unsigned)((N + 15) / 16), 1024, lds, st>>>(x, q, s, y, bias, (int)N);
    return snx_launch_check("k_w8_gemv1");
}

}  // namespace

extern "C" {

int snx_w4a16_splitk_span(size_t M, size_t K, int group) {
    if (M < 1 || M > 16 || K % 128 != 0 || group < 128 || (group & (group - 1)) != 0 ||
        K % (size_t)group != 0)
        return 0;
    const size_t steps = K / 128;
    for (size_t d = 8; d >= 1; d--)
        if (steps % d == 0) return (int)(d * 128);
    return 0;
}

int snx_k_w4a16_splitk(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                       const uint32_t* qzeros, float* part, size_t M, size_t N, size_t K,
                       int group, int kspan, void* st) {
    const int G = (int)(K / (size_t)group), gshift = __builtin_ctz((unsigned)group);
    const size_t lds = 16 * ((size_t)kspan * 2 + 16) + (size_t)(kspan / 128) * 16 * 4;
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)(K / (size_t)kspan));
    if (qzeros)
        k_w4a16_splitk<true><<<grid, 256, lds, S(st)>>>(x, qw, scales, qzeros, part, (int)M, (int)N,
                                                        (int)K, G, gshift, kspan);
    else
        k_w4a16_splitk<false><<<grid, 256, lds, S(st)>>>(x, qw, scales, qzeros, part, (int)M, (int)N,
                                                         (int)K, G, gshift, kspan);
    return snx_launch_check("k_w4a16_splitk");
}

int snx_k_w4a16_reduce(const float* part, void* y, int y_f32, int S_, size_t MN, size_t N,
                       const float* bias, void* st) {
    k_w4a16_reduce<<<(unsigned)((MN + 255) / 256), 256, 0, S(st)>>>(part, y, y_f32, S_, MN, (int)N,
                                                                     bias);
    return snx_launch_check("k_w4a16_reduce");
}

int snx_k_gather_cols(const uint16_t* x, const uint16_t* perm, uint16_t* xs, size_t M, size_t K,
                      void* st) {
    const size_t total = M * K;
    k_gather_cols<<<(unsigned)((total + 255) / 256), 256, 0, S(st)>>>(x, perm, xs, (int)K, total);
    return snx_launch_check("k_gather_cols");
}

int snx_k_w4_permute_cols(const uint32_t* qw, const uint16_t* perm, uint32_t* qs, size_t N,
                          size_t K, void* st) {
    const size_t words = N * (K / 8);
    k_w4_permute_cols<<<(unsigned)((words + 255) / 256), 256, 0, S(st)>>>(qw, perm, qs, (int)K, words);
    return snx_launch_check("k_w4_permute_cols");
}

int snx_k_w8_gemv(const float* x, const int8_t* q, const float* s, float* y, const float* bias,
                  size_t M, size_t N, size_t K, void* st) {
    if (M == 1 && K % 1024 == 0 && K <= 16384) {
        switch (K / 1024) {
            case 1: return launch_w8_gemv1<1>(x, q, s, y, bias, N, S(st));
            case 2: return launch_w8_gemv1<2>(x, q, s, y, bias, N, S(st));
            case 3: return launch_w8_gemv1<3>(x, q, s, y, bias, N, S(st));
            case 4: return launch_w8_gemv1<4>(x, q, s, y, bias, N, S(st));
            case 5: return launch_w8_gemv1<5>(x, q, s, y, bias, N, S(st));
            case 6: return launch_w8_gemv1<6>(x, q, s, y, bias, N, S(st));
            case 7: return launch_w8_gemv1<7>(x, q, s, y, bias, N, S(st));
            case 8: return launch_w8_gemv1<8>(x, q, s, y, bias, N, S(st));
            case 9: return launch_w8_gemv1<9>(x, q, s, y, bias, N, S(st));
            case 10: return launch_w8_gemv1<10>(x, q, s, y, bias, N, S(st));
            case 11: return launch_w8_gemv1<11>(x, q, s, y, bias, N, S(st));
            case 12: return launch_w8_gemv1<12>(x, q, s, y, bias, N, S(st));
            case 13: return launch_w8_gemv1<13>(x, q, s, y, bias, N, S(st));
            case 14: return launch_w8_gemv1<14>(x, q, s, y, bias, N, S(st));
            case 15: return launch_w8_gemv1<15>(x, q, s, y, bias, N, S(st));
            default: return launch_w8_gemv1<16>(x, q, s, y, bias, N, S(st));
        }
    }
    if (K % 16 == 0) {
        constexpr int R = 4;
        size_t waves = (N + R - 1) / R;
        k_w8_gemv<R><<<(unsigned)((waves + 3) / 4), 256, 0, S(st)>>>(x, q, s, y, bias, (int)M, (int)N,
                                                                     (int)K);
    } else {
        k_w8_gemv_any<<<(unsigned)((N + 3) / 4), 256, 0, S(st)>>>(x, q, s, y, bias, (int)M, (int)N,
                                                                   (int)K);
    }
    return snx_launch_check("k_w8_gemv");
}

int snx_w4a16_gemv_supported(size_t M, size_t N, size_t K, int group) {
    (void)N;
    return M >= 1 && M <= 64 && K % 512 == 0 && group > 0 && group % 128 == 0 && K % group == 0;
}

size_t snx_w4a16_small_lds(size_t M, size_t K, int perm) {
    size_t lds = M * (K * 2 + 16) + (K / 128) * 16 + 4 * 64 * 16;
    if (perm) lds += M * K * 2 + K * 2;   // raw activations + perm
    return lds;
}

// The streaming M = 1 kernel: group 128, K a multiple of 256 up to 16384,
// scales 16-byte (K = 2048 T) or 4-byte (other K) and qzeros 4-byte aligned.
int snx_w4a16_gemv1_ok(size_t M, size_t K, int group, const void* scales, const void* qzeros) {
    W4Launch a{};
    a.M = (int)M;
    a.K = (int)K;
    a.group = group;
    a.scales = static_cast<const uint16_t*>(scales);
    a.qz = static_cast<const uint32_t*>(qzeros);
    return K <= 16384 && gemv1_ok(a);
}

// The LDS-staged kernel: M <= 4, power-of-two groups, at most 8 items/thread.
int snx_w4a16_small_ok(size_t M, size_t K, int group, int perm) {
    return M >= 1 && M <= 4 && K % 512 == 0 && group >= 128 && (group & (group - 1)) == 0 &&
           K % (size_t)group == 0 && snx_w4a16_small_lds(M, K, perm) <= 65536 &&
           M * (K / 8) <= 8 * 256;
}

// The GLU form of the M = 1 kernel applies: its shapes, with the stacked
// [2F][K] weights within the buffer offsets.
int snx_w4a16_gemv1_swiglu_ok(size_t F, size_t K, int group, const void* scales, const void* qzeros) {
    return F && K % 2048 == 0 && snx_w4a16_gemv1_ok(1, K, group, scales, qzeros) && (uint64_t)F * K < kNoRecord;
}

// M = 1 gate/up projection with the SwiGLU step (the GLU form of the M = 1
// kernel): x bf16 [K], stacked weights [2F][K], out bf16 [F].
int snx_k_w4a16_gemv1_swiglu(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                             const uint32_t* qzeros, const float* bias, uint16_t* out, size_t F,
                             size_t K, int group, void* st) {
    if (!snx_w4a16_gemv1_swiglu_ok(F, K, group, scales, qzeros)) {
        snx_set_error("w4a16 swiglu gemv: F=%zu K=%zu group %d is not an M = 1 kernel shape", F, K, group);
        return -1;
    }
    W4Launch a{x, qw, scales, qzeros, nullptr, out, bias, 0, 1, (int)F, (int)K, (int)(K / 128), group,
               0, S(st)};
    switch (K / 2048) {
        case 1: return launch_gemv1_glu_t<1>(a);
        case 2: return launch_gemv1_glu_t<2>(a);
        case 3: return launch_gemv1_glu_t<3>(a);
        case 4: return launch_gemv1_glu_t<4>(a);
        case 5: return launch_gemv1_glu_t<5>(a);
        case 6: return launch_gemv1_glu_t<6>(a);
        case 7: return launch_gemv1_glu_t<7>(a);
        default: return launch_gemv1_glu_t<8>(a);
    }
}

int snx_k_w4a16_gemv(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                     const uint32_t* qzeros, const uint16_t* perm, void* y, const float* bias,
                     int y_f32, size_t M, size_t N, size_t K, int group, void* st) {
    const int G = (int)(K / (size_t)group);
    const size_t lds = snx_w4a16_small_lds(M, K, perm != NULL);
    const size_t items = M * (K / 8);
    W4Launch a{x, qw, scales, qzeros, perm, y, bias, y_f32, (int)M, (int)N, (int)K, G, group, lds, S(st)};
    if (gemv1_ok(a)) return perm ? launch_gemv1<true>(a) : launch_gemv1<false>(a);
    if (snx_w4a16_small_ok(M, K, group, perm != NULL)) {
        if (perm) {
            if (items <= 2 * 256) return launch_small<2, true>(a);
            if (items <= 4 * 256) return launch_small<4, true>(a);
            return launch_small<8, true>(a);
        }
        if (items <= 2 * 256) return launch_small<2, false>(a);
        if (items <= 4 * 256) return launch_small<4, false>(a);
        return launch_small<8, false>(a);
    }
    if (perm) {
        snx_set_error("w4a16 gemv: column-permuted weights need M <= 4 here (M=%zu)", M);
        return -1;
    }
    if (M <= 16)
        return launch_w4a16<1>(x, qw, scales, qzeros, y, bias, y_f32, (int)M, (int)N, (int)K, G, group, S(st));
    if (M <= 32)
        return launch_w4a16<2>(x, qw, scales, qzeros, y, bias, y_f32, (int)M, (int)N, (int)K, G, group, S(st));
    return launch_w4a16<4>(x, qw, scales, qzeros, y, bias, y_f32, (int)M, (int)N, (int)K, G, group, S(st));
}

size_t snx_w4a16_mt_lds(size_t M, size_t K, int perm) {
    return M * (K * 2 + 16) + 2 * 8 * 64 * 16 + (perm ? K * 2 : 0);
}

int snx_w4a16_mt_ok(size_t M, size_t K, int group, int perm) {
    return M >= 2 && M <= 16 && group == 128 && K % 1024 == 0 && K >= 1024 && K <= 4096 &&
           snx_w4a16_mt_lds(M, K, perm) <= 160 * 1024;
}

int snx_k_w4a16_gemv_mt(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                        const uint32_t* qzeros, const uint16_t* perm, void* y, const float* bias,
                        int y_f32, size_t M, size_t N, size_t K, void* st) {
    if (!snx_w4a16_mt_ok(M, K, 128, perm != NULL)) {
        snx_set_error("w4a16 gemv: M=%zu K=%zu outside the small-M kernel", M, K);
        return -1;
    }
    const int ncu = snx::cu_count();
    const size_t ngroups = (N + 15) / 16;
    const int grid = (int)(ngroups < (size_t)ncu ? ngroups : (size_t)ncu);
    const size_t lds = snx_w4a16_mt_lds(M, K, perm != NULL);
    if (perm)
        return launch_gemv_mt_k<true>(x, qw, scales, qzeros, perm, y, bias, y_f32, (int)M, (int)N, (int)K,
                                      lds, grid, S(st));
    return launch_gemv_mt_k<false>(x, qw, scales, qzeros, perm, y, bias, y_f32, (int)M, (int)N, (int)K,
                                   lds, grid, S(st));
}

int snx_k_w4a16_generic(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                        const uint32_t* qzeros, const int32_t* g_idx, size_t G, void* y,
                        const float* bias, int y_f32, size_t M, size_t N, size_t K, int group,
                        void* st) {
    k_w4a16_generic<<<(unsigned)((N + 3) / 4), 256, 0, S(st)>>>(
        x, qw, scales, qzeros, g_idx, y, bias, y_f32, (int)M, (int)N, (int)K, (int)G, group);
    return snx_launch_check("k_w4a16_generic");
}

}  // extern "C"
