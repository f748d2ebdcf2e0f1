// w4_gemm_kernels.hip - W4A16 prefill GEMM for gfx950 (MFMA-bound, bf16).
//
// y[m][n] = sum_k x[m][k] * (q[n][k] - z[n][g]) * s[n][g],  g = k / group,
// fp32 accumulation, for large M (prefill / continuous batches).
//
//  1. k_w4_prep_x: one pass over the activations writes them in the order
//     the MFMA operands take them (per 128-column step: 16-byte chunks
//     permuted, and {0,4,1,5,2,6,3,7} inside a chunk, the order of the nibble
//     unpack) and the fp32 sums X[t][m] of every 128-column step t.
//  2. k_w4a16_gemm: 128x256 output tiles, 8 waves side by side along N (each
//     128 rows x 32 columns = 4 blocks of v_mfma_f32_32x32x16_bf16, which
//     runs at twice the rate of the 16x16x32 form on gfx950), K step 128.
//     Activation, packed-weight, scale, zero-point and step-sum slices move
//     global->LDS with buffer_load ... lds through a three-stage ring; each wave
//     streams the next-but-one stage in one load per MFMA sub-step.
//     Activation rows are 256 B with 16-byte chunks XOR-swizzled by
//     (row & 15); 64-byte weight rows rotate their chunks by bsw(row); both
//     fragment reads are bank-conflict free.  Nibbles become bf16 (128 + q)
//     with one v_and_or_b32 per pair; each step folds into the fp32 result as
//     y += s * acc (VALU) - X * s * (128 + z) (a rank-1 fp32 MFMA), which
//     removes the bias and zero point exactly.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "codec.h"
#include "launch.h"
#include "../snx_internal.h"

using namespace snx;

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int GBM = 128, GBN = 256, GBK = 128;
constexpr int GLDS_A = GBM * GBK * 2;           // 32 KB of bf16 activations
constexpr int GLDS_B = GBN * GBK / 2;           // 16 KB of packed weights

// ---------------------------------------------------------------- prep pass
// One thread per 8 columns of PREP_ITEMS items: thread t of block b takes
// items 1024 b + 256 i + t (i < 4), all four loads issued before the first
// is used (with one load per thread the pass is bound by load latency, not
// by its bytes).  K % 128 == 0, so the 16 items of one 128-column step are
// 16 consecutive lanes.
constexpr int PREP_ITEMS = 4;

__global__ void __launch_bounds__(256) k_w4_prep_x(const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ xp,
                                                   float* __restrict__ xs, int K, int Mp,
                                                   uint32_t items) {
    // item indices in 32 bits (the host keeps items below 2^31)
    const uint32_t base = blockIdx.x * (256u * PREP_ITEMS) + threadIdx.x;
    const uint32_t k8n = (uint32_t)K >> 3;
    u32x4 v[PREP_ITEMS];
#pragma unroll
    for (int i = 0; i < PREP_ITEMS; i++) {
        const uint32_t it = base + 256u * i;
        v[i] = *reinterpret_cast<const u32x4*>(x + (size_t)(it < items ? it : items - 1) * 8);
    }
#pragma unroll
    for (int i = 0; i < PREP_ITEMS; i++) {
        const uint32_t it = base + 256u * i;
        const bool live = it < items;
        const uint32_t itc = live ? it : items - 1;
        const uint32_t m = itc / k8n;
        const uint32_t k8 = itc - m * k8n;
        u32x4 p;
        p[0] = __builtin_amdgcn_perm(v[i][2], v[i][0], 0x05040100u);
        p[1] = __builtin_amdgcn_perm(v[i][2], v[i][0], 0x07060302u);
        p[2] = __builtin_amdgcn_perm(v[i][3], v[i][1], 0x05040100u);
        p[3] = __builtin_amdgcn_perm(v[i][3], v[i][1], 0x07060302u);
        // input chunk 8 h + s of its 128-column step goes to chunk 2 s + h
        const uint32_t jin = k8 & 15, jout = 2 * (jin & 7) + (jin >> 3);
        if (live) *reinterpret_cast<u32x4*>(xp + (size_t)(itc - jin + jout) * 8) = p;
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++)
            sum += __builtin_bit_cast(float, v[i][e] << 16) + __builtin_bit_cast(float, v[i][e] & 0xFFFF0000u);
        sum += __shfl_xor(sum, 8);
        sum += __shfl_xor(sum, 4);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 1);
        if (live && (k8 & 15) == 0) xs[(size_t)(k8 >> 4) * (uint32_t)Mp + m] = sum;
    }
}

// ----------------------------------------------------------------- the GEMM
constexpr int W4_WN = 8;   // waves along N (8 / W4_WN along M)
constexpr int W4_GROUP_M = 8;   // rows of tiles per band of the tile order
// LDS ring of three stages (one K step of 128 columns each):
//   A   128 rows x 256 B  bf16 activations, chunk c of row r at c ^ (r & 15)
//   B   256 rows x 64 B   packed weights,   chunk c of row r at c ^ bsw(r)
//   X   128 fp32          step sums of the tile's rows
//   S   256 u32           fp16 scale pair (g & ~1, g | 1) of every tile column
//   Z   256 u32           zero-point word of every tile column
// Every wave issues exactly 8 direct loads per stage, so "stage kt landed"
// is vmcnt(8) while stage kt + 1 is still in flight.
constexpr int GOFF_B = GLDS_A, GOFF_X = GOFF_B + GLDS_B, GOFF_S = GOFF_X + GBM * 4;
constexpr int GOFF_Z = GOFF_S + GBN * 4, GRING = GOFF_Z + GBN * 4;
constexpr int GSTAGES = 3;

// 64-byte weight rows: rows 2 and 4 apart share banks, so each row's four
// 16-byte chunks rotate by bits 1-3 of the row (conflict-free 16-lane reads)
__device__ __forceinline__ int bsw(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

// The MFMAs see weights 128 + q (bf16 of the nibble), so each 128-column
// step t gives acc_t = sum_k x[m][k] (128 + q[n][k]) and
//   y[m][n] = sum_t (s_t[n] acc_t[m][n] - X_t[m] c_t[n]),
//   X_t[m] = sum of x[m][k] over step t,  c_t[n] = s_t[n] (128 + z_t[n]).
// Per step, s_t acc_t is one VALU FMA per element and the rank-1 term
// X_t c_t goes to the matrix cores: one v_mfma_f32_32x32x1_f32 (two 32x32
// outer products) per pair of result blocks, accumulating in fp32.
//
// Products use v_mfma_f32_32x32x16_bf16 (operand lane l: row / column l % 32,
// k = 8 (l / 32) + e; result value v of lane l: row 8 (v / 4) + 4 (l / 32) +
// v % 4, column l % 32).  Sub-step s of a step takes packed word 8 h + s of
// each weight column in lanes with h = l / 32, so a lane's eight words for the
// step are 32 contiguous bytes; the prep pass stores the activations to match
// (chunk 2 s + h of a prepared row = original columns of word 8 h + s).
// SWIGLU: the weights are a stacked [2F][K] gate/up projection and the output
// is [M][F] = bf16(silu(gate) * up) (N = F).  Tile column c < 128 is gate
// column n0 + c, column c >= 128 the up column F + n0 + c - 128 of the same
// output column, so waves 0-3 hold gate values and waves 4-7 the matching up
// values; the epilogue pairs them through LDS.
// PREP (SwiGLU only): the output is written as the next projection's
// prepared input instead of plain rows (a SwiGLU MLP's down projection reads
// exactly silu(gate) * up): tile column block tn is that projection's
// 128-column step tn, so y takes the bf16 values in the prep pass's slot
// order and `part`, read as float [F / 128][Mp], the step sums, summed in
// the prep pass's order (bit-identical to running the prep pass on the plain
// rows).
// SPLIT > 1 (too few tiles to fill the CUs, such as the QKV projection of one
// GPU's tensor-parallel shard, or the tiles past the last full round of
// CUs): workgroup unit v covers tile tile0 + v % ntiles and
// the K steps of span v / ntiles (K / SPLIT columns).  Each wave stores its
// span's fp32 results to its slot of `part` (system-coherent policy, so no
// L2 keeps a copy another XCD cannot see), waits until they are written and
// counts itself in cnt[tile][wave]; the last of the SPLIT waves of a
// (tile, wave) adds the slots in span order (the same fp32 sums whichever
// wave is last), returns the counter to 0 and writes the output.  No wave
// waits for another.
template <bool ZEROS, bool YF32, int WN, bool SWIGLU, int SPLIT = 1, bool PREP = false>
__global__ void __launch_bounds__(512) k_w4a16_gemm(const uint16_t* __restrict__ xp,
                                                    const float* __restrict__ xs,
                                                    const uint32_t* __restrict__ qw,
                                                    const uint16_t* __restrict__ scales,
                                                    const uint32_t* __restrict__ qz,
                                                    void* __restrict__ y,
                                                    const float* __restrict__ bias, int M, int N,
                                                    int K, int G, int gshift, int Mp, int tiles_m,
                                                    u32x4* __restrict__ part, uint32_t* __restrict__ cnt,
                                                    int tile0) {
    static_assert(SPLIT == 1 || !SWIGLU, "the SwiGLU epilogue takes whole-K tiles");
    static_assert(!PREP || (SWIGLU && !YF32), "the prepared output is the SwiGLU form's bf16 rows");
    // WN waves along N, 8 / WN along M: each wave owns RW rows x CW columns,
    // FM x FN blocks of 32 x 32; the result sits in FM / 2 x FN pairs of
    // blocks stacked along M (the 2-block f32 MFMA's output)
    constexpr int WM = 8 / WN, RW = GBM / WM, CW = GBN / WN, FM = RW / 32, FN = CW / 32;
    constexpr int QM = FM / 2;
    static_assert(FM % 2 == 0 && FN >= 1, "wave tile must hold pairs of 32-row blocks");
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int r32 = lane & 31, h = lane >> 5;

    // XCD-aware order: consecutive units share an XCD
    const int b = blockIdx.x, nb = gridDim.x;
    const int unit = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
    // this launch covers tiles tile0 .. tile0 + ntiles - 1 (the span
    // partials and counters are indexed by the launch's own tile number)
    const int ntiles = nb / SPLIT;
    const int tile = SPLIT == 1 ? unit : unit % ntiles, span = SPLIT == 1 ? 0 : unit / ntiles;
    // tile t -> (tm, tn) in bands of W4_GROUP_M rows of tiles, M fastest
    // within a band: the ~32 tiles an XCD runs at once span 8 activation row
    // blocks and ~4 weight column blocks, so every K step's slices are
    // shared by several of them in the XCD's L2 (row-major order over all
    // 15 row blocks of T = 1849 shared each activation slice by only ~2)
    int tm, tn;
    {
        const int tiles_n = (N + (SWIGLU ? GBN / 2 : GBN) - 1) / (SWIGLU ? GBN / 2 : GBN);
        const int t = tile0 + tile, band = W4_GROUP_M * tiles_n, g = t / band, r = t - g * band;
        const int gm = tiles_m - g * W4_GROUP_M < W4_GROUP_M ? tiles_m - g * W4_GROUP_M : W4_GROUP_M;
        tm = g * W4_GROUP_M + r % gm;
        tn = r / gm;
    }
    const int m0 = tm * GBM, n0 = tn * (SWIGLU ? GBN / 2 : GBN);
    // weight row of tile column c (clamped into the matrix)
    auto wcol = [&](int c) -> int {
        if (!SWIGLU) return n0 + c < N ? n0 + c : N - 1;
        const int o = n0 + (c & (GBN / 2 - 1)) < N ? n0 + (c & (GBN / 2 - 1)) : N - 1;
        return c < GBN / 2 ? o : N + o;
    };

    // direct-load sources (byte offsets; operands < 4 GiB).  A: wave w,
    // instruction i fills 1 KB block 8 i + w = tile rows 4 blk .. 4 blk + 3,
    // lane -> (row, LDS chunk)
    const uint32_t krow = (uint32_t)K * 2;      // bytes per activation row
    const uint32_t wrowb = (uint32_t)K / 2;     // bytes per packed weight row
    uint32_t ga[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = (8 * i + wave) * 4 + (lane >> 4);
        const int gr = m0 + row < M ? m0 + row : M - 1;
        const int chunk = (lane & 15) ^ (row & 15);
        ga[i] = (uint32_t)gr * krow + (uint32_t)chunk * 16u;
    }
    // W: 16 rows per 1 KB block, 4 lanes per 64-byte row
    uint32_t gw[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int row = (8 * i + wave) * 16 + (lane >> 2);
        const int gn = wcol(row);
        gw[i] = (uint32_t)gn * wrowb + (uint32_t)((lane & 3) ^ bsw(row)) * 16u;
    }
    // scales (waves 0-3) or zero words (waves 4-7) of tile column 64 (w&3) + lane;
    // without zero points waves 4-7 repeat the scale load (same bytes, same slot)
    const int sn = wcol(64 * (wave & 3) + lane);
    const bool zload = ZEROS && wave >= 4;
    const int zw = (G + 7) >> 3;
    // buffer resources: buffer_load ... lds is counted by vmcnt alone, so
    // LDS fragment reads stay in flight while the loads of later stages fly
    // (global_load_lds also counts in lgkmcnt and forces lgkmcnt(0) waits)
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void*)xp, (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)qw, (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)(ZEROS ? (const void*)qz : (const void*)scales),
                                                                        (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc((void*)scales, (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t rxs = __builtin_amdgcn_make_buffer_rsrc((void*)xs, (short)0, -1, 0x00020000);
    const uint32_t zoff = (uint32_t)sn * (uint32_t)zw * 4u, soff = (uint32_t)sn * (uint32_t)G * 2u;
    const uint32_t xsoff = (uint32_t)(m0 + (wave & 1) * 64 + lane) * 4u;
    // load p (0..7) of the eight each wave issues for stage kt into ring slot buf
    auto dpart = [&](int buf, int kt, int p) {
        uint8_t* base = lds + buf * GRING;
        if (p < 4) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(base + (8 * p + wave) * 1024), 16, ga[p],
                                                     kt * (GBK * 2), 0, 0);
        } else if (p < 6) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_ptr_t)(base + GOFF_B + (8 * (p - 4) + wave) * 1024), 16,
                                                     gw[p - 4], kt * (GBK / 2), 0, 0);
        } else if (p == 6) {
            const int g = (kt * GBK) >> gshift;
            if (zload)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(base + GOFF_Z + 256 * (wave & 3)), 4,
                                                         zoff + (uint32_t)(g >> 3) * 4u, 0, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsc, (lds_ptr_t)(base + GOFF_S + 256 * (wave & 3)), 4,
                                                         soff + (uint32_t)(g & ~1) * 2u, 0, 0, 0);
        } else {
            // step sums of the tile's 128 rows (each half loaded by four waves)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rxs, (lds_ptr_t)(base + GOFF_X + (wave & 1) * 256), 4, xsoff,
                                                     kt * Mp * 4, 0, 0);
        }
    };
    auto dload = [&](int buf, int kt) {
#pragma unroll
        for (int p = 0; p < 8; p++) dpart(buf, kt, p);
    };

    f32x32 yq[QM][FN];
#pragma unroll
    for (int i = 0; i < QM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) yq[i][j] = f32x32{};

    uint32_t nib_mask, bf_bias;
    asm volatile("s_mov_b32 %0, 0xf000f" : "=s"(nib_mask));
    asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(bf_bias));

    const int nk = K / GBK / SPLIT, kb = span * nk;   // this unit's K steps: kb .. kb + nk - 1
    // activation fragment: row wm RW + 32 i + r32, logical chunk 2 s + h
    // (rows 16 apart share the swizzle, so row & 15 = r32 & 15)
    const uint8_t* arow = lds + (wm * RW + r32) * (GBK * 2);
    // weight words 8 h .. 8 h + 7 of column wn CW + 32 j + r32 = chunks 2 h, 2 h + 1
    const int brow = wn * CW + r32;
    const uint8_t* wrow0 = lds + GOFF_B + brow * (GBK / 2) + (((2 * h) ^ bsw(brow)) << 4);
    const uint8_t* wrow1 = lds + GOFF_B + brow * (GBK / 2) + (((2 * h + 1) ^ bsw(brow)) << 4);

    // fold one 128-column step into the result: y += s * acc - X (s (128 + z))
    auto fold = [&](const f32x16 (&acc)[FM][FN], const float* xr, const uint32_t* sr,
                    const uint32_t* zr, int g) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const uint16_t hs = (uint16_t)(sr[j] >> (16 * (g & 1)));
            const float sf = (float)__builtin_bit_cast(_Float16, hs);
            const uint32_t z = ZEROS ? (zr[j] >> (4 * (g & 7))) & 15u : 8u;
            const float nc = -sf * (float)(128u + z);
#pragma unroll
            for (int i = 0; i < QM; i++) {
                yq[i][j] = __builtin_amdgcn_mfma_f32_32x32x1f32(xr[i], nc, yq[i][j], 0, 0, 0);
#pragma unroll
                for (int u = 0; u < 2; u++)
#pragma unroll
                    for (int e = 0; e < 16; e++)
                        yq[i][j][16 * u + e] = __builtin_fmaf(sf, acc[2 * i + u][j][e], yq[i][j][16 * u + e]);
            }
        }
    };

    uint32_t sr[FN], zr[FN];
    float xr[QM];
    f32x16 acc[FM][FN];
    dload(0, kb);
    dload(1, kb + (nk > 1 ? 1 : 0));
    for (int kt = kb; kt < kb + nk; kt++) {
        const int cur = (kt - kb) % GSTAGES;
        // vmcnt(8): stage kt landed, kt + 1 may fly; lgkmcnt(0): this wave is
        // done with stage kt - 1.  A raw barrier: a __syncthreads() fence would
        // wait for stage kt + 1 as well.
        __builtin_amdgcn_s_waitcnt(0x0078);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);    // nothing below moves above the wait
        const int kn = kt + 2 < kb + nk ? kt + 2 : kb + nk - 1;   // past the end: reload, unused
        const int nbuf = (kt - kb + 2) % GSTAGES;

        const uint8_t* ab = arow + cur * GRING;
        u32x4 wv[FN][2];
#pragma unroll
        for (int j = 0; j < FN; j++) {
            wv[j][0] = *reinterpret_cast<const u32x4*>(wrow0 + cur * GRING + j * 32 * (GBK / 2));
            wv[j][1] = *reinterpret_cast<const u32x4*>(wrow1 + cur * GRING + j * 32 * (GBK / 2));
        }
#pragma unroll
        for (int s = 0; s < 8; s++) {
            bf16x8 fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; i++)
                fa[i] = *reinterpret_cast<const bf16x8*>(ab + i * 32 * (GBK * 2) +
                                                          (((2 * s + h) ^ (r32 & 15)) << 4));
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const uint32_t w = wv[j][s >> 2][s & 3];
                u32x4 bq;
                bq[0] = (w & nib_mask) | bf_bias;
                bq[1] = ((w >> 4) & nib_mask) | bf_bias;
                bq[2] = ((w >> 8) & nib_mask) | bf_bias;
                bq[3] = ((w >> 12) & nib_mask) | bf_bias;
                fb[j] = __builtin_bit_cast(bf16x8, bq);
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        fa[i], fb[j], s == 0 ? f32x16{} : acc[i][j], 0, 0, 0);
            // stage kt + 2 streams in one load per sub-step, between the MFMAs
            dpart(nbuf, kn, s);
        }
        // this step's sums, scales and zero words; the 2-block f32 MFMA takes
        // row 64 i + lane of the wave's rows
        const uint8_t* st = lds + cur * GRING;
#pragma unroll
        for (int i = 0; i < QM; i++)
            xr[i] = reinterpret_cast<const float*>(st + GOFF_X)[wm * RW + 64 * i + lane];
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int c = wn * CW + j * 32 + r32;
            sr[j] = reinterpret_cast<const uint32_t*>(st + GOFF_S)[c];
            zr[j] = ZEROS ? reinterpret_cast<const uint32_t*>(st + GOFF_Z)[c] : 0u;
        }
        fold(acc, xr, sr, zr, (kt * GBK) >> gshift);
    }
    __builtin_amdgcn_s_waitcnt(0x0070);   // the ring's last (unused) loads drain before exit

    bool last = true;                     // this wave writes its results (SPLIT: the last span to arrive)
    if constexpr (SPLIT > 1) {
        // slot (unit, wave): QM x FN results x 8 pieces of 16 B per lane, lane-major
        constexpr int NP = QM * FN * 8, SLOTB = NP * 64 * 16;
        constexpr int kSysCoherent = 1 | 16;          // buffer cache policy sc0 sc1
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
            (void*)part, (short)0, nb * 8 * SLOTB, 0x00020000);
        const uint32_t mine = (uint32_t)((span * ntiles + tile) * 8 + wave) * SLOTB;
#pragma unroll
        for (int i = 0; i < QM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int p = 0; p < 8; p++) {
                    // elements copied to scalars first: a bit cast of a vector
                    // element operand reads the wrong element with this compiler
                    const float f0 = yq[i][j][4 * p], f1 = yq[i][j][4 * p + 1];
                    const float f2 = yq[i][j][4 * p + 2], f3 = yq[i][j][4 * p + 3];
                    const u32x4 v = {__builtin_bit_cast(uint32_t, f0), __builtin_bit_cast(uint32_t, f1),
                                     __builtin_bit_cast(uint32_t, f2), __builtin_bit_cast(uint32_t, f3)};
                    __builtin_amdgcn_raw_buffer_store_b128(v, rp, lane * 16,
                                                           mine + ((i * FN + j) * 8 + p) * 1024, kSysCoherent);
                }
        // the slot is written before it is counted, and no result register is
        // written before the stores have read it (a 16-byte store reads its
        // data after issue): nothing below moves above this wait
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0x0f70);           // vmcnt(0)
        __builtin_amdgcn_sched_barrier(0);
        uint32_t c = 0;
        if (lane == 0) c = atomicAdd(&cnt[tile * 8 + wave], 1u);
        last = __builtin_amdgcn_readfirstlane(c) == SPLIT - 1;
      if (last) {
        // the last wave of this (tile, wave): the spans' slots in span order, in
        // chunks of 4 pieces x SPLIT spans, each chunk's offsets carrying a zero
        // the previous chunk's sums produce (so the loads cannot all be hoisted)
        const uint32_t first = (uint32_t)(tile * 8 + wave) * SLOTB, sstride = (uint32_t)ntiles * 8 * SLOTB;
        uint32_t dep = 0;
#pragma unroll
        for (int i = 0; i < QM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int p0 = 0; p0 < 8; p0 += 4) {
                    u32x4 v[SPLIT][4];
#pragma unroll
                    for (int s2 = 0; s2 < SPLIT; s2++)
#pragma unroll
                        for (int pp = 0; pp < 4; pp++)
                            v[s2][pp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                rp, lane * 16, first + dep + s2 * sstride + ((i * FN + j) * 8 + p0 + pp) * 1024,
                                kSysCoherent));
#pragma unroll
                    for (int pp = 0; pp < 4; pp++)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const uint32_t w0 = v[0][pp][e];
                            float r = __builtin_bit_cast(float, w0);
#pragma unroll
                            for (int s2 = 1; s2 < SPLIT; s2++) {
                                const uint32_t w = v[s2][pp][e];
                                r += __builtin_bit_cast(float, w);
                            }
                            yq[i][j][4 * (p0 + pp) + e] = r;
                        }
                    const f32x16 ch = __builtin_shufflevector(yq[i][j], yq[i][j], 0, 1, 2, 3, 4, 5, 6, 7, 8, 9,
                                                              10, 11, 12, 13, 14, 15);
                    const f32x16 cl = __builtin_shufflevector(yq[i][j], yq[i][j], 16, 17, 18, 19, 20, 21, 22, 23,
                                                              24, 25, 26, 27, 28, 29, 30, 31);
                    asm volatile("s_mov_b32 %0, 0" : "=s"(dep) : "v"(p0 == 0 ? ch : cl));
                }
        if (lane == 0) atomicExch(&cnt[tile * 8 + wave], 0u);   // ready for the next call
      }
    }

    if constexpr (!SWIGLU) {
        // 16-byte aligned output rows: each wave stages its RW x CW results in a
        // private LDS region (after a barrier: every wave is past the ring and
        // every direct load has landed) and writes them back as 16-byte row
        // pieces, instead of one 2- or 4-byte store per value.  A wave reads
        // back only what it wrote, so no barrier sits between the two.
        constexpr int EB = YF32 ? 4 : 2, RB = CW * EB + 16, PPR = CW * EB / 16;
        static_assert(8 * RW * RB <= GSTAGES * GRING, "the staged results fit in the ring");
        if ((reinterpret_cast<uintptr_t>(y) & 15) == 0 && N % (16 / EB) == 0) {
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_s_barrier();
            if (!last) return;
            uint8_t* reg = lds + wave * (RW * RB);
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int n = n0 + wn * CW + j * 32 + r32;
                const float bv = bias && n < N ? bias[n] : 0.0f;
#pragma unroll
                for (int i = 0; i < QM; i++)
#pragma unroll
                    for (int u = 0; u < 2; u++)
#pragma unroll
                        for (int v = 0; v < 16; v++) {
                            const int row = 32 * (2 * i + u) + 8 * (v >> 2) + 4 * h + (v & 3);
                            const float val = yq[i][j][16 * u + v] + bv;
                            if (YF32)
                                *reinterpret_cast<float*>(reg + row * RB + (j * 32 + r32) * 4) = val;
                            else
                                *reinterpret_cast<uint16_t*>(reg + row * RB + (j * 32 + r32) * 2) = bf16_out(val);
                        }
            }
#pragma unroll
            for (int t = 0; t < RW * PPR / 64; t++) {
                const int q = t * 64 + lane, row = q / PPR, pc = q % PPR;
                const int m = m0 + wm * RW + row, n = n0 + wn * CW + pc * (16 / EB);
                const u32x4 val = *reinterpret_cast<const u32x4*>(reg + row * RB + pc * 16);
                if (m < M && n < N)
                    *reinterpret_cast<u32x4*>(reinterpret_cast<uint8_t*>(y) + ((size_t)m * N + n) * EB) = val;
            }
            return;
        }
        if (!last) return;
    }

    if constexpr (SWIGLU) {
        static_assert(WN == 8 && FN == 1 && RW == GBM, "SwiGLU pairs wave w with wave w + 4");
        // every wave is done with the ring: reuse it for the fp32 gate and up
        // tiles, [256 tile columns][GBM rows + 1] (the pad spreads the banks)
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_s_barrier();
        constexpr int XS = GBM + 1;
        float* ex = reinterpret_cast<float*>(lds);
        const int c = wn * CW + r32;                            // tile column 0..255
        const float bv = bias ? bias[wcol(c)] : 0.0f;
#pragma unroll
        for (int i = 0; i < QM; i++)
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    ex[c * XS + 32 * (2 * i + u) + 8 * (v >> 2) + 4 * h + (v & 3)] = yq[i][0][16 * u + v] + bv;
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_s_barrier();
        if constexpr (PREP) {
            // wave w: output rows 16 w .. 16 w + 15, four per pass; lane l
            // takes the 8 columns of chunk j = l % 16 of row 16 w + 4 p + l / 16.
            // The 16 lanes of a row are the 16 threads of one step in the prep
            // pass (same chunk sums, same xor butterfly), and chunk j goes to
            // slot chunk 2 (j % 8) + j / 8 with its values in the order
            // {0,4,1,5,2,6,3,7}.  Host: F % 128 == 0, rows 16-byte aligned.
            const int j = lane & 15, jout = 2 * (j & 7) + (j >> 3);
            uint16_t* xo = static_cast<uint16_t*>(y);
            float* so = reinterpret_cast<float*>(part);
            const int step = n0 / (GBN / 2);
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const int row = 16 * wave + 4 * p + (lane >> 4), m = m0 + row;
                uint32_t a[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int oc = 8 * j + e;
                    a[e] = bf16_out(silu_mul_fast(ex[oc * XS + row], ex[(oc + GBN / 2) * XS + row]));
                }
                float sum = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    sum += __builtin_bit_cast(float, a[2 * e] << 16) + __builtin_bit_cast(float, a[2 * e + 1] << 16);
                sum += __shfl_xor(sum, 8);
                sum += __shfl_xor(sum, 4);
                sum += __shfl_xor(sum, 2);
                sum += __shfl_xor(sum, 1);
                if (m < M) {
                    const u32x4 pk = {a[0] | a[4] << 16, a[1] | a[5] << 16, a[2] | a[6] << 16, a[3] | a[7] << 16};
                    *reinterpret_cast<u32x4*>(xo + (size_t)m * N + (size_t)step * (GBN / 2) + jout * 8) = pk;
                    if (j == 0) so[(size_t)step * Mp + m] = sum;
                }
            }
            return;
        }
        // wave w: output rows 16 w .. 16 w + 15, two columns per lane
        const int oc = 2 * (lane & 63);                         // output column pair 0..126
        const int n = n0 + oc;
#pragma unroll 4
        for (int r = 0; r < 16; r++) {
            const int row = 16 * wave + r, m = m0 + row;
            const float g0 = ex[oc * XS + row], g1 = ex[(oc + 1) * XS + row];
            const float u0 = ex[(oc + GBN / 2) * XS + row], u1 = ex[(oc + 1 + GBN / 2) * XS + row];
            const uint32_t packed = (uint32_t)bf16_out(silu_mul_fast(g0, u0)) |
                                    (uint32_t)bf16_out(silu_mul_fast(g1, u1)) << 16;
            if (m < M && n + 1 < N)
                *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(y) + (size_t)m * N + n) = packed;
            else if (m < M && n < N)
                reinterpret_cast<uint16_t*>(y)[(size_t)m * N + n] = (uint16_t)packed;
        }
        return;
    }

    // value 16 u + v of pair (i, j), lane l: block (2 i + u, j), row
    // 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32
#pragma unroll
    for (int i = 0; i < QM; i++) {
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int n = n0 + wn * CW + j * 32 + r32;
            if (n >= N) continue;
            const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int m = m0 + wm * RW + 32 * (2 * i + u) + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (m >= M) continue;
                    if (YF32)
                        reinterpret_cast<float*>(y)[(size_t)m * N + n] = yq[i][j][16 * u + v] + bv;
                    else
                        reinterpret_cast<uint16_t*>(y)[(size_t)m * N + n] = bf16_out(yq[i][j][16 * u + v] + bv);
                }
        }
    }
}

// Launches tiles [tile0, tile0 + count) of the tile grid (all of it when
// count < 0) in SPLIT K spans.
template <bool ZEROS, bool YF32, int WN, bool SWIGLU, int SPLIT>
int launch_w4_gemm_s(const uint16_t* xp, const float* xs, const uint32_t* qw,
                     const uint16_t* scales, const uint32_t* qz, void* y, const float* bias, int M,
                     int N, int K, int group, int Mp, void* part, uint32_t* cnt, hipStream_t st,
                     int tile0 = 0, int count = -1) {
    const int tn_cols = SWIGLU ? GBN / 2 : GBN;
    const int tiles_m = (M + GBM - 1) / GBM, tiles_n = (N + tn_cols - 1) / tn_cols;
    const int ntiles = count < 0 ? tiles_m * tiles_n : count;
    const size_t lds = (size_t)GSTAGES * GRING;
    static std::atomic<uint64_t> lds_done{0};   // > 64 KB of LDS per workgroup, per device
    const void* kfn = reinterpret_cast<const void*>(&k_w4a16_gemm<ZEROS, YF32, WN, SWIGLU, SPLIT>);
    if (snx::lds_optin(kfn, (int)lds, lds_done) != hipSuccess) {
        snx_set_error("w4a16 gemm: cannot reserve %zu bytes of LDS", lds);
        return -1;
    }
    const int gshift = __builtin_ctz((unsigned)group);
    k_w4a16_gemm<ZEROS, YF32, WN, SWIGLU, SPLIT><<<ntiles * SPLIT, 512, lds, st>>>(
        xp, xs, qw, scales, qz, y, bias, M, N, K, K / group, gshift, Mp, tiles_m,
        static_cast<u32x4*>(part), cnt, tile0);
    return snx_launch_check("k_w4a16_gemm");
}

template <bool ZEROS, bool YF32, int WN, bool SWIGLU>
int launch_w4_gemm(const uint16_t* xp, const float* xs, const uint32_t* qw,
                   const uint16_t* scales, const uint32_t* qz, void* y, const float* bias, int M,
                   int N, int K, int group, int Mp, int split, void* part, uint32_t* cnt, hipStream_t st) {
    if constexpr (!SWIGLU) {
        if (split == 4)
            return launch_w4_gemm_s<ZEROS, YF32, WN, false, 4>(xp, xs, qw, scales, qz, y, bias, M, N, K, group, Mp,
                                                               part, cnt, st);
        if (split == 2) {
            const int ntiles = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN), ncu = snx::cu_count();
            if (ntiles > ncu) {
                // the full rounds whole-K, the remaining tiles (at most half a
                // round) in two spans on twice as many workgroups
                const int full = ntiles - ntiles % ncu;
                const int rc = launch_w4_gemm_s<ZEROS, YF32, WN, false, 1>(xp, xs, qw, scales, qz, y, bias, M, N, K,
                                                                           group, Mp, nullptr, nullptr, st, 0, full);
                if (rc) return rc;
                return launch_w4_gemm_s<ZEROS, YF32, WN, false, 2>(xp, xs, qw, scales, qz, y, bias, M, N, K, group,
                                                                   Mp, part, cnt, st, full, ntiles - full);
            }
            return launch_w4_gemm_s<ZEROS, YF32, WN, false, 2>(xp, xs, qw, scales, qz, y, bias, M, N, K, group, Mp,
                                                               part, cnt, st);
        }
    }
    return launch_w4_gemm_s<ZEROS, YF32, WN, SWIGLU, 1>(xp, xs, qw, scales, qz, y, bias, M, N, K, group, Mp,
                                                         nullptr, nullptr, st);
}

// SiLU(gate) * up between the gate/up and down projections of a SwiGLU MLP:
// gu [T][2F] bf16 (gate in columns [0, F), up in [F, 2F)), out [T][F] bf16,
// out = bf16(g / (1 + exp(-g)) * u) in fp32.  One thread per 8 columns.
// Both kernels below call this one out-of-line function, so the fused
// quantizer sees exactly the bf16 values k_silu_mul writes.
__device__ __attribute__((noinline)) uint32_t silu_mul_pair(uint32_t gv, uint32_t uv) {
    const float g0 = __builtin_bit_cast(float, gv << 16), g1 = __builtin_bit_cast(float, gv & 0xFFFF0000u);
    const float u0 = __builtin_bit_cast(float, uv << 16), u1 = __builtin_bit_cast(float, uv & 0xFFFF0000u);
    const float r0 = g0 / (1.0f + expf(-g0)) * u0;
    const float r1 = g1 / (1.0f + expf(-g1)) * u1;
    return (uint32_t)bf16_out(r0) | (uint32_t)bf16_out(r1) << 16;
}

__global__ void __launch_bounds__(256) k_silu_mul(const uint16_t* __restrict__ gu,
                                                  uint16_t* __restrict__ out, int F, size_t items) {
    const size_t it = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (it >= items) return;
    const int f8n = F >> 3;
    const size_t t = it / (size_t)f8n;
    const int f = (int)(it - t * (size_t)f8n) * 8;
    const u32x4 gv = *reinterpret_cast<const u32x4*>(gu + t * (size_t)(2 * F) + f);
    const u32x4 uv = *reinterpret_cast<const u32x4*>(gu + t * (size_t)(2 * F) + F + f);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = silu_mul_pair(gv[e], uv[e]);
    *reinterpret_cast<u32x4*>(out + t * (size_t)F + f) = o;
}

// fp32 gate/up [T][2F] -> bf16(silu(g) * u) [T][F], the rule of the fused
// SwiGLU epilogue (silu_mul_fast); one thread per 8 columns.
__global__ void __launch_bounds__(256) k_silu_mul_f32(const float* __restrict__ gu,
                                                      uint16_t* __restrict__ out, int F, size_t items) {
    const size_t it = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (it >= items) return;
    const int f8n = F >> 3;
    const size_t t = it / (size_t)f8n;
    const int f = (int)(it - t * (size_t)f8n) * 8;
    const float* g = gu + t * (size_t)(2 * F) + f;
    const float* u = g + F;
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++)
        o[e] = (uint32_t)bf16_out(silu_mul_fast(g[2 * e], u[2 * e])) |
               (uint32_t)bf16_out(silu_mul_fast(g[2 * e + 1], u[2 * e + 1])) << 16;
    *reinterpret_cast<u32x4*>(out + t * (size_t)F + f) = o;
}

// SwiGLU followed by the per-token int8 quantizer of the W8A8 down
// projection, one workgroup per token: the bf16 SwiGLU row goes to LDS, a
// block reduction gives max|h|, and the codes follow the reference's
// per-row rule (quantize_int8.c:157-177: scale = max/127, or 1 below
// FLT_MIN; q = clamp(roundf(h * (1/scale)), -128, 127)) applied to the bf16
// values.  F % 8 == 0, F <= 32768 (64 KB of LDS).
__global__ void __launch_bounds__(256) k_silu_mul_quant_int8(const uint16_t* __restrict__ gu,
                                                             int8_t* __restrict__ q,
                                                             float* __restrict__ scales, int F) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint32_t* hrow = reinterpret_cast<uint32_t*>(smem);       // F/2 words of bf16 pairs
    __shared__ float red[4];
    const size_t t = blockIdx.x;
    const uint16_t* g = gu + t * (size_t)(2 * F);
    const int f8n = F >> 3;
    float m = 0.0f;
    for (int c = threadIdx.x; c < f8n; c += 256) {
        const u32x4 gv = *reinterpret_cast<const u32x4*>(g + c * 8);
        const u32x4 uv = *reinterpret_cast<const u32x4*>(g + F + c * 8);
        u32x4 h;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            h[e] = silu_mul_pair(gv[e], uv[e]);
            // the scan skips NaN like the reference's `a > max_abs`
            const float a0 = fabsf(__builtin_bit_cast(float, h[e] << 16));
            const float a1 = fabsf(__builtin_bit_cast(float, h[e] & 0xFFFF0000u));
            m = a0 > m ? a0 : m;
            m = a1 > m ? a1 : m;
        }
        *reinterpret_cast<u32x4*>(hrow + c * 4) = h;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(m, o);
        m = v > m ? v : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < 4; w++) m = red[w] > m ? red[w] : m;
    const float s = m < FLT_MIN ? 1.0f : m / 127.0f;
    const float inv = 1.0f / s;
    if (threadIdx.x == 0) scales[t] = s;
    int8_t* qr = q + t * (size_t)F;
    for (int c = threadIdx.x; c < f8n; c += 256) {
        const u32x4 h = *reinterpret_cast<const u32x4*>(hrow + c * 4);
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int32_t c0 = clampi(round_i32(__builtin_bit_cast(float, h[e] << 16) * inv), -128, 127);
            const int32_t c1 = clampi(round_i32(__builtin_bit_cast(float, h[e] & 0xFFFF0000u) * inv), -128, 127);
            const uint32_t pair = ((uint32_t)c0 & 0xFFu) | (((uint32_t)c1 & 0xFFu) << 8);
            if (e < 2) lo |= pair << (16 * e);
            else hi |= pair << (16 * (e - 2));
        }
        *reinterpret_cast<uint2*>(qr + c * 8) = make_uint2(lo, hi);
    }
}

}  // namespace

extern "C" {

int snx_k_silu_mul_f32(const float* gu, uint16_t* out, size_t T, size_t F, void* st) {
    const size_t items = T * (F / 8);
    k_silu_mul_f32<<<(unsigned)((items + 255) / 256), 256, 0, S(st)>>>(gu, out, (int)F, items);
    return snx_launch_check("k_silu_mul_f32");
}

int snx_k_silu_mul(const uint16_t* gu, uint16_t* out, size_t T, size_t F, void* st) {
    const size_t items = T * (F / 8);
    k_silu_mul<<<(unsigned)((items + 255) / 256), 256, 0, S(st)>>>(gu, out, (int)F, items);
    return snx_launch_check("k_silu_mul");
}

int snx_k_silu_mul_quant_int8(const uint16_t* gu, int8_t* q, float* scales, size_t T, size_t F,
                              void* st) {
    if (F > 32768 || T > 0x7fffffff) {
        snx_set_error("silu_mul_quant_int8: F=%zu (max 32768) or T=%zu too large", F, T);
        return -1;
    }
    k_silu_mul_quant_int8<<<(unsigned)T, 256, F * 2, S(st)>>>(gu, q, scales, (int)F);
    return snx_launch_check("k_silu_mul_quant_int8");
}


size_t snx_w4_prep_rows(size_t M) { return (M + GBM - 1) / GBM * GBM; }

int snx_w4a16_gemm_ok(size_t M, size_t N, size_t K, int group) {
    // the stage loads read fp16 scales in aligned pairs: an even group count
    return M >= 1 && N >= 1 && K >= GBK && K % GBK == 0 && group >= GBK &&
           (group & (group - 1)) == 0 && K % (size_t)group == 0 && (K / group) % 2 == 0 &&
           M * K * 2 < (1ull << 32) && N * K / 2 < (1ull << 32);
}

int snx_k_w4_prep_x(const uint16_t* x, uint16_t* xp, float* xs, size_t M, size_t K, size_t Mp,
                    void* st) {
    const size_t items = M * (K / 8);
    const size_t per = 256 * PREP_ITEMS;
    if (items == 0 || items >= (1ull << 31)) {
        snx_set_error("w4a16 activation pass: %zu x %zu activations out of range", M, K);
        return -1;
    }
    k_w4_prep_x<<<(unsigned)((items + per - 1) / per), 256, 0, S(st)>>>(x, xp, xs, (int)K, (int)Mp,
                                                                         (uint32_t)items);
    return snx_launch_check("k_w4_prep_x");
}

// K spans of the prefill GEMM for M x N x K (no SwiGLU step): 4 or 2 when
// the tiles fill at most a quarter or a half of the CUs and each span keeps
// at least two 128-column steps; 2 as well when the tiles exceed a round of
// the CUs by at most half a round (the launcher then runs the full rounds
// whole-K and only the remaining tiles in two spans: the QKV projection's
// 360 tiles on 256 CUs); else 1.
int snx_w4a16_gemm_splits(size_t M, size_t N, size_t K) {
    const size_t ntiles = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN);
    const size_t ncu = (size_t)snx::cu_count(), nk = K / GBK;
    if (ntiles * 4 <= ncu && nk % 4 == 0 && nk >= 8) return 4;
    if (ntiles * 2 <= ncu && nk % 2 == 0 && nk >= 4) return 2;
    const size_t rem = ntiles % ncu;
    if (ntiles > ncu && rem > 0 && rem * 2 <= ncu && nk % 2 == 0 && nk >= 4) return 2;
    return 1;
}

// Bytes of the span partials (`part`) and arrival counters (`cnt`) of a
// `splits`-span call: a 16 KB slot per (unit, wave) of the tiles that take
// spans (past a full round of CUs only the remaining ones), a counter per
// (tile, wave).
size_t snx_w4a16_gemm_part_bytes(size_t M, size_t N, int splits) {
    size_t ntiles = ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN);
    const size_t ncu = (size_t)snx::cu_count();
    if (ntiles > ncu) ntiles %= ncu;
    return ntiles * (size_t)splits * 8 * (2 * 8 * 64 * 16);
}
size_t snx_w4a16_gemm_cnt_bytes(size_t M, size_t N) {
    return ((M + GBM - 1) / GBM) * ((N + GBN - 1) / GBN) * 8 * sizeof(uint32_t);
}

int snx_k_w4a16_gemm(const uint16_t* xp, const float* xs, const uint32_t* qw,
                     const uint16_t* scales, const uint32_t* qzeros, void* y, const float* bias,
                     int y_f32, size_t M, size_t N, size_t K, int group, size_t Mp, int splits,
                     void* part, uint32_t* cnt, void* st) {
    const int m = (int)M, n = (int)N, k = (int)K, mp = (int)Mp;
    if (splits > 1 && (!part || !cnt || splits != snx_w4a16_gemm_splits(M, N, K))) {
        snx_set_error("w4a16 gemm: %d K spans need their partials and counters (and a shape that takes them)", splits);
        return -1;
    }
    if (qzeros) {
        if (y_f32) return launch_w4_gemm<true, true, W4_WN, false>(xp, xs, qw, scales, qzeros, y, bias, m, n, k, group, mp, splits, part, cnt, S(st));
        return launch_w4_gemm<true, false, W4_WN, false>(xp, xs, qw, scales, qzeros, y, bias, m, n, k, group, mp, splits, part, cnt, S(st));
    }
    if (y_f32) return launch_w4_gemm<false, true, W4_WN, false>(xp, xs, qw, scales, qzeros, y, bias, m, n, k, group, mp, splits, part, cnt, S(st));
    return launch_w4_gemm<false, false, W4_WN, false>(xp, xs, qw, scales, qzeros, y, bias, m, n, k, group, mp, splits, part, cnt, S(st));
}

int snx_k_w4a16_gemm_swiglu_prep(const uint16_t* xp, const float* xs, const uint32_t* qw,
                                 const uint16_t* scales, const uint32_t* qzeros, uint16_t* out_xp,
                                 float* out_xs, const float* bias, size_t M, size_t F, size_t K, int group,
                                 size_t Mp, void* st) {
    const int m = (int)M, f = (int)F, k = (int)K, mp = (int)Mp;
    const int tiles_m = (m + GBM - 1) / GBM, tiles_n = (f + GBN / 2 - 1) / (GBN / 2);
    const size_t lds = (size_t)GSTAGES * GRING;
    const int gshift = __builtin_ctz((unsigned)group);
    static std::atomic<uint64_t> lds_done[2];   // > 64 KB of LDS per workgroup, per device
#define SNX_GP(Z)                                                                                        \
    do {                                                                                                 \
        const void* kfn = reinterpret_cast<const void*>(&k_w4a16_gemm<Z, false, W4_WN, true, 1, true>); \
        if (snx::lds_optin(kfn, (int)lds, lds_done[Z ? 1 : 0]) != hipSuccess) {                         \
            snx_set_error("w4a16 gemm: cannot reserve %zu bytes of LDS", lds);                          \
            return -1;                                                                                   \
        }                                                                                                \
        k_w4a16_gemm<Z, false, W4_WN, true, 1, true><<<tiles_m * tiles_n, 512, lds, S(st)>>>(           \
            xp, xs, qw, scales, qzeros, out_xp, bias, m, f, k, k / group, gshift, mp, tiles_m,           \
            reinterpret_cast<u32x4*>(out_xs), nullptr, 0);                                               \
    } while (0)
    if (qzeros) SNX_GP(true);
    else SNX_GP(false);
#undef SNX_GP
    return snx_launch_check("k_w4a16_gemm");
}

int snx_k_w4a16_gemm_swiglu(const uint16_t* xp, const float* xs, const uint32_t* qw,
                            const uint16_t* scales, const uint32_t* qzeros, uint16_t* out,
                            const float* bias, size_t M, size_t F, size_t K, int group, size_t Mp,
                            void* st) {
    const int m = (int)M, f = (int)F, k = (int)K, mp = (int)Mp;
    if (qzeros)
        return launch_w4_gemm<true, false, W4_WN, true>(xp, xs, qw, scales, qzeros, out, bias, m, f, k, group, mp, 1,
                                                        nullptr, nullptr, S(st));
    return launch_w4_gemm<false, false, W4_WN, true>(xp, xs, qw, scales, qzeros, out, bias, m, f, k, group, mp, 1,
                                                     nullptr, nullptr, S(st));
}

}  // extern "C"
