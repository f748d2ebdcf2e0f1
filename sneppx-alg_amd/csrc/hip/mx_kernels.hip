// mx_kernels.hip - MX (micro-scaling) encode / decode on gfx950, bit-exact
// with the reference's numpy implementation
// (bindings/python/SneppX_ALG/interface_bindings/mx_formats.py:75-222).
//
// Everything is integer work on the float32 bit patterns:
//   * block peak: max |x| (a NaN or an infinity makes the block non-finite);
//   * shared exponent s = floor(log2 peak) - E + (mantissa(peak) > mantissa(
//     max_element)), plus the reference's rounding at exact ties
//     (mx_ties.inc);
//   * element code of v = x * 2^-s: sign, exponent field clamped to
//     [0, 2^e_bits - 1] (exponent -bias and below encode as subnormals),
//     mantissa rounded half-to-even and clipped (no carry into the exponent,
//     mx_formats.py:113-119), packed as a little-endian bitstream;
//   * decode: +-(2^m + mant) * 2^(field - bias - m) (field 0: mant *
//     2^(1 - bias - m)) times 2^s, one correctly rounded ldexp.
// Non-finite blocks follow what the reference's float->int64 casts do on
// x86-64 (INT64_MIN): stored exponent 0, codes sign | max subnormal mantissa
// for nonzero elements, 0 for zeros and NaNs.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../snx_internal.h"

namespace {

#include "mx_ties.inc"

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

struct Fmt {
    int bits, mb, bias, E, fmax, mmax, row;
    uint32_t cfield;   // float32 mantissa field of max_element's significand
};

// f: 0 e4m3, 1 e5m2, 2 e3m2, 3 e2m3, 4 e2m1 (rows of the tie tables)
__host__ __device__ inline Fmt fmt_of(int f) {
    const int mb = f == 0 ? 3 : f == 1 ? 2 : f == 2 ? 2 : f == 3 ? 3 : 1;
    const int eb = f == 0 ? 4 : f == 1 ? 5 : f == 2 ? 3 : f == 3 ? 2 : 2;
    const int bias = f == 0 ? 7 : f == 1 ? 15 : f == 2 ? 3 : 1;
    Fmt F;
    F.mb = mb;
    F.bits = 1 + eb + mb;
    F.bias = bias;
    F.fmax = (1 << eb) - 1;
    F.E = F.fmax - bias;
    F.mmax = (1 << mb) - 1;
    F.cfield = (uint32_t)((1 << mb) - 1) << (23 - mb);
    F.row = f;
    return F;
}

// |x| as (exponent, 24-bit significand) for finite nonzero x
__host__ __device__ inline void split(uint32_t b, int& e, uint32_t& sig) {
    const uint32_t ex = (b >> 23) & 0xFF, man = b & 0x7FFFFF;
    if (ex) {
        e = (int)ex - 127;
        sig = man | 0x800000u;
    } else {
        const int p = 31 - __builtin_clz(man);   // leading bit of a denormal
        e = p - 149;
        sig = man << (23 - p);
    }
}

// shared exponent for a finite positive peak; tie table 32 (block peaks,
// float32 log2) or 64 (per-tensor peaks, float64 log2)
__host__ __device__ inline int scale_of(uint32_t peak_bits, const Fmt& F, bool tensor) {
    int e;
    uint32_t sig;
    split(peak_bits, e, sig);
    const uint32_t mf = sig & 0x7FFFFF;
    int s = e - F.E;
    if (mf > F.cfield) {
        s += 1;
    } else if (mf == F.cfield) {
        const int i = e - kMxTieELo;
        if (i >= 0 && i < 32 * kMxTieWords) {
            const uint32_t w = tensor ? kMxTie64[F.row][i >> 5] : kMxTie32[F.row][i >> 5];
            s += (int)((w >> (i & 31)) & 1u);
        }
    }
    return s;
}

// round-half-even of sig / 2^sh (sh >= 1), saturating large shifts to 0
__device__ inline uint32_t rne_shift(uint32_t sig, int sh) {
    if (sh > 40) return 0;
    const uint64_t v = sig;
    const uint64_t q = v >> sh, rem = v & ((1ull << sh) - 1), half = 1ull << (sh - 1);
    return (uint32_t)(q + ((rem > half || (rem == half && (q & 1))) ? 1 : 0));
}

// code of v = x * 2^-s for finite x (mx_formats.py:99-123); an infinite x
// (per-tensor overflow) takes the cast path: sign | max subnormal mantissa
__device__ inline uint32_t encode(float x, int s, const Fmt& F) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    const uint32_t sign = (b >> 31) & (x < 0.0f ? 1u : 0u);
    if ((b & 0x7FFFFFFFu) == 0) return 0;
    if ((b & 0x7F800000u) == 0x7F800000u)   // inf / NaN
        return (b & 0x7FFFFFu) ? 0u : (sign << (F.bits - 1)) | (uint32_t)F.mmax;
    int e;
    uint32_t sig;
    split(b, e, sig);
    const int ev = e - s;   // exponent of v
    uint32_t field, mant;
    if (ev > F.E) {                 // above the largest binade: saturate
        field = (uint32_t)F.fmax;
        mant = (uint32_t)F.mmax;
    } else if (ev <= -F.bias) {     // subnormal: round(|v| * 2^(m + bias - 1))
        field = 0;
        mant = rne_shift(sig, 23 - (ev + F.mb + F.bias - 1));
        if (mant > (uint32_t)F.mmax) mant = (uint32_t)F.mmax;
    } else {
        field = (uint32_t)(ev + F.bias);
        mant = rne_shift(sig & 0x7FFFFF, 23 - F.mb);
        if (mant > (uint32_t)F.mmax) mant = (uint32_t)F.mmax;
    }
    return (sign << (F.bits - 1)) | (field << F.mb) | mant;
}

// non-finite block (mx_formats.py:193-199 with exponent INT64_MIN)
__device__ inline uint32_t encode_nonfinite(float x, const Fmt& F) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    if ((b & 0x7FFFFFFFu) == 0 || x != x) return 0;
    return ((x < 0.0f ? 1u : 0u) << (F.bits - 1)) | (uint32_t)F.mmax;
}

__device__ inline float decode(uint32_t c, int s, const Fmt& F) {
    const uint32_t field = (c >> F.mb) & (uint32_t)F.fmax, mant = c & (uint32_t)F.mmax;
    const bool neg = (c >> (F.bits - 1)) & 1u;
    const float v = field ? ldexpf((float)((1u << F.mb) + mant), (int)field - F.bias - F.mb + s)
                          : ldexpf((float)mant, 1 - F.bias - F.mb + s);
    return neg ? -v : v;
}

// little-endian bitstream writer for one byte-aligned run
struct BitOut {
    uint8_t* p;
    uint64_t acc;
    int n;
    __device__ void put(uint32_t code, int bits) {
        acc |= (uint64_t)code << n;
        n += bits;
        while (n >= 8) {
            *p++ = (uint8_t)acc;
            acc >>= 8;
            n -= 8;
        }
    }
    __device__ void flush() {
        if (n > 0) *p = (uint8_t)acc;
    }
};

__device__ inline uint32_t get_bits(const uint8_t* base, size_t bitpos, int bits) {
    const size_t byte = bitpos >> 3;
    const int sh = (int)(bitpos & 7);
    uint32_t w = base[byte];
    if (sh + bits > 8) w |= (uint32_t)base[byte + 1] << 8;
    return (w >> sh) & ((1u << bits) - 1u);
}

// ---- blocked: one thread per block of bs elements (bs % 8 == 0) ----------
__global__ void __launch_bounds__(256) k_mx_quant_blocks(const float* __restrict__ x,
                                                         uint8_t* __restrict__ packed,
                                                         int8_t* __restrict__ scales, size_t rows,
                                                         size_t cols, int bs, int f) {
    const Fmt F = fmt_of(f);
    const size_t nb = (cols + bs - 1) / bs;
    const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= rows * nb) return;
    const size_t r = blk / nb, j = blk - r * nb;
    const float* xr = x + r * cols;
    const size_t c0 = j * (size_t)bs;
    float peak = 0.0f;
    bool nonfinite = false;
    for (int i = 0; i < bs; i++) {
        const size_t c = c0 + i;
        const float v = c < cols ? xr[c] : 0.0f;
        const float a = fabsf(v);
        nonfinite |= !(a <= 3.4028234663852886e38f);   // NaN or inf
        peak = a > peak ? a : peak;
    }
    int s = 0;
    if (!nonfinite) s = scale_of(__builtin_bit_cast(uint32_t, peak > 0.0f ? peak : 1.0f), F, false);
    scales[blk] = nonfinite ? (int8_t)0 : (int8_t)(uint8_t)(uint32_t)s;   // int8 cast wraps
    BitOut out{packed + blk * (size_t)(bs * F.bits / 8), 0, 0};
    for (int i = 0; i < bs; i++) {
        const size_t c = c0 + i;
        const float v = c < cols ? xr[c] : 0.0f;
        out.put(nonfinite ? encode_nonfinite(v, F) : encode(v, s, F), F.bits);
    }
    out.flush();
}

__global__ void __launch_bounds__(256) k_mx_dequant_blocks(const uint8_t* __restrict__ packed,
                                                           const int8_t* __restrict__ scales,
                                                           float* __restrict__ y, size_t rows,
                                                           size_t cols, int bs, int f) {
    const Fmt F = fmt_of(f);
    const size_t nb = (cols + bs - 1) / bs;
    const size_t it = (size_t)blockIdx.x * 256 + threadIdx.x;   // one item = 8 elements
    const size_t per_row = nb * (size_t)bs / 8;
    if (it >= rows * per_row) return;
    const size_t r = it / per_row, g = it - r * per_row;
    const size_t c0 = g * 8;
    if (c0 >= cols) return;
    const int s = scales[r * nb + c0 / bs];
    const uint8_t* base = packed + r * (nb * (size_t)bs * F.bits / 8);
    for (int i = 0; i < 8 && c0 + i < cols; i++)
        y[r * cols + c0 + i] = decode(get_bits(base, (c0 + i) * (size_t)F.bits, F.bits), s, F);
}

// ---- per tensor --------------------------------------------------------------
// stats[0] = max |x| over non-NaN elements (as bits), stats[1] = any NaN
__global__ void __launch_bounds__(256) k_mx_tensor_stats(const float* __restrict__ x, size_t n,
                                                         uint32_t* __restrict__ part) {
    float m = 0.0f;
    uint32_t nan = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float a = fabsf(x[i]);
        if (a != a) nan = 1;
        else m = a > m ? a : m;
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float v = __shfl_xor(m, o);
        m = v > m ? v : m;
        nan |= (uint32_t)__shfl_xor((int)nan, o);
    }
    __shared__ float sm[4];
    __shared__ uint32_t sn[4];
    if ((threadIdx.x & 63) == 0) {
        sm[threadIdx.x >> 6] = m;
        sn[threadIdx.x >> 6] = nan;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) {
            m = sm[w] > m ? sm[w] : m;
            nan |= sn[w];
        }
        part[2 * blockIdx.x] = __builtin_bit_cast(uint32_t, m);
        part[2 * blockIdx.x + 1] = nan;
    }
}

// one thread per 8 elements (a byte-aligned run of 8 * bits bits)
__global__ void __launch_bounds__(256) k_mx_quant_tensor(const float* __restrict__ x,
                                                         uint8_t* __restrict__ packed, size_t n,
                                                         int s, int f) {
    const Fmt F = fmt_of(f);
    const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (g * 8 >= n) return;
    BitOut out{packed + g * (size_t)F.bits, 0, 0};
    for (int i = 0; i < 8; i++) {
        const size_t k = g * 8 + i;
        if (k >= n) break;
        // float32 division by 2^s (mx_formats.py:171): one correctly rounded ldexp
        out.put(encode(ldexpf(x[k], -s), 0, F), F.bits);
    }
    out.flush();
}

__global__ void __launch_bounds__(256) k_mx_dequant_tensor(const uint8_t* __restrict__ packed,
                                                           float* __restrict__ y, size_t n, int s,
                                                           int f) {
    const Fmt F = fmt_of(f);
    const size_t k = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (k >= n) return;
    y[k] = decode(get_bits(packed, k * (size_t)F.bits, F.bits), s, F);
}

unsigned grid_of(size_t items) {
    const size_t g = (items + 255) / 256;
    return (unsigned)(g ? g : 1);
}

// One code one binade lower (value / 2) in the same 8-bit format, MB mantissa
// bits: fields >= 2 lose one exponent step exactly; field 1 and subnormals
// become subnormals k / 2 (k = the value in units of the smallest subnormal),
// rounded half to even when k is odd.  Returns the code; *inexact counts the
// rounded ones.
template <int MB>
__device__ inline uint32_t half_code(uint32_t c, int* inexact) {
    const uint32_t sign = c & 0x80u, mag = c & 0x7Fu, e = mag >> MB, m = mag & ((1u << MB) - 1u);
    if (e >= 2) return sign | (mag - (1u << MB));
    const uint32_t k = e ? (1u << MB) + m : m;          // value in subnormal units
    uint32_t h = k >> 1;
    if (k & 1u) {
        h += h & 1u;
        (*inexact)++;
    }
    return sign | h;    // h <= 2^MB: a subnormal, or exactly the smallest normal
}

// Reference MXFP8 blocks -> codes the gfx950 matrix cores decode to the same
// values (OCP e4m3fn / e5m2 have no finite all-ones exponent, the reference
// has: E4M3 0x7F = 480, E5M2 field 31 = 65536 .. 114688).  A block holding
// such a code is re-encoded one binade lower with exponent s + 1 (exact but
// for odd subnormal-unit values at the new scale, which round half to even);
// other blocks are copied.  One thread per 32-element block; F 0 = e4m3,
// 1 = e5m2.  A block at the largest exponent (127) stays as it is.
template <int F>
__global__ void __launch_bounds__(256) k_mx_to_mfma(const uint8_t* __restrict__ in,
                                                    const int8_t* __restrict__ sin,
                                                    uint8_t* __restrict__ out,
                                                    int8_t* __restrict__ sout, size_t nblocks,
                                                    unsigned int* __restrict__ rounded) {
    constexpr int MB = F == 0 ? 3 : 2;
    const size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    u32x4 v[2];
    v[0] = reinterpret_cast<const u32x4*>(in + b * 32)[0];
    v[1] = reinterpret_cast<const u32x4*>(in + b * 32)[1];
    const int s = sin[b];
    uint32_t any = 0;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t w = v[i][e];
            if (F == 0)   // a byte whose low 7 bits are all ones carries into bit 7
                any |= ((w & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u;
            else          // exponent field 31
                any |= ((w & 0x7C7C7C7Cu) + 0x04040404u) & 0x80808080u;
        }
    if (!any || s >= 127) {
        reinterpret_cast<u32x4*>(out + b * 32)[0] = v[0];
        reinterpret_cast<u32x4*>(out + b * 32)[1] = v[1];
        sout[b] = (int8_t)s;
        return;
    }
    int inexact = 0;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t w = v[i][e];
            uint32_t r = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) r |= half_code<MB>((w >> (8 * j)) & 0xFFu, &inexact) << (8 * j);
            v[i][e] = r;
        }
    reinterpret_cast<u32x4*>(out + b * 32)[0] = v[0];
    reinterpret_cast<u32x4*>(out + b * 32)[1] = v[1];
    sout[b] = (int8_t)(s + 1);
    if (inexact && rounded) atomicAdd(rounded, (unsigned)inexact);
}

// Exponents of one GEMM operand in the block-32 form the matrix-core GEMMs
// read (one int8 per 32 elements of a row: the matrix cores scale 32-element
// blocks).  rep > 0: a blocked tensor whose block is 32 * rep elements, each
// exponent repeated for its rep 32-element pieces.  rep == 0: a per-tensor
// exponent (NVFP4), where the product's exponent t = sA + sW is what
// matters; A takes ceil(t / 2) and W floor(t / 2) (which = 0 / 1), so that
// neither reaches -128, which the E8M0 conversion clamps to 2^-127 (at
// t < -254 both halves clamp to -127, and every product then underflows to
// zero in fp32 as it does at the exact exponent).
__global__ void __launch_bounds__(256) k_mx_expand_scales(const int8_t* __restrict__ src,
                                                          const int8_t* __restrict__ sA,
                                                          const int8_t* __restrict__ sW,
                                                          int8_t* __restrict__ dst, size_t rows,
                                                          uint32_t kb32, uint32_t rep, int which) {
    const size_t n = rows * kb32;
    int pt = 0;
    if (rep == 0) {
        const int t = (int)sA[0] + (int)sW[0];
        const int hi = t - (t >> 1), lo = t >> 1;          // ceil, floor (arithmetic shift)
        pt = which == 0 ? hi : lo;
        pt = pt < -127 ? -127 : pt;
    }
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        if (rep == 0) {
            dst[i] = (int8_t)pt;
        } else {
            const size_t r = i / kb32, c = i % kb32;
            dst[i] = src[r * (kb32 / rep) + c / rep];
        }
    }
}

}  // namespace

extern "C" {

int snx_mx_scale_host(uint32_t peak_bits, int f, int tensor) {
    return scale_of(peak_bits, fmt_of(f), tensor != 0);
}

int snx_k_mx_quant_blocks(const float* x, uint8_t* packed, int8_t* scales, size_t rows,
                          size_t cols, int bs, int f, void* st) {
    const size_t nb = (cols + bs - 1) / bs;
    if (rows * nb >= (1ull << 38)) {
        snx_set_error("mx quantize: too many blocks");
        return -1;
    }
    k_mx_quant_blocks<<<grid_of(rows * nb), 256, 0, S(st)>>>(x, packed, scales, rows, cols, bs, f);
    return snx_launch_check("k_mx_quant_blocks");
}

int snx_k_mx_dequant_blocks(const uint8_t* packed, const int8_t* scales, float* y, size_t rows,
                            size_t cols, int bs, int f, void* st) {
    const size_t nb = (cols + bs - 1) / bs;
    k_mx_dequant_blocks<<<grid_of(rows * nb * (size_t)bs / 8), 256, 0, S(st)>>>(packed, scales, y, rows,
                                                                               cols, bs, f);
    return snx_launch_check("k_mx_dequant_blocks");
}

int snx_mx_tensor_parts(size_t n) {
    const size_t b = (n + 255) / 256;
    return (int)(b < 1024 ? (b ? b : 1) : 1024);
}

int snx_k_mx_tensor_stats(const float* x, size_t n, uint32_t* part, int nparts, void* st) {
    k_mx_tensor_stats<<<nparts, 256, 0, S(st)>>>(x, n, part);
    return snx_launch_check("k_mx_tensor_stats");
}

int snx_k_mx_quant_tensor(const float* x, uint8_t* packed, size_t n, int s, int f, void* st) {
    k_mx_quant_tensor<<<grid_of((n + 7) / 8), 256, 0, S(st)>>>(x, packed, n, s, f);
    return snx_launch_check("k_mx_quant_tensor");
}

int snx_k_mx_dequant_tensor(const uint8_t* packed, float* y, size_t n, int s, int f, void* st) {
    k_mx_dequant_tensor<<<grid_of(n), 256, 0, S(st)>>>(packed, y, n, s, f);
    return snx_launch_check("k_mx_dequant_tensor");
}

int snx_k_mx_expand_scales(const int8_t* src, const int8_t* sA, const int8_t* sW, int8_t* dst,
                           size_t rows, size_t kb32, unsigned rep, int which, void* st) {
    if (kb32 == 0 || kb32 > 0xffffffffu || (rep && kb32 % rep)) {
        snx_set_error("mx scales: %zu blocks of 32 per row do not split into blocks of %u", kb32, 32 * rep);
        return -1;
    }
    k_mx_expand_scales<<<grid_of(rows * kb32), 256, 0, S(st)>>>(src, sA, sW, dst, rows, (uint32_t)kb32, rep,
                                                                which);
    return snx_launch_check("k_mx_expand_scales");
}

int snx_k_mx_to_mfma(const uint8_t* in, const int8_t* sin, uint8_t* out, int8_t* sout,
                     size_t nblocks, int f, unsigned int* rounded, void* st) {
    if (f == 0)
        k_mx_to_mfma<0><<<grid_of(nblocks), 256, 0, S(st)>>>(in, sin, out, sout, nblocks, rounded);
    else
        k_mx_to_mfma<1><<<grid_of(nblocks), 256, 0, S(st)>>>(in, sin, out, sout, nblocks, rounded);
    return snx_launch_check("k_mx_to_mfma");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// MXFP4 GEMM: out[m][n] = sum_k A[m][k] W[n][k] with A, W in the reference's
// MXFP4 encoding (blocks of 32 along K, int8 exponents), on
// v_mfma_scale_f32_32x32x64_f8f6f4 (E2M1 operands, E8M0 block scales, fp32
// accumulators).  The E2M1 codes are the OCP ones, so the matrix cores see
// exactly the reference's values; an int8 exponent s becomes the E8M0 byte
// s + 127 (s = -128 is clamped to 2^-127).  Operand lane l: row / column
// l % 32, elements 32 (l / 32) .. +31 of the 64-element step = 16 bytes of
// codes and one scale byte (the block's exponent).
// Workgroup: 128 x 128 outputs, 4 waves of 64 x 64 (2 x 2 blocks of 32);
// every wave loads its fragments straight from global memory, the next K
// step's while the current one computes.
namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ inline int e8m0(int8_t s) { return s < -127 ? 0 : (int)s + 127; }

template <bool YF32>
__global__ void __launch_bounds__(256) k_mxfp4_gemm(const uint8_t* __restrict__ A,
                                                    const int8_t* __restrict__ sA,
                                                    const uint8_t* __restrict__ W,
                                                    const int8_t* __restrict__ sW,
                                                    void* __restrict__ out, int M, int N, int K) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r32 = lane & 31, h = lane >> 5;
    const int m0 = blockIdx.y * 128 + (wave >> 1) * 64, n0 = blockIdx.x * 128 + (wave & 1) * 64;
    const int kb = K / 32;   // scale blocks per row
    int ra[2], rb[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int r = m0 + 32 * i + r32, c = n0 + 32 * i + r32;
        ra[i] = r < M ? r : M - 1;
        rb[i] = c < N ? c : N - 1;
    }
    auto load = [&](int ks, u32x4 (&fa)[2], u32x4 (&fb)[2], int (&sa)[2], int (&sb)[2]) {
        const int blk = 2 * ks + h;   // this lane's 32-element block
#pragma unroll
        for (int i = 0; i < 2; i++) {
            fa[i] = *reinterpret_cast<const u32x4*>(A + (size_t)ra[i] * (K / 2) + (size_t)blk * 16);
            fb[i] = *reinterpret_cast<const u32x4*>(W + (size_t)rb[i] * (K / 2) + (size_t)blk * 16);
            sa[i] = e8m0(sA[(size_t)ra[i] * kb + blk]);
            sb[i] = e8m0(sW[(size_t)rb[i] * kb + blk]);
        }
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = f32x16{};
    const int nks = K / 64;
    u32x4 fa[2], fb[2];
    int sa[2], sb[2];
    load(0, fa, fb, sa, sb);
    for (int ks = 0; ks < nks; ks++) {
        u32x4 na[2], nb[2];
        int nsa[2], nsb[2];
        load(ks + 1 < nks ? ks + 1 : ks, na, nb, nsa, nsb);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const i32x8 a = {(int)fa[i][0], (int)fa[i][1], (int)fa[i][2], (int)fa[i][3], 0, 0, 0, 0};
                const i32x8 b = {(int)fb[j][0], (int)fb[j][1], (int)fb[j][2], (int)fb[j][3], 0, 0, 0, 0};
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc[i][j], 4, 4, 0,
                                                                            sa[i], 0, sb[j]);
            }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            fa[i] = na[i];
            fb[i] = nb[i];
            sa[i] = nsa[i];
            sb[i] = nsb[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + 32 * j + r32;
            if (n >= N) continue;
#pragma unroll
            for (int v = 0; v < 16; v++) {   // 32x32 C layout: row 8 (v/4) + 4 (l/32) + v%4
                const int m = m0 + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
                if (m >= M) continue;
                if (YF32)
                    reinterpret_cast<float*>(out)[(size_t)m * N + n] = acc[i][j][v];
                else
                    reinterpret_cast<uint16_t*>(out)[(size_t)m * N + n] =
                        __builtin_bit_cast(uint16_t, (__bf16)acc[i][j][v]);
            }
        }
}

}  // namespace

extern "C" int snx_k_mxfp4_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W,
                                const int8_t* sW, void* out, int y_f32, size_t M, size_t N,
                                size_t K, void* st) {
    if (M > 0x7fffffff || N > 0x7fffffff || K > 0x7fffffff || (M + 127) / 128 > 65535) {
        snx_set_error("mxfp4 gemm: shape too large");
        return -1;
    }
    dim3 grid((unsigned)((N + 127) / 128), (unsigned)((M + 127) / 128));
    if (y_f32)
        k_mxfp4_gemm<true><<<grid, 256, 0, S(st)>>>(A, sA, W, sW, out, (int)M, (int)N, (int)K);
    else
        k_mxfp4_gemm<false><<<grid, 256, 0, S(st)>>>(A, sA, W, sW, out, (int)M, (int)N, (int)K);
    return snx_launch_check("k_mxfp4_gemm");
}
