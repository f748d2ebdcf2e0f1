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

}  // extern "C"
