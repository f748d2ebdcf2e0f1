// quant_kernels.hip - bit-exact quantize / dequantize kernels for gfx950.
//
// Built with -ffp-contract=off and IEEE denormals (see the Makefile): every
// multiply, divide and add here rounds exactly where the reference's C does,
// so codes, scales and dequantised values match it bit for bit.  All kernels
// are HBM-bound integer/byte work: coalesced grid-stride loops, wave-level
// reductions through DPP/shuffles, no MFMA.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>

#include "codec.h"
#include "../snx_internal.h"

using namespace snx;

namespace {

constexpr int kBlock = 256;
constexpr int kMaxParts = 1024;

hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

int grid_for(size_t work, int per_block, int cap = 8192) {
    size_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    return (int)(g > (size_t)cap ? cap : g);
}

// max over non-NaN values, as the reference's `if (a > m) m = a`
__device__ __forceinline__ float nanless_max(float a, float b) { return b > a ? b : a; }
__device__ __forceinline__ float nanless_min(float a, float b) { return b < a ? b : a; }

__device__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = nanless_max(v, __shfl_xor(v, o));
    return v;
}
__device__ float wave_min(float v) {
    for (int o = 32; o > 0; o >>= 1) v = nanless_min(v, __shfl_xor(v, o));
    return v;
}
__device__ int wave_min_int(int v) {
    for (int o = 32; o > 0; o >>= 1) {
        int u = __shfl_xor(v, o);
        v = u < v ? u : v;
    }
    return v;
}

template <typename F>
__device__ float block_reduce(float v, F op, float* sh) {
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o));
    __syncthreads();
    if (lane == 0) sh[w] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < nw; i++) r = op(r, sh[i]);
    return r;
}

// ---------------------------------------------------------------- reductions
__device__ __forceinline__ float as_f32(float v) { return v; }
__device__ __forceinline__ float as_f32(uint16_t v) {   // bf16 bits
    return __builtin_bit_cast(float, (uint32_t)v << 16);
}

template <typename T = float>
__global__ void k_absmax(const T* __restrict__ x, size_t n, float* __restrict__ part) {
    __shared__ float sh[16];
    float m = 0.0f;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        m = nanless_max(m, fabsf(as_f32(x[i])));
    m = block_reduce(m, nanless_max, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

__global__ void k_minmax(const float* __restrict__ x, size_t n, float* __restrict__ part) {
    __shared__ float sh[16];
    float lo = INFINITY, hi = -INFINITY;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float v = x[i];
        lo = nanless_min(lo, v);
        hi = nanless_max(hi, v);
    }
    lo = block_reduce(lo, nanless_min, sh);
    hi = block_reduce(hi, nanless_max, sh);
    if (threadIdx.x == 0) {
        part[2 * blockIdx.x] = lo;
        part[2 * blockIdx.x + 1] = hi;
    }
}

// One block turns the partials into the reference's scale (and zero point).
__global__ void k_finalize(const float* __restrict__ part, int nparts, int kind,
                           const float* __restrict__ x, float* __restrict__ rec,
                           float* __restrict__ scale_out) {
    __shared__ float sh[16];
    if (kind == SNX_SCALE_ASYM255) {
        float lo = INFINITY, hi = -INFINITY;
        for (int i = threadIdx.x; i < nparts; i += blockDim.x) {
            lo = nanless_min(lo, part[2 * i]);
            hi = nanless_max(hi, part[2 * i + 1]);
        }
        lo = block_reduce(lo, nanless_min, sh);
        hi = block_reduce(hi, nanless_max, sh);
        if (threadIdx.x == 0) {
            // quantize_int8.c:102-106: the scan starts from input[0], so a NaN
            // there pins both ends to NaN; later NaNs never compare.
            float x0 = x[0];
            if (x0 != x0) lo = hi = x0;
            float s = 1.0f, zp = 0.0f, degenerate = 1.0f;
            if (!(hi - lo < FLT_MIN)) {
                s = (hi - lo) / 255.0f;
                zp = (float)clampi(round_i32(-lo / s), 0, 255);
                degenerate = 0.0f;
            }
            rec[0] = s;
            rec[1] = 1.0f / s;
            rec[2] = zp;
            rec[3] = degenerate;
            if (scale_out) scale_out[0] = s;
        }
        return;
    }
    float m = 0.0f;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = nanless_max(m, part[i]);
    m = block_reduce(m, nanless_max, sh);
    if (kind == SNX_SCALE_MODELZOO) {
        // weights.c:233-240: the scan ignores NaN (a false compare); the
        // multiplier is 127 / max, or 1 for an all-zero tensor
        if (threadIdx.x == 0) {
            const float mult = m > 0.0f ? 127.0f / m : 1.0f;
            rec[0] = mult;
            rec[1] = 1.0f / mult;
            rec[2] = 0.0f;
            rec[3] = 0.0f;
            if (scale_out) scale_out[0] = mult;
        }
        return;
    }
    if (threadIdx.x == 0) {
        float div = kind == SNX_SCALE_SYM127 ? 127.0f : kind == SNX_SCALE_SYM7 ? 7.0f : 240.0f;
        bool degenerate = m < FLT_MIN;
        float s = degenerate ? 1.0f : m / div;
        rec[0] = s;
        rec[1] = 1.0f / s;
        rec[2] = 0.0f;
        rec[3] = degenerate ? 1.0f : 0.0f;
        if (scale_out) scale_out[0] = s;
    }
}

// ------------------------------------------------------------ vector codecs
__global__ void k_quant_int8_sym(const float* __restrict__ x, int8_t* __restrict__ q, size_t n,
                                 const float* __restrict__ rec) {
    float inv = rec[1];
    bool zero = rec[3] != 0.0f;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        q[i] = zero ? 0 : (int8_t)clampi(round_i32(x[i] * inv), -128, 127);
}

// weights.c:242-247: v = x * m clamped to [-128, 127], converted by
// truncation toward zero; the x86 conversion of NaN gives 0, so does this one.
__global__ void k_quant_int8_modelzoo(const float* __restrict__ x, int8_t* __restrict__ q,
                                      size_t n, const float* __restrict__ rec) {
    const float mult = rec[0];
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float v = x[i] * mult;
        if (v > 127.0f) v = 127.0f;
        else if (v < -128.0f) v = -128.0f;
        q[i] = v != v ? (int8_t)0 : (int8_t)(int)v;
    }
}

__global__ void k_dequant_int8_sym(const int8_t* __restrict__ q, float* __restrict__ y, size_t n,
                                   float scale) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = (float)q[i] * scale;
}

__global__ void k_quant_int8_asym(const float* __restrict__ x, int8_t* __restrict__ q, size_t n,
                                  const float* __restrict__ rec) {
    float s = rec[0], zp = rec[2];
    bool zero = rec[3] != 0.0f;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float t = x[i] / s;
        q[i] = zero ? 0 : (int8_t)(uint8_t)clampi(round_i32(t + zp), 0, 255);
    }
}

__global__ void k_dequant_int8_asym(const int8_t* __restrict__ q, float* __restrict__ y, size_t n,
                                    float scale, float zp) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = ((float)(uint8_t)q[i] - zp) * scale;
}

__global__ void k_quant_int4_sym(const float* __restrict__ x, uint8_t* __restrict__ p, size_t n,
                                 const float* __restrict__ rec) {
    float inv = rec[1];
    bool zero = rec[3] != 0.0f;
    size_t nb = (n + 1) / 2;
    for (size_t b = blockIdx.x * (size_t)blockDim.x + threadIdx.x; b < nb;
         b += (size_t)gridDim.x * blockDim.x) {
        uint32_t v = 0;
        if (!zero) {
            v = (uint32_t)clampi(round_i32(x[2 * b] * inv), -8, 7) & 0xFu;
            if (2 * b + 1 < n) v |= ((uint32_t)clampi(round_i32(x[2 * b + 1] * inv), -8, 7) & 0xFu) << 4;
        }
        p[b] = (uint8_t)v;
    }
}

__global__ void k_dequant_int4_sym(const uint8_t* __restrict__ p, float* __restrict__ y, size_t n,
                                   float scale) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        int v = (p[i >> 1] >> ((i & 1) * 4)) & 0xF;
        y[i] = (float)(v >= 8 ? v - 16 : v) * scale;
    }
}

// With rec (the per-tensor scaled form) the value encoded is x / s, one
// correctly rounded division, not x * (1/s): for s = amax/240 the quotient
// puts the largest element at 240 (code 0x77) in about twice as many cases,
// where the product's 239.99998 truncates to 224.
template <int FMT, typename T = float>
__global__ void k_fp8_encode(const T* __restrict__ x, uint8_t* __restrict__ c, size_t n,
                             const float* __restrict__ rec) {
    float s = rec ? rec[0] : 1.0f;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float v = rec ? as_f32(x[i]) / s : as_f32(x[i]);
        c[i] = FMT == 0 ? fp8_e4m3_encode(v) : fp8_e5m2_encode(v);
    }
}

template <int FMT>
__global__ void k_fp8_decode(const uint8_t* __restrict__ c, float* __restrict__ y, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = FMT == 0 ? fp8_e4m3_decode(c[i]) : fp8_e5m2_decode(c[i]);
}

// ------------------------------------------------------- row / group codecs
// quantize_int8.c:157-177: one block per row.
__device__ __forceinline__ float load_f(const float* p) { return *p; }
__device__ __forceinline__ float load_f(const uint16_t* p) {   // bf16 bits
    return __builtin_bit_cast(float, (uint32_t)*p << 16);
}

template <bool RNE, typename T>
__global__ void k_quant_int8_rows(const T* __restrict__ x, int8_t* __restrict__ q,
                                  float* __restrict__ scales, size_t rows, size_t cols) {
    __shared__ float sh[16];
    for (size_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const T* xr = x + r * cols;
        float m = 0.0f;
        for (size_t c = threadIdx.x; c < cols; c += blockDim.x) m = nanless_max(m, fabsf(load_f(xr + c)));
        m = block_reduce(m, nanless_max, sh);
        float s = m < FLT_MIN ? 1.0f : m / 127.0f;
        float inv = 1.0f / s;
        if (threadIdx.x == 0) scales[r] = s;
        for (size_t c = threadIdx.x; c < cols; c += blockDim.x) {
            const float v = load_f(xr + c) * inv;
            q[r * cols + c] = (int8_t)clampi(RNE ? rne_i32(v) : round_i32(v), -128, 127);
        }
        __syncthreads();
    }
}

// Per-tensor fp8 of bf16 activations, 8 values (one 16-byte load) per
// thread and step: the partial max|x| (NaN ignored) and the scaled e4m3
// codes e4m3(x / s) of k_absmax / k_fp8_encode; n % 8 == 0, x 16-byte and
// c 8-byte aligned.
__global__ void __launch_bounds__(256) k_absmax_bf16_v8(const uint16_t* __restrict__ x, size_t n8,
                                                        float* __restrict__ part) {
    __shared__ float sh[16];
    float m = 0.0f;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n8; i += (size_t)gridDim.x * blockDim.x) {
        const uint4 v = reinterpret_cast<const uint4*>(x)[i];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            m = nanless_max(m, fabsf(__builtin_bit_cast(float, w[e] << 16)));
            m = nanless_max(m, fabsf(__builtin_bit_cast(float, w[e] & 0xFFFF0000u)));
        }
    }
    m = block_reduce(m, nanless_max, sh);
    if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// The scale comes from the partial maxima: every block reduces them (nparts
// floats from L2) to s = max/240 (1 below FLT_MIN), the rule of k_finalize's
// SNX_SCALE_FP8_240, and block 0 writes it to *scale_out for the GEMM.
__global__ void __launch_bounds__(256) k_fp8_encode_bf16_v8(const uint16_t* __restrict__ x,
                                                            uint8_t* __restrict__ c, size_t n8,
                                                            const float* __restrict__ part, int nparts,
                                                            float* __restrict__ scale_out) {
    __shared__ float sh[16];
    float m = 0.0f;
    for (int i = threadIdx.x; i < nparts; i += blockDim.x) m = nanless_max(m, part[i]);
    m = block_reduce(m, nanless_max, sh);
    const float s = m < FLT_MIN ? 1.0f : m / 240.0f;
    if (blockIdx.x == 0 && threadIdx.x == 0) scale_out[0] = s;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n8; i += (size_t)gridDim.x * blockDim.x) {
        const uint4 v = reinterpret_cast<const uint4*>(x)[i];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[2] = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const uint32_t lo = fp8_e4m3_encode(__builtin_bit_cast(float, w[e] << 16) / s);
            const uint32_t hi = fp8_e4m3_encode(__builtin_bit_cast(float, w[e] & 0xFFFF0000u) / s);
            o[e >> 1] |= (lo | hi << 8) << (16 * (e & 1));
        }
        reinterpret_cast<uint2*>(c)[i] = make_uint2(o[0], o[1]);
    }
}

// Per-token int8 of bf16 activations, one pass: quantize_int8.c:157-177 on
// each row (max|x| ignoring NaN, s = max/127 or 1 below FLT_MIN, code
// clamp(roundf(x * (1/s)), -128, 127)), with the row held in registers -
// one 256-thread block per row, CH 16-byte chunks (8 values) per thread, so
// a row is read from memory once.  cols % 8 == 0, cols <= 2048 CH.
typedef uint32_t u32x4q __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2q __attribute__((ext_vector_type(2)));
template <int CH>
__global__ void __launch_bounds__(256) k_quant_rows_bf16_reg(const uint16_t* __restrict__ x,
                                                             int8_t* __restrict__ q,
                                                             float* __restrict__ scales, size_t rows,
                                                             int cols) {
    __shared__ float sh[16];
    const int nch = cols >> 3;
    for (size_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const uint16_t* xr = x + r * (size_t)cols;
        u32x4q v[CH];
        float m = 0.0f;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int ch = threadIdx.x + 256 * c;
            v[c] = ch < nch ? *reinterpret_cast<const u32x4q*>(xr + 8 * ch) : u32x4q{0u, 0u, 0u, 0u};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                m = nanless_max(m, fabsf(__builtin_bit_cast(float, v[c][e] << 16)));
                m = nanless_max(m, fabsf(__builtin_bit_cast(float, v[c][e] & 0xFFFF0000u)));
            }
        }
        m = block_reduce(m, nanless_max, sh);
        const float s = m < FLT_MIN ? 1.0f : m / 127.0f;
        const float inv = 1.0f / s;
        if (threadIdx.x == 0) scales[r] = s;
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int ch = threadIdx.x + 256 * c;
            if (ch >= nch) break;
            u32x2q o;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                uint32_t w = 0u;
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint32_t b = v[c][2 * h + e];
                    const int lo = clampi(round_i32(__builtin_bit_cast(float, b << 16) * inv), -128, 127);
                    const int hi = clampi(round_i32(__builtin_bit_cast(float, b & 0xFFFF0000u) * inv), -128, 127);
                    w |= ((uint32_t)(lo & 0xFF) | (uint32_t)(hi & 0xFF) << 8) << (16 * e);
                }
                o[h] = w;
            }
            *reinterpret_cast<u32x2q*>(q + r * (size_t)cols + 8 * ch) = o;
        }
        __syncthreads();   // sh is reused by the next row's reduction
    }
}

// tensor.c:2180-2195 (SNEPPX_tensor_fake_quant): q = floorf(x * (1/scale) +
// 0.5f) clamped to [-2^(b-1), 2^(b-1) - 1], times scale; compiled without
// contraction, so the multiply and the add round separately as in the oracle.
__global__ void k_fake_quant(const float* __restrict__ x, float* __restrict__ y, size_t n,
                             float scale, float inv, float lo, float hi) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float q = floorf(x[i] * inv + 0.5f);
        if (q < lo) q = lo;
        if (q > hi) q = hi;
        y[i] = q * scale;
    }
}

// awq.c:135-161: one wave per (row, group).
__global__ void k_awq_quantize(const float* __restrict__ w, int8_t* __restrict__ q,
                               float* __restrict__ scales, size_t rows, size_t cols, size_t g) {
    size_t ng = (cols + g - 1) / g;
    size_t seg = blockIdx.x;
    for (; seg < rows * ng; seg += gridDim.x) {
        size_t r = seg / ng, j = seg % ng;
        size_t lo = j * g, hi = lo + g < cols ? lo + g : cols;
        const float* xr = w + r * cols;
        float m = 0.0f;
        for (size_t c = lo + threadIdx.x; c < hi; c += 64) m = nanless_max(m, fabsf(xr[c]));
        m = wave_max(m);
        float s = m < FLT_MIN ? 1.0f : m / 127.0f;
        float inv = 1.0f / s;
        if (threadIdx.x == 0) scales[r * ng + j] = s;
        for (size_t c = lo + threadIdx.x; c < hi; c += 64)
            q[r * cols + c] = (int8_t)clampi(round_i32(xr[c] * inv), -128, 127);
    }
}

// gptq.c:189-239 in closed form (the Cholesky "inverse" of I has unit
// diagonal and -0.0f below it, so error feedback adds signed zeros until a
// non-finite error appears, after which every later column of the group
// reads NaN): codes = clamp(roundf(w / scale)), columns after the first
// non-finite error -> code of NaN.  One wave per (row, group).
__global__ void k_gptq_quantize(const float* __restrict__ w, int8_t* __restrict__ q,
                                float* __restrict__ scales, int32_t* __restrict__ zeros,
                                size_t rows, size_t cols, size_t g, int qmin, int qmax) {
    size_t ng = (cols + g - 1) / g;
    for (size_t seg = blockIdx.x; seg < rows * ng; seg += gridDim.x) {
        size_t r = seg / ng, j = seg % ng;
        size_t lo = j * g, hi = lo + g < cols ? lo + g : cols;
        const float* xr = w + r * cols;
        float m = 0.0f;
        for (size_t c = lo + threadIdx.x; c < hi; c += 64) m = nanless_max(m, fabsf(xr[c]));
        m = wave_max(m);
        bool degenerate = m < FLT_MIN;
        float s = degenerate ? 1.0f : m / (float)qmax;
        float inv = 1.0f / s;
        if (threadIdx.x == 0) {
            scales[r * ng + j] = s;
            if (zeros) zeros[r * ng + j] = 0;
        }
        int first_bad = INT_MAX;
        if (!degenerate) {
            for (size_t c = lo + threadIdx.x; c < hi; c += 64) {
                float v = xr[c];
                float qv = (float)clampi(round_i32(v * inv), qmin, qmax) * s;
                float err = qv - v;
                if (!isfinite(err) && (int)(c - lo) < first_bad) first_bad = (int)(c - lo);
            }
            first_bad = wave_min_int(first_bad);
        }
        if (q) {
            for (size_t c = lo + threadIdx.x; c < hi; c += 64) {
                float v = (int)(c - lo) > first_bad ? __builtin_nanf("") : xr[c];
                q[r * cols + c] = (int8_t)clampi(round_i32(v / s), -128, 127);
            }
        }
    }
}

// awq.c:48-120: one wave per (row, 128-column group), columns in order; the
// lanes evaluate the candidate scales of one column concurrently, each with
// the reference's sequential loss sum, and the first strictly smallest loss
// wins.  The group lives in LDS and is updated in place as columns scale.
__global__ void __launch_bounds__(64) k_awq_scale_weights(float* __restrict__ w,
                                                         const float* __restrict__ act,
                                                         float* __restrict__ scale_out,
                                                         size_t rows, size_t cols) {
    __shared__ float seg[128];
    const size_t g = 128, ng = (cols + g - 1) / g;
    const int lane = threadIdx.x;
    for (size_t sidx = blockIdx.x; sidx < rows * ng; sidx += gridDim.x) {
        size_t r = sidx / ng, j = sidx % ng;
        size_t lo = j * g, len = (lo + g < cols ? lo + g : cols) - lo;
        float* row = w + r * cols + lo;
        for (size_t c = lane; c < len; c += 64) seg[c] = row[c];
        __syncthreads();
        for (size_t c = 0; c < len; c++) {
            float gm = 0.0f;
            for (size_t k = lane; k < len; k += 64) gm = nanless_max(gm, fabsf(seg[k]));
            gm = wave_max(gm);
            float best_s = 1.0f;
            if (!(gm < FLT_MIN)) {
                float a = act[lo + c];
                float alpha = a < 1.0f ? a : 1.0f;
                float step = (1.0f - alpha) / 20.0f;
                if (step < 0.001f) step = 0.001f;
                float best_loss = 1e20f;
                // candidates in chunks of 64: candidate i = alpha + step + ... (i adds)
                float s_chunk = alpha;          // value of candidate (chunk * 64)
                bool chunk_ok = s_chunk <= 1.0f;
                while (chunk_ok) {
                    float s = s_chunk;
                    bool ok = s <= 1.0f;
                    for (int i = 0; i < lane; i++) {
                        s = s + step;
                        ok = ok && (s <= 1.0f);
                    }
                    float loss = __builtin_nanf("");
                    if (ok) {
                        float inv_s = 1.0f / s;
                        float mq = 0.0f;
                        for (size_t k = 0; k < len; k++) mq = nanless_max(mq, fabsf(seg[k] * s));
                        float qs = mq < FLT_MIN ? 1.0f : mq / 127.0f;
                        float acc = 0.0f;
                        for (size_t k = 0; k < len; k++) {
                            float t = seg[k] * s;
                            int32_t qi = clampi(round_i32(t / qs), -128, 127);
                            float d = (float)qi * qs;
                            d = d * inv_s;
                            d = d - seg[k];
                            float sq = d * d;
                            acc = acc + sq;
                        }
                        loss = acc / (float)len;
                    }
                    // first strictly smaller loss in candidate order: minimum
                    // loss, ties to the lowest index; NaN never wins.
                    float bl = (ok && loss < best_loss) ? loss : INFINITY;
                    int bi = (ok && loss < best_loss) ? lane : INT_MAX;
                    for (int o = 32; o > 0; o >>= 1) {
                        float ol = __shfl_xor(bl, o);
                        int oi = __shfl_xor(bi, o);
                        if (ol < bl || (ol == bl && oi < bi)) { bl = ol; bi = oi; }
                    }
                    if (bi != INT_MAX) {
                        best_loss = bl;
                        best_s = __shfl(s, bi);
                    }
                    // next chunk starts 64 additions further on
                    float s_next = __shfl(s, 63) + step;
                    bool all_ok = __shfl((int)ok, 63) != 0;
                    chunk_ok = all_ok && (s_next <= 1.0f);
                    s_chunk = s_next;
                }
            }
            if (lane == 0) {
                float v = seg[c] * best_s;
                seg[c] = v;
                scale_out[r * cols + lo + c] = best_s;
            }
            __syncthreads();
        }
        for (size_t c = lane; c < len; c += 64) row[c] = seg[c];
        __syncthreads();
    }
}

// gptq.c:55-79: upper triangle accumulated sample by sample, then mirrored.
__global__ void k_hessian(float* __restrict__ h, const float* __restrict__ a, size_t n,
                          size_t dim) {
    size_t r = blockIdx.y * 16 + threadIdx.y, c = blockIdx.x * 16 + threadIdx.x;
    if (blockIdx.x < blockIdx.y) return;   // tile entirely below the diagonal
    if (r >= dim || c >= dim || c < r) return;
    float acc = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float p = a[i * dim + r] * a[i * dim + c];
        acc = acc + p;
    }
    h[r * dim + c] = acc;
    if (c != r) h[c * dim + r] = acc;
}

__global__ void k_hessian_reg(float* __restrict__ h, size_t dim) {
    float reg = 1e-5f * h[0];
    if (reg < 1e-8f) reg = 1e-5f;
    __syncthreads();
    for (size_t i = threadIdx.x; i < dim; i += blockDim.x) h[i * dim + i] = h[i * dim + i] + reg;
}

// gptq.c:134-172 with an arbitrary h_inv: sequential over columns inside one
// workgroup; w is updated in global memory between barriers.
__global__ void k_gptq_block(float* __restrict__ w, const float* __restrict__ hinv,
                             float* __restrict__ qw, float* __restrict__ out, size_t n,
                             int qmin, int qmax) {
    __shared__ float sh[16];
    __shared__ float coef_sh;
    __shared__ int apply_sh;
    float m = 0.0f;
    for (size_t i = threadIdx.x; i < n; i += blockDim.x) m = nanless_max(m, fabsf(w[i]));
    m = block_reduce(m, nanless_max, sh);
    if (m < FLT_MIN) {
        for (size_t i = threadIdx.x; i < n; i += blockDim.x) qw[i] = 0.0f;
        if (threadIdx.x == 0) {
            out[0] = 1.0f;
            out[1] = 0.0f;
        }
        return;
    }
    float s = m / (float)qmax;
    float inv = 1.0f / s;
    if (threadIdx.x == 0) {
        out[0] = s;
        out[1] = 0.0f;
    }
    for (size_t j = 0; j < n; j++) {
        if (threadIdx.x == 0) {
            float wj = w[j];
            float qv = (float)clampi(round_i32(wj * inv), qmin, qmax) * s;
            float err = qv - wj;
            qw[j] = qv;
            float hd = hinv[j * n + j];
            apply_sh = fabsf(hd) > 1e-10f;
            coef_sh = -err / hd;
        }
        __syncthreads();
        if (apply_sh) {
            float coef = coef_sh;
            for (size_t k = j + 1 + threadIdx.x; k < n; k += blockDim.x) {
                float p = coef * hinv[k * n + j];
                w[k] = w[k] + p;
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------- W4 (build-defined)
// a20 AWQ-style uint4: block per row, a wave per group (strided), zero
// nibbles gathered in LDS and written once per row.
__global__ void k_w4_awq_quantize(const float* __restrict__ w, uint32_t* __restrict__ qw,
                                  uint16_t* __restrict__ scales, uint32_t* __restrict__ qzeros,
                                  size_t N, size_t K, int group) {
    extern __shared__ uint8_t zsh[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    const size_t G = K / group, zw = (G + 7) / 8, kw = K / 8;
    for (size_t n = blockIdx.x; n < N; n += gridDim.x) {
        const float* xr = w + n * K;
        for (size_t j = wave; j < G; j += nwaves) {
            const float* x = xr + j * group;
            float lo = INFINITY, hi = -INFINITY;
            for (int i = lane; i < group; i += 64) {
                lo = nanless_min(lo, x[i]);
                hi = nanless_max(hi, x[i]);
            }
            lo = wave_min(lo);
            hi = wave_max(hi);
            float x0 = x[0];
            if (x0 != x0) lo = hi = x0;
            bool degenerate = hi - lo < FLT_MIN;
            uint16_t s16 = 0x3C00u;
            float s = 1.0f;
            int32_t z = 0;
            if (!degenerate) {
                s16 = w4_scale_f16((hi - lo) / 15.0f);
                s = f16_to_f32(s16);
                z = clampi(round_i32(-lo / s), 0, 15);
            }
            float zf = (float)z;
            for (int wd = lane; wd < group / 8; wd += 64) {
                uint32_t word = 0;
                if (!degenerate) {
#pragma unroll
                    for (int t = 0; t < 8; t++) {
                        float v = x[wd * 8 + t] / s;
                        word |= (uint32_t)clampi(round_i32(v + zf), 0, 15) << (4 * t);
                    }
                }
                qw[n * kw + (j * group) / 8 + wd] = word;
            }
            if (lane == 0) {
                scales[n * G + j] = s16;
                zsh[j] = (uint8_t)z;
            }
        }
        __syncthreads();
        for (size_t zi = threadIdx.x; zi < zw; zi += blockDim.x) {
            uint32_t word = 0;
            for (int t = 0; t < 8 && zi * 8 + t < G; t++) word |= (uint32_t)zsh[zi * 8 + t] << (4 * t);
            qzeros[n * zw + zi] = word;
        }
        __syncthreads();
    }
}

// a21 GPTQ act-order int4: block per row; group maxima and first-poisoned
// columns through LDS atomics (order-independent), then codes per word.
__global__ void k_w4_gptq_quantize(const float* __restrict__ w, const int32_t* __restrict__ g_idx,
                                   size_t G, uint32_t* __restrict__ qw,
                                   uint16_t* __restrict__ scales, size_t N, size_t K) {
    extern __shared__ uint32_t gsh[];   // [G] max bits, [G] first bad column
    uint32_t* gmax = gsh;
    uint32_t* gbad = gsh + G;
    for (size_t n = blockIdx.x; n < N; n += gridDim.x) {
        const float* xr = w + n * K;
        for (size_t j = threadIdx.x; j < G; j += blockDim.x) {
            gmax[j] = 0u;
            gbad[j] = 0xFFFFFFFFu;
        }
        __syncthreads();
        for (size_t k = threadIdx.x; k < K; k += blockDim.x) {
            float a = fabsf(xr[k]);
            if (a == a) atomicMax(&gmax[g_idx[k]], f2u(a));   // non-negative: bits order = value order
        }
        __syncthreads();
        for (size_t k = threadIdx.x; k < K; k += blockDim.x) {
            int32_t gj = g_idx[k];
            float m = u2f(gmax[gj]);
            if (m < FLT_MIN) continue;
            float s = m / 7.0f;
            float inv = 1.0f / s;
            float v = xr[k];
            float qv = (float)clampi(round_i32(v * inv), -7, 7) * s;
            float err = qv - v;
            if (!isfinite(err)) atomicMin(&gbad[gj], (uint32_t)k);
        }
        __syncthreads();
        for (size_t j = threadIdx.x; j < G; j += blockDim.x) {
            float m = u2f(gmax[j]);
            scales[n * G + j] = w4_scale_f16(m < FLT_MIN ? 1.0f : m / 7.0f);
        }
        for (size_t wd = threadIdx.x; wd < K / 8; wd += blockDim.x) {
            uint32_t word = 0;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                size_t k = wd * 8 + t;
                int32_t gj = g_idx[k];
                float m = u2f(gmax[gj]);
                float s = m < FLT_MIN ? 1.0f : m / 7.0f;
                float v = (uint32_t)k > gbad[gj] ? __builtin_nanf("") : xr[k];
                int32_t c = clampi(round_i32(v / s), -128, 127);
                word |= (uint32_t)(clampi(c, -8, 7) + 8) << (4 * t);
            }
            qw[n * (K / 8) + wd] = word;
        }
        __syncthreads();
    }
}

}  // namespace

// ------------------------------------------------------------- launchers
extern "C" {

// FP8 scalar codecs of the reference API (quantize_fp8.c:41-100, 146-201):
// pure bit manipulation, evaluated on the host with the kernels' own codec.
uint8_t SNEPPX_float_to_fp8_e4m3(float value) { return fp8_e4m3_encode(value); }
float SNEPPX_fp8_e4m3_to_float(uint8_t fp8) { return fp8_e4m3_decode(fp8); }
uint8_t SNEPPX_float_to_fp8_e5m2(float value) { return fp8_e5m2_encode(value); }
float SNEPPX_fp8_e5m2_to_float(uint8_t fp8) { return fp8_e5m2_decode(fp8); }

int snx_reduce_parts(size_t n) { return grid_for(n, kBlock * 16, kMaxParts); }

int snx_k_absmax(const float* x, size_t n, float* part, int nparts, void* st) {
    k_absmax<<<nparts, kBlock, 0, S(st)>>>(x, n, part);
    return snx_launch_check("k_absmax");
}

int snx_k_minmax(const float* x, size_t n, float* part, int nparts, void* st) {
    k_minmax<<<nparts, kBlock, 0, S(st)>>>(x, n, part);
    return snx_launch_check("k_minmax");
}

int snx_k_finalize_scale(const float* part, int nparts, int kind, const float* x, float* rec,
                         float* scale_out, void* st) {
    k_finalize<<<1, kBlock, 0, S(st)>>>(part, nparts, kind, x, rec, scale_out);
    return snx_launch_check("k_finalize");
}

int snx_k_quant_int8_sym(const float* x, int8_t* q, size_t n, const float* rec, void* st) {
    k_quant_int8_sym<<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(x, q, n, rec);
    return snx_launch_check("k_quant_int8_sym");
}

int snx_k_quant_int8_modelzoo(const float* x, int8_t* q, size_t n, const float* rec, void* st) {
    k_quant_int8_modelzoo<<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(x, q, n, rec);
    return snx_launch_check("k_quant_int8_modelzoo");
}

int snx_k_dequant_int8_sym(const int8_t* q, float* y, size_t n, float scale, void* st) {
    k_dequant_int8_sym<<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(q, y, n, scale);
    return snx_launch_check("k_dequant_int8_sym");
}

int snx_k_quant_int8_asym(const float* x, int8_t* q, size_t n, const float* rec, void* st) {
    k_quant_int8_asym<<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(x, q, n, rec);
    return snx_launch_check("k_quant_int8_asym");
}

int snx_k_dequant_int8_asym(const int8_t* q, float* y, size_t n, float scale, int32_t zp, void* st) {
    k_dequant_int8_asym<<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(q, y, n, scale, (float)zp);
    return snx_launch_check("k_dequant_int8_asym");
}

int snx_k_quant_int4_sym(const float* x, uint8_t* p, size_t n, const float* rec, void* st) {
    k_quant_int4_sym<<<grid_for((n + 1) / 2, kBlock * 4), kBlock, 0, S(st)>>>(x, p, n, rec);
    return snx_launch_check("k_quant_int4_sym");
}

int snx_k_dequant_int4_sym(const uint8_t* p, float* y, size_t n, float scale, void* st) {
    k_dequant_int4_sym<<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(p, y, n, scale);
    return snx_launch_check("k_dequant_int4_sym");
}

int snx_k_fp8_encode(const float* x, uint8_t* c, size_t n, int fmt, const float* rec, void* st) {
    if (n == 0) return 0;
    if (fmt == 0)
        k_fp8_encode<0><<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(x, c, n, rec);
    else
        k_fp8_encode<1><<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(x, c, n, rec);
    return snx_launch_check("k_fp8_encode");
}

int snx_k_fp8_decode(const uint8_t* c, float* y, size_t n, int fmt, void* st) {
    if (n == 0) return 0;
    if (fmt == 0)
        k_fp8_decode<0><<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(c, y, n);
    else
        k_fp8_decode<1><<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(c, y, n);
    return snx_launch_check("k_fp8_decode");
}

int snx_k_quant_int8_rows(const float* x, int8_t* q, float* scales, size_t rows, size_t cols,
                          int rne, void* st) {
    int grid = (int)(rows < 65536 ? rows : 65536);
    if (rne)
        k_quant_int8_rows<true, float><<<grid, kBlock, 0, S(st)>>>(x, q, scales, rows, cols);
    else
        k_quant_int8_rows<false, float><<<grid, kBlock, 0, S(st)>>>(x, q, scales, rows, cols);
    return snx_launch_check("k_quant_int8_rows");
}

int snx_k_quant_int8_rows_bf16(const uint16_t* x, int8_t* q, float* scales, size_t rows,
                               size_t cols, void* st) {
    int grid = (int)(rows < 65536 ? rows : 65536);
    k_quant_int8_rows<false, uint16_t><<<grid, kBlock, 0, S(st)>>>(x, q, scales, rows, cols);
    return snx_launch_check("k_quant_int8_rows_bf16");
}

int snx_k_quant_rows_bf16_fast(const uint16_t* x, int8_t* q, float* scales, size_t rows, size_t cols,
                               void* st) {
    if (cols % 8 || cols > 8192 || ((uintptr_t)x & 15u) || ((uintptr_t)q & 7u))
        return snx_k_quant_int8_rows_bf16(x, q, scales, rows, cols, st);
    const int grid = (int)(rows < 65536 ? rows : 65536);
    if (cols <= 2048)
        k_quant_rows_bf16_reg<1><<<grid, 256, 0, S(st)>>>(x, q, scales, rows, (int)cols);
    else if (cols <= 4096)
        k_quant_rows_bf16_reg<2><<<grid, 256, 0, S(st)>>>(x, q, scales, rows, (int)cols);
    else
        k_quant_rows_bf16_reg<4><<<grid, 256, 0, S(st)>>>(x, q, scales, rows, (int)cols);
    return snx_launch_check("k_quant_rows_bf16_reg");
}

int snx_k_absmax_bf16(const uint16_t* x, size_t n, float* part, int nparts, void* st) {
    if (n % 8 == 0 && ((uintptr_t)x & 15u) == 0)
        k_absmax_bf16_v8<<<nparts, kBlock, 0, S(st)>>>(x, n / 8, part);
    else
        k_absmax<uint16_t><<<nparts, kBlock, 0, S(st)>>>(x, n, part);
    return snx_launch_check("k_absmax_bf16");
}

int snx_k_fp8_encode_bf16_pt(const uint16_t* x, uint8_t* c, size_t n, const float* part, int nparts,
                             float* scale_out, void* st) {
    k_fp8_encode_bf16_v8<<<grid_for(n / 8, kBlock * 2), kBlock, 0, S(st)>>>(x, c, n / 8, part, nparts, scale_out);
    return snx_launch_check("k_fp8_encode_bf16_v8");
}

int snx_k_fp8_encode_bf16(const uint16_t* x, uint8_t* c, size_t n, const float* rec, void* st) {
    if (n == 0) return 0;
    k_fp8_encode<0, uint16_t><<<grid_for(n, kBlock * 4), kBlock, 0, S(st)>>>(x, c, n, rec);
    return snx_launch_check("k_fp8_encode_bf16");
}

int snx_k_fake_quant(const float* x, float* y, size_t n, float scale, int bits, void* st) {
    const float lo = (float)(-(1 << (bits - 1))), hi = (float)((1 << (bits - 1)) - 1);
    const size_t blocks = (n + kBlock - 1) / kBlock;
    const int grid = (int)(blocks < 65536 ? blocks : 65536);
    k_fake_quant<<<grid, kBlock, 0, S(st)>>>(x, y, n, scale, 1.0f / scale, lo, hi);
    return snx_launch_check("k_fake_quant");
}

int snx_k_awq_quantize(const float* w, int8_t* q, float* scales, size_t rows, size_t cols,
                       size_t group, void* st) {
    size_t segs = rows * ((cols + group - 1) / group);
    int grid = (int)(segs < (1u << 20) ? segs : (1u << 20));
    k_awq_quantize<<<grid, 64, 0, S(st)>>>(w, q, scales, rows, cols, group);
    return snx_launch_check("k_awq_quantize");
}

int snx_k_gptq_quantize(const float* w, int8_t* q, float* scales, int32_t* zeros, size_t rows,
                        size_t cols, size_t group, int bits, int sym, void* st) {
    int qmax = (1 << (bits - 1)) - 1, qmin = -qmax;
    if (!sym) {
        qmax = (1 << bits) - 1;
        qmin = 0;
    }
    size_t segs = rows * ((cols + group - 1) / group);
    int grid = (int)(segs < (1u << 20) ? segs : (1u << 20));
    k_gptq_quantize<<<grid, 64, 0, S(st)>>>(w, q, scales, zeros, rows, cols, group, qmin, qmax);
    return snx_launch_check("k_gptq_quantize");
}

int snx_k_awq_scale_weights(float* w, const float* act, float* scale_out, size_t rows,
                            size_t cols, void* st) {
    size_t segs = rows * ((cols + 127) / 128);
    int grid = (int)(segs < (1u << 20) ? segs : (1u << 20));
    k_awq_scale_weights<<<grid, 64, 0, S(st)>>>(w, act, scale_out, rows, cols);
    return snx_launch_check("k_awq_scale_weights");
}

int snx_k_gptq_hessian(float* h, const float* act, size_t n, size_t dim, void* st) {
    size_t t = (dim + 15) / 16;
    if (t > 65535) {
        snx_set_error("gptq_compute_hessian: dim %zu too large", dim);
        return -1;
    }
    k_hessian<<<dim3((unsigned)t, (unsigned)t), dim3(16, 16), 0, S(st)>>>(h, act, n, dim);
    if (snx_launch_check("k_hessian")) return -1;
    k_hessian_reg<<<1, kBlock, 0, S(st)>>>(h, dim);
    return snx_launch_check("k_hessian_reg");
}

int snx_k_gptq_block(float* w, const float* h_inv, float* qw, float* out, size_t n, int bits,
                     int sym, void* st) {
    int qmax = (1 << (bits - 1)) - 1, qmin = -qmax;
    if (!sym) {
        qmax = (1 << bits) - 1;
        qmin = 0;
    }
    k_gptq_block<<<1, kBlock, 0, S(st)>>>(w, h_inv, qw, out, n, qmin, qmax);
    return snx_launch_check("k_gptq_block");
}

int snx_k_w4_awq_quantize(const float* w, uint32_t* qw, uint16_t* scales, uint32_t* qzeros,
                          size_t N, size_t K, int group, void* st) {
    size_t G = K / (size_t)group;
    int grid = (int)(N < 65536 ? N : 65536);
    k_w4_awq_quantize<<<grid, kBlock, G + 8, S(st)>>>(w, qw, scales, qzeros, N, K, group);
    return snx_launch_check("k_w4_awq_quantize");
}

int snx_k_w4_gptq_quantize(const float* w, const int32_t* g_idx, size_t G, uint32_t* qw,
                           uint16_t* scales, size_t N, size_t K, void* st) {
    if (G > 4096) {
        snx_set_error("w4 gptq: %zu groups exceed the 4096 the kernel stages in LDS", G);
        return -1;
    }
    int grid = (int)(N < 65536 ? N : 65536);
    k_w4_gptq_quantize<<<grid, kBlock, 2 * G * sizeof(uint32_t), S(st)>>>(w, g_idx, G, qw, scales, N, K);
    return snx_launch_check("k_w4_gptq_quantize");
}

}  // extern "C"
