// codec.h - scalar codecs shared by the gfx950 kernels and the host-side FP8
// scalar API.  Every function reproduces the reference's arithmetic bit for
// bit; the comment on each names the reference lines.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define SNX_HD __host__ __device__ __forceinline__

namespace snx {

SNX_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
SNX_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// (int)roundf(v) with the value the reference's x86-64 build produces for NaN
// and out-of-range results (cvttss2si's INT32_MIN).  roundf: ties away from 0.
SNX_HD int32_t round_i32(float v) {
    float r = roundf(v);
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int32_t)r : INT32_MIN;
}

// The same conversion with ties to even (rintf under the default rounding
// mode): the "round-half-even" reading of the C1 config, offered as an
// explicit option next to the reference's roundf.
SNX_HD int32_t rne_i32(float v) {
    float r = rintf(v);
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int32_t)r : INT32_MIN;
}

SNX_HD int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

// quantize_fp8.c:41-69 (mantissa truncated; exponent > 8, Inf, NaN -> 0x78)
SNX_HD uint8_t fp8_e4m3_encode(float v) {
    uint32_t u = f2u(v);
    uint32_t sign = (u >> 24) & 0x80u;
    int e = (int)((u >> 23) & 0xFFu) - 127;
    if (e == 128) return (uint8_t)(sign | 0x78u);
    if (e == -127 || e < -6) return (uint8_t)sign;
    if (e > 8) return (uint8_t)(sign | 0x78u);
    return (uint8_t)(sign | (uint32_t)(e + 7) << 3 | ((u >> 20) & 7u));
}

// quantize_fp8.c:78-100 (field 15 -> Inf/NaN; 0x00 and 0x80 -> +0)
SNX_HD float fp8_e4m3_decode(uint8_t c) {
    uint32_t field = (c >> 3) & 15u, m = c & 7u, sign = (uint32_t)(c & 0x80u) << 24;
    if (field == 15u) return m ? u2f(0x7FC00000u) : u2f(sign | 0x7F800000u);
    if ((c & 0x7Fu) == 0) return 0.0f;
    return u2f(sign | (field + 120u) << 23 | m << 20);
}

// quantize_fp8.c:146-172 (keeps mantissa bit 22 only, in code bit 0)
SNX_HD uint8_t fp8_e5m2_encode(float v) {
    uint32_t u = f2u(v);
    uint32_t sign = (u >> 24) & 0x80u;
    int e = (int)((u >> 23) & 0xFFu) - 127;
    if (e == 128) return (uint8_t)(sign | 0x7Cu);
    if (e == -127 || e < -14) return (uint8_t)sign;
    if (e > 15) return (uint8_t)(sign | 0x7Cu);
    return (uint8_t)(sign | (uint32_t)(e + 15) << 2 | ((u >> 22) & 1u));
}

// quantize_fp8.c:180-201
SNX_HD float fp8_e5m2_decode(uint8_t c) {
    uint32_t field = (c >> 2) & 31u, m = c & 3u, sign = (uint32_t)(c & 0x80u) << 24;
    if (field == 31u) return m ? u2f(0x7FC00000u) : u2f(sign | 0x7F800000u);
    if ((c & 0x7Fu) == 0) return 0.0f;
    return u2f(sign | (field + 112u) << 23 | m << 21);
}

// IEEE binary16 from fp32, round to nearest even.
SNX_HD uint16_t f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    uint32_t h, rest, half;
    if (a >= 0x38800000u) {
        h = ((a >> 23) - 112u) << 10 | ((a >> 13) & 0x3FFu);
        rest = a & 0x1FFFu;
        half = 0x1000u;
    } else {
        if (a <= 0x33000000u) return (uint16_t)sign;
        uint32_t full = (a & 0x7FFFFFu) | 0x800000u, sh = 126u - (a >> 23);
        h = full >> sh;
        rest = full & ((1u << sh) - 1u);
        half = 1u << (sh - 1u);
    }
    if (rest > half || (rest == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

SNX_HD float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3FFu;
    if (e == 31u) return u2f(sign | 0x7F800000u | m << 13);
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f;
        return sign ? -v : v;
    }
    return u2f(sign | (e + 112u) << 23 | m << 13);
}

// Device kernels: the same value with one v_cvt_f32_f16 (exact for every
// fp16, subnormals included: gfx9 keeps fp16 denormals).
__device__ __forceinline__ float f16_dev(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Stored W4 scale: fp16, kept positive-finite (underflow -> 2^-24, overflow -> 65504).
SNX_HD uint16_t w4_scale_f16(float s) {
    uint16_t h = f32_to_f16(s);
    if ((h & 0x7FFFu) == 0) return 1u;
    if ((h & 0x7FFFu) == 0x7C00u) return (uint16_t)((h & 0x8000u) | 0x7BFFu);
    return h;
}

SNX_HD uint16_t f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

SNX_HD float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

// Output conversion of the linear kernels: gfx950's v_cvt_pk_bf16_f32 (round
// to nearest even, NaN stays NaN) -- the same value as f32_to_bf16 for every
// non-NaN input.
__device__ __forceinline__ uint16_t bf16_out(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two outputs in one v_cvt_pk_bf16_f32: lo in bits 0..15, hi in 16..31 (each
// the value bf16_out gives).
__device__ __forceinline__ uint32_t bf16x2_out(float lo, float hi) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{lo, hi}, b2));
}

// SiLU(g) * u as the fused SwiGLU epilogue computes it: the exponential and
// the reciprocal on the hardware's fast approximations (about 1 ulp each,
// far below the bf16 rounding of the result).  Large negative g gives
// exp = inf, rcp = 0 and a zero product; NaN propagates.
__device__ __forceinline__ float silu_mul_fast(float g, float u) {
    return g * u * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

}  // namespace snx
