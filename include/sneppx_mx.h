/*
 * sneppx_mx.h - MX (micro-scaling) formats on gfx950.
 *
 * The reference implements MX encode/decode in Python/numpy
 * (bindings/python/SneppX_ALG/interface_bindings/mx_formats.py: quantize_mx,
 * dequantize_mx, formats at :53-72).  These entry points compute the same
 * packed codes and int8 scale exponents on the device, bit for bit, for 2-D
 * tensors blocked along the last axis (the reference's default
 * block_axis=-1): a [rows][cols] float32 tensor is padded with zeros to a
 * multiple of the block size per row, every block of `block_size` elements
 * shares a power-of-two exponent (int8, one per block, [rows][nblocks]), and
 * the codes of all padded elements form one little-endian bitstream in
 * row-major order.  With one exponent per tensor (NVFP4's default, or
 * block_size -1) the codes of the rows*cols elements are packed without
 * padding.
 *
 * The reference's element formats use every exponent field for finite values
 * (E4M3 reaches 480, E5M2 114688), unlike the OCP formats of the gfx950
 * matrix cores; its fp4/fp6 formats coincide with OCP's, so only MXFP4 /
 * MXFP6 codes decode on the matrix cores to the reference's values.
 *
 * Returns 0 / -1 (text in SNEPPX_qlinear_last_error()).
 */
#ifndef SNEPPX_MX_H
#define SNEPPX_MX_H

#include <stddef.h>
#include <stdint.h>

#include "sneppx_qlinear.h"

#ifdef __cplusplus
extern "C" {
#endif

/* MXFormat of mx_formats.py:38-45, in the order of MX_FORMATS (:53-72) */
typedef enum {
    SNEPPX_MXFP8_E4M3 = 0,
    SNEPPX_MXFP8_E5M2 = 1,
    SNEPPX_MXFP6_E3M2 = 2,
    SNEPPX_MXFP6_E2M3 = 3,
    SNEPPX_MXFP4_E2M1 = 4,
    SNEPPX_NVFP4_E2M1 = 5
} SNEPPXMXFormat;

/* Bits per element and default block size (0 = one scale per tensor). */
int SNEPPX_mx_bits(SNEPPXMXFormat fmt);
int SNEPPX_mx_default_block(SNEPPXMXFormat fmt);

/* Sizes of the outputs for a [rows][cols] tensor; block_size 0 picks the
 * format's default (so NVFP4 is per tensor).  -1 / 0 on a bad format or a
 * block size that is not a multiple of 8. */
size_t SNEPPX_mx_packed_bytes(SNEPPXMXFormat fmt, size_t rows, size_t cols, int block_size);
size_t SNEPPX_mx_scale_count(SNEPPXMXFormat fmt, size_t rows, size_t cols, int block_size);

/* quantize_mx (mx_formats.py:144-201).  x float32 [rows][cols] (device),
 * packed uint8 and scales int8 (device) of the sizes above.  block_size: 0 =
 * the format's default, otherwise a positive multiple of 8, or -1 for one
 * scale per tensor.  Per-tensor quantization returns -1 where the reference
 * raises (an infinite peak, an exponent outside int8) and waits for the
 * device (the exponent is checked on the host). */
int SNEPPX_dev_quantize_mx(const float* x, uint8_t* packed, int8_t* scales, size_t rows,
                           size_t cols, SNEPPXMXFormat fmt, int block_size, SNEPPXStream stream);

/* dequantize_mx (mx_formats.py:204-222): y float32 [rows][cols] = the
 * reference's float64 result rounded to float32 (exact unless it overflows
 * or underflows float32). */
int SNEPPX_dev_dequantize_mx(const uint8_t* packed, const int8_t* scales, float* y, size_t rows,
                             size_t cols, SNEPPXMXFormat fmt, int block_size, SNEPPXStream stream);

/* MXFP4 x MXFP4 linear on the gfx950 scaled matrix cores (no reference
 * counterpart; the reference stops at encode/decode): out[m][n] =
 * sum_k A[m][k] W[n][k] where A [M][K] and W [N][K] are MXFP4 tensors as
 * SNEPPX_dev_quantize_mx writes them with the default block of 32 (packed
 * [rows][K/2] bytes, exponents [rows][K/32]).  out is bf16 or fp32 [M][N]
 * (out_dtype SNEPPX_BFLOAT16 / SNEPPX_FLOAT32), fp32 accumulation; the fp4
 * products are exact on the matrix cores.  K % 64 == 0. */
int SNEPPX_qlinear_mxfp4_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W,
                              const int8_t* sW, void* out, SNEPPXDtype out_dtype, size_t M,
                              size_t N, size_t K, SNEPPXStream stream);

/* The same linear for every MX format (no reference counterpart):
 * A [M][K] and W [N][K] both in `fmt` (MXFP8 E4M3 / E5M2, MXFP6 E3M2 / E2M3,
 * MXFP4, and NVFP4 with its per-tensor exponent, sA / sW one int8 each, as
 * SNEPPX_qlinear_mx_gemm_bs with block 0), as SNEPPX_dev_quantize_mx writes
 * them with the default block;
 * out bf16 or fp32 [M][N], fp32 accumulation on the scaled f8f6f4 matrix
 * cores (the block exponents go in as their E8M0 scales).  FP6 and FP4 codes
 * are the matrix cores' own.  The reference's FP8 codes with an all-ones
 * exponent field (E4M3 0x7F = 480, E5M2 65536 .. 114688) are not, so MXFP8
 * operands first pass through SNEPPX_mx_to_mfma into the calling thread's
 * workspace (one read and write of A and W per call).  MXFP8/6: K % 128 == 0,
 * exponents 4-byte aligned; MXFP4 as SNEPPX_qlinear_mxfp4_gemm.  In every MX
 * GEMM an exponent of -128 (the reference's int8 cast gives it to blocks
 * whose peak lies near 2^-128 times the format's largest element) is taken
 * as -127: the matrix cores' E8M0 scale has no 2^-128. */
int SNEPPX_qlinear_mx_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                           SNEPPXMXFormat fmt, void* out, SNEPPXDtype out_dtype, size_t M,
                           size_t N, size_t K, SNEPPXStream stream);

/* SNEPPX_qlinear_mx_gemm for operands quantized with any block the
 * matrix cores can scale exactly (no reference counterpart; the block rule
 * is SNEPPX_dev_quantize_mx's, mx_formats.py:147-150,165): block_size 0 is
 * the format's default (32, or per tensor for NVFP4), a negative one per
 * tensor, a positive one a multiple of 32 dividing K.  Per tensor, sA and sW
 * are one int8 each and every 32-element block takes them as its scales
 * (mx_formats.py:165-172, 199-203); a block of 32 r repeats each exponent for
 * its r pieces of 32.  Blocks that are no multiple of 32 (e.g. 16) return -1:
 * the matrix cores scale 32 elements with one exponent.  NVFP4 runs the
 * MXFP4 kernels (the same E2M1 codes).  E2M1 per tensor with K % 256 == 0
 * and M, N >= 128 passes the two exponents to every MFMA as constant scales
 * (the product's exponent split as ceil / floor of its half, each at least
 * -127) and needs no workspace; other cases rewrite the exponents into the
 * calling thread's workspace (M + N rows of K/32 bytes). */
int SNEPPX_qlinear_mx_gemm_bs(const uint8_t* A, const int8_t* sA, const uint8_t* W,
                              const int8_t* sW, SNEPPXMXFormat fmt, int block_size, void* out,
                              SNEPPXDtype out_dtype, size_t M, size_t N, size_t K,
                              SNEPPXStream stream);

/* Reference MX codes of a [rows][cols] block-32 tensor -> codes and
 * exponents the matrix cores decode to the same values (no reference
 * counterpart).  MXFP8: every block holding an all-ones-exponent code is
 * re-encoded one binade lower with its exponent + 1 -- exact, except that
 * elements worth an odd number of the smallest subnormal at the new exponent
 * round half to even (counted into *rounded, a device counter, when given);
 * a block already at exponent 127 is left as it is.  Other formats are copied.
 * For weights converted once and kept: SNEPPX_qlinear_mx_gemm_mfma then skips
 * the per-call conversion.  cols % 32 == 0. */
int SNEPPX_mx_to_mfma(const uint8_t* packed, const int8_t* scales, uint8_t* out_packed,
                      int8_t* out_scales, size_t rows, size_t cols, SNEPPXMXFormat fmt,
                      unsigned int* rounded, SNEPPXStream stream);

/* SNEPPX_qlinear_mx_gemm on operands already in matrix-core form
 * (SNEPPX_mx_to_mfma output, or FP6 / FP4 tensors as quantized). */
int SNEPPX_qlinear_mx_gemm_mfma(const uint8_t* A, const int8_t* sA, const uint8_t* W,
                                const int8_t* sW, SNEPPXMXFormat fmt, void* out,
                                SNEPPXDtype out_dtype, size_t M, size_t N, size_t K,
                                SNEPPXStream stream);

#ifdef __cplusplus
}
#endif

#endif /* SNEPPX_MX_H */
