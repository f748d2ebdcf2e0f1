/*
 * sneppx_qlinear.h - device-pointer quantizers and quantized linears (gfx950).
 *
 * The reference has no GEMV/GEMM on its quantized path (its linears are fp32
 * matmuls, kernel/tensor/tensor.c:1753-1828 called from
 * kernel/attention/attention.c:366-368,433,500-502,584 and
 * kernel/inference/inference_engine.c:264).  These entry points are the new
 * MI355X path in the reference's style: plain C types, 0 on success, -1 on
 * error, caller-allocated outputs.  Unlike the host API in
 * sneppx_quantization.h, every pointer here is a DEVICE pointer and every call
 * is asynchronous on `stream` (a hipStream_t; NULL is the default stream).
 *
 * Layouts (row-major; W is [N, K], output-major, y = x . W^T as in the
 * reference's Python QuantizedLinear, bindings/python/.../quantization.py:451):
 *   W8     qweight int8 [N][K], scales fp32 [N]  (SNEPPX_quantize_int8_channel)
 *   W4     qweight uint32 [N][K/8], element k at bits 4*(k%8) (the reference's
 *          int4 nibble order, quantize_int8.c:206-216, read as little-endian
 *          words); scales fp16 [N][G]; qzeros uint32 [N][ceil(G/8)], group j at
 *          bits 4*(j%8), or NULL for symmetric codes with implicit zero 8.
 *          Groups are `group` contiguous columns, or given per column by
 *          g_idx int32 [K] (GPTQ act-order) with G groups.
 *   x/y    bf16 (uint16 bit patterns) or fp32 as stated per function.
 *   bias   fp32 [N] or NULL: every linear computes y = x . W^T + bias, the
 *          bias added to the fp32 result before the output is rounded (the
 *          `out = out + self.bias` of QuantizedLinear.forward,
 *          bindings/python/.../quantization.py:451-454).
 * Failure text: SNEPPX_qlinear_last_error() (thread-local, last failing call).
 */
#ifndef SNEPPX_QLINEAR_H
#define SNEPPX_QLINEAR_H

#include <stddef.h>
#include <stdint.h>

#include "sneppx_quantization.h"

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t; NULL = default stream */
typedef void* SNEPPXStream;

/* No reference counterpart: last error of this thread, "" if none. */
const char* SNEPPX_qlinear_last_error(void);

/* No reference counterpart, for callers that destroy streams: frees
 * (ordered after the work already queued on `stream`) the scratch
 * workspaces the calling thread holds for `stream` and those that ended
 * threads left on it.  Call it before hipStreamDestroy.  Workspaces are
 * otherwise kept per (device, stream, slot) for each host thread and pass to
 * a later thread when their thread ends, so they do not grow with the number
 * of threads that ever called.  Returns 0. */
int SNEPPX_qlinear_release_workspaces(SNEPPXStream stream);

/* ---- device quantizers (bit-exact with the host API / reference) ------- */

/* Device form of SNEPPX_quantize_int8_channel (quantize_int8.c:157-177):
 * per-row symmetric int8 with scale max|row|/127.  Used for C1/C4 weights
 * (per output channel) and C4 activations (per token = per row). */
int SNEPPX_dev_quantize_int8_channel(const float* in, int8_t* q, float* scales,
                                     size_t rows, size_t cols, SNEPPXStream stream);

/* Rounding of the quantizers' x * (1/scale).  SNEPPX_ROUND_HALF_AWAY is the
 * reference's roundf (quantize_int8.c:61,172) and the default everywhere;
 * SNEPPX_ROUND_HALF_EVEN is offered for callers that specify ties to even. */
typedef enum { SNEPPX_ROUND_HALF_AWAY = 0, SNEPPX_ROUND_HALF_EVEN = 1 } SNEPPXRounding;

/* SNEPPX_dev_quantize_int8_channel with a choice of rounding (no reference
 * counterpart for SNEPPX_ROUND_HALF_EVEN); scales are identical in both. */
int SNEPPX_dev_quantize_int8_channel_rounding(const float* in, int8_t* q, float* scales,
                                              size_t rows, size_t cols, SNEPPXRounding rounding,
                                              SNEPPXStream stream);

/* Device form of SNEPPX_tensor_fake_quant (kernel/tensor/tensor.c:2180-2195,
 * the QAT forward): out = clamp(floorf(in * (1/scale) + 0.5f), -2^(b-1),
 * 2^(b-1) - 1) * scale over n floats (in may equal out).  -1 for scale <= 0 or
 * bits outside [2, 16], as the reference's NULL return. */
int SNEPPX_dev_fake_quant(const float* in, float* out, size_t n, float scale, int bits,
                          SNEPPXStream stream);

/* W4 AWQ-style asymmetric uint4 (build-defined, generalises
 * quantize_int8.c:98-123 to 4 bits with a stored fp16 scale):
 * per (row, group): s = fp16((max-min)/15), z = clamp(roundf(-min/s), 0, 15),
 * q = clamp(roundf(w/s + z), 0, 15).  K % 8 == 0, K % group == 0. */
int SNEPPX_dev_quantize_w4_awq(const float* w, uint32_t* qweight, uint16_t* scales,
                               uint32_t* qzeros, size_t N, size_t K, int group,
                               SNEPPXStream stream);

/* GPTQ act-order symmetric int4 (build-defined; equals gptq.c:189-239 with
 * bits 4, sym 1, applied to the columns of each g_idx group in ascending k):
 * codes c in [-7, 7] stored as c + 8; scale max|w_group|/7 stored as fp16. */
int SNEPPX_dev_quantize_w4_gptq(const float* w, const int32_t* g_idx, size_t G,
                                uint32_t* qweight, uint16_t* scales,
                                size_t N, size_t K, SNEPPXStream stream);

/* Per-tensor scaled FP8 E4M3 with the reference encoder (quantize_fp8.c:41-69):
 * s = max|x|/240 (1 when below FLT_MIN), code = e4m3(x / s), a correctly
 * rounded division (not x * (1/s): the two differ in the last bit, which the
 * truncating encoder can turn into a whole code step).  *scale_out is a
 * device float. */
int SNEPPX_dev_quantize_fp8_e4m3_scaled(const float* in, uint8_t* out, float* scale_out,
                                        size_t n, SNEPPXStream stream);

/* ---- quantized linears ---------------------------------------------------- */

/* C1: W8 weight-only, fp32 activations: y[m][n] = s[n] * sum_k x[m][k]*q[n][k]
 * (+ bias[n]) in fp32.  x fp32 [M][K], y fp32 [M][N].  Decode GEMV, HBM-bound. */
int SNEPPX_qlinear_w8_gemv(const float* x, const int8_t* qweight, const float* scales,
                           const float* bias, float* y, size_t M, size_t N, size_t K,
                           SNEPPXStream stream);

/* C2/C3/C5: W4A16.  x bf16 [M][K]; y [M][N] in y_dtype (SNEPPX_BFLOAT16 or
 * SNEPPX_FLOAT32); fp32 accumulation.  qzeros NULL => symmetric zero 8.
 * g_idx NULL => contiguous groups of `group` columns; otherwise g_idx[k] in
 * [0, G).  Small M runs the decode GEMV; large M the MFMA prefill GEMM. */
int SNEPPX_qlinear_w4a16(const uint16_t* x, const uint32_t* qweight, const uint16_t* scales,
                         const uint32_t* qzeros, const int32_t* g_idx, size_t G,
                         const float* bias, void* y, SNEPPXDtype y_dtype, size_t M, size_t N,
                         size_t K, int group, SNEPPXStream stream);

/* Allocation-free form of SNEPPX_qlinear_w4a16 (no counterpart in the
 * reference).  For callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * Same arguments, dispatch and results (bit-identical) as
 * SNEPPX_qlinear_w4a16, with one exception: where the allocating entry point
 * splits the prefill GEMM's K into spans (few output tiles, e.g. one GPU's
 * tensor-parallel QKV shard, or the tiles past the last full round of CUs,
 * e.g. the Llama-3-8B QKV projection at 1849 tokens), this one runs that
 * GEMM whole-K, the same
 * product with another fp32 summation order, so a bf16 output can differ
 * in its last bit.  The scratch the split-K decode and the prefill
 * GEMM need (fp32 partials, prepared activations) comes from one static
 * device array of SNEPPX_NOALLOC_SCRATCH_BYTES per GPU, held from the first
 * call on that GPU until the process ends, instead of a workspace.  A call
 * that needs more scratch than that returns -1 with the reason (for
 * example split-K partials K/1024 * M * N * 4 bytes, prefill 2 M K bytes and
 * more).  Every call on a GPU shares its array: calls that overlap on one GPU
 * (two streams, two threads) race on it and must be serialised by the
 * caller.  Nothing in the array needs to start at zero. */
#define SNEPPX_NOALLOC_SCRATCH_BYTES (32u << 20)
int SNEPPX_qlinear_w4a16_noalloc(const uint16_t* x, const uint32_t* qweight,
                                 const uint16_t* scales, const uint32_t* qzeros,
                                 const int32_t* g_idx, size_t G, const float* bias, void* y,
                                 SNEPPXDtype y_dtype, size_t M, size_t N, size_t K, int group,
                                 SNEPPXStream stream);

/* C3 fast path, step 1 (once per layer, at load time): GPTQ act-order
 * weights (qweight in column order k, g_idx int32 [K]) -> group-contiguous
 * order.  perm (uint16 [K], device) receives the stable argsort of g_idx and
 * qweight_sorted[n] holds column perm[k'] of row n at position k'.  Every
 * group must hold exactly K/G columns (g_idx = order // group, as GPTQ writes
 * it); otherwise -1 and the caller keeps SNEPPX_qlinear_w4a16 with g_idx.
 * K <= 65536.  Synchronous (g_idx is sorted on the host). */
int SNEPPX_qlinear_w4_actorder_prepare(const uint32_t* qweight, const int32_t* g_idx, size_t G,
                                       uint32_t* qweight_sorted, uint16_t* perm,
                                       size_t N, size_t K, SNEPPXStream stream);

/* C3 fast path, step 2: y = x . W^T for prepared weights.  Scales (and
 * optional qzeros) stay [N][G] in group order; the group of sorted column k'
 * is k' / group with group = K/G.  The activations are gathered by perm
 * inside the decode kernel (M <= 4) or by one gather pass (other M). */
int SNEPPX_qlinear_w4a16_actorder(const uint16_t* x, const uint32_t* qweight_sorted,
                                  const uint16_t* scales, const uint32_t* qzeros,
                                  const uint16_t* perm, const float* bias, void* y,
                                  SNEPPXDtype y_dtype, size_t M, size_t N, size_t K, int group,
                                  SNEPPXStream stream);

/* C5 SwiGLU step between the gate/up and down projections (no reference
 * counterpart; the reference's MLP is fp32): gate_up bf16 [T][2F] with gate
 * in columns [0, F) and up in [F, 2F); out bf16 [T][F] =
 * bf16(g / (1 + exp(-g)) * u) computed in fp32.  F % 8 == 0. */
int SNEPPX_qlinear_silu_mul(const uint16_t* gate_up, uint16_t* out, size_t T, size_t F,
                            SNEPPXStream stream);

/* C5 gate/up projection with the SwiGLU step fused (no reference
 * counterpart for the fused form; the activation is the SWIGLU rule of
 * kernel/activations/gated_activations.c:33-52, act = g / (1 + exp(-g)),
 * out = act * u).  qweight / scales / qzeros hold the stacked gate/up
 * projection [2F][K] in the W4 layout, gate rows first; bias is fp32 [2F]
 * or NULL.  out bf16 [M][F] = bf16(silu(g) * u) with g = x . Wg^T + bias[n]
 * and u = x . Wu^T + bias[F + n] kept in fp32 (no bf16 round trip of the
 * [M][2F] projection).  M >= 256 runs the prefill GEMM with the SwiGLU in
 * its epilogue; fewer rows run the decode linear into fp32 scratch, then
 * the same rule.  The exponential and reciprocal use the hardware's fast
 * approximations (about 1 ulp, below the bf16 rounding).  F % 8 == 0. */
int SNEPPX_qlinear_w4a16_swiglu(const uint16_t* x, const uint32_t* qweight,
                                const uint16_t* scales, const uint32_t* qzeros, const float* bias,
                                uint16_t* out, size_t M, size_t F, size_t K, int group,
                                SNEPPXStream stream);

/* A SwiGLU MLP block in W4A16 (no single reference counterpart: it is
 * SNEPPX_qlinear_w4a16_swiglu followed by SNEPPX_qlinear_w4a16 on its
 * output, the SwiGLU rule of gated_activations.c:33-52 between the two
 * projections): y[m][n] = down(silu(gate(x)) * up(x)).
 * x bf16 [M][H]; gate/up weights as for SNEPPX_qlinear_w4a16_swiglu
 * (stacked [2F][H], gu_bias fp32 [2F] or NULL); down weights as for
 * SNEPPX_qlinear_w4a16 with K = F (dn_bias fp32 [N] or NULL); y [M][N] in
 * y_dtype (bf16 or fp32); one group size for both projections.  For
 * prefill row counts the gate/up GEMM writes its SwiGLU rows straight into
 * the down GEMM's prepared input (F % 128 == 0), which saves the down
 * projection's activation pass; the results are bit-identical to the two
 * calls above (which is what other shapes run).  Scratch: the calling
 * thread's workspaces on `stream`. */
int SNEPPX_qlinear_w4a16_mlp(const uint16_t* x, const uint32_t* gu_qweight, const uint16_t* gu_scales,
                             const uint32_t* gu_qzeros, const float* gu_bias, const uint32_t* dn_qweight,
                             const uint16_t* dn_scales, const uint32_t* dn_qzeros, const float* dn_bias,
                             void* y, SNEPPXDtype y_dtype, size_t M, size_t H, size_t F, size_t N,
                             int group, SNEPPXStream stream);

/* SNEPPX_qlinear_silu_mul fused with the per-token int8 quantizer the W8A8
 * down projection needs (no reference counterpart; the rule is
 * SNEPPX_quantize_int8_channel, quantize_int8.c:157-177, applied to the bf16
 * rows SNEPPX_qlinear_silu_mul would write): q int8 [T][F], scales fp32 [T].
 * One pass instead of SwiGLU + quantize.  F % 8 == 0, F <= 32768. */
int SNEPPX_qlinear_silu_mul_quant_int8(const uint16_t* gate_up, int8_t* q, float* scales,
                                       size_t T, size_t F, SNEPPXStream stream);

/* Per-token int8 of bf16 activations (SNEPPX_quantize_int8_channel,
 * quantize_int8.c:157-177, on the bf16 values): for C4 inputs that come out
 * of a bf16 op.  in bf16 [rows][cols], q int8, scales fp32 [rows]. */
int SNEPPX_dev_quantize_int8_channel_bf16(const uint16_t* in, int8_t* q, float* scales,
                                          size_t rows, size_t cols, SNEPPXStream stream);

/* C4 int8: out[m][n] = bf16(((float)acc * sA[m]) * sW[n] (+ bias[n])),
 * acc = sum_k A*W in int32 (exact).  A int8 [M][K] (per-token scales sA fp32
 * [M]), W int8 [N][K] (per-channel sW fp32 [N]), out bf16 [M][N]. */
int SNEPPX_qlinear_w8a8_i8(const int8_t* A, const float* sA, const int8_t* W,
                           const float* sW, const float* bias, uint16_t* out, size_t M,
                           size_t N, size_t K, SNEPPXStream stream);

/* C4 int8 accumulators only: C int32 [M][N] = A . W^T (for bit-exact checks). */
int SNEPPX_qlinear_i8_gemm_i32(const int8_t* A, const int8_t* W, int32_t* C,
                               size_t M, size_t N, size_t K, SNEPPXStream stream);

/* C4 fp8: A, W are reference E4M3 codes (|x/s| < 256 so every code is an
 * OCP e4m3fn value of equal magnitude); per-tensor scales sA, sW are device
 * floats; fp32 accumulation; out bf16 [M][N] = bf16((acc * sA) * sW (+ bias[n])). */
int SNEPPX_qlinear_w8a8_fp8(const uint8_t* A, const float* sA, const uint8_t* W,
                            const float* sW, const float* bias, uint16_t* out, size_t M,
                            size_t N, size_t K, SNEPPXStream stream);

/* C4 with the activations quantized inside the call (no reference
 * counterpart as one call): A bf16 [M][K] as it leaves the previous op, out
 * bf16 [M][N].  int8: A per token with the rule of SNEPPX_quantize_int8_channel
 * (quantize_int8.c:157-177) on each row of A, into a workspace (M*K bytes +
 * M scales), then SNEPPX_qlinear_w8a8_i8 with W int8 [N][K] and per-channel
 * sW [N].  fp8: A per tensor as SNEPPX_dev_quantize_fp8_e4m3_scaled (s_A =
 * max|A|/240, codes e4m3(a / s_A)), then SNEPPX_qlinear_w8a8_fp8 with W's
 * codes and its device scale sW.  Bit-identical to quantizing A with those
 * entry points (on A converted to fp32, exact for bf16) and calling the
 * GEMM. */
int SNEPPX_qlinear_w8a8_i8_dyn(const uint16_t* A, const int8_t* W, const float* sW,
                               const float* bias, uint16_t* out, size_t M, size_t N, size_t K,
                               SNEPPXStream stream);
int SNEPPX_qlinear_w8a8_fp8_dyn(const uint16_t* A, const uint8_t* W, const float* sW,
                                const float* bias, uint16_t* out, size_t M, size_t N, size_t K,
                                SNEPPXStream stream);

#ifdef __cplusplus
}
#endif

#endif /* SNEPPX_QLINEAR_H */
