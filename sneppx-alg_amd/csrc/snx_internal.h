/*
 * snx_internal.h - C-ABI between the C host layer and the HIP translation
 * units of libsneppx_quant.so (not installed; the public surface is in
 * include/).  Launchers take device pointers and a hipStream_t (as void*),
 * enqueue their kernels and return 0, or -1 with the error text set.
 */
#ifndef SNX_INTERNAL_H
#define SNX_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

void snx_set_error(const char* fmt, ...);
/* device scratch reused by every call on (current device, stream, slot) from
 * the calling host thread; slot 1 is for a call made from inside another
 * one.  NULL on failure. */
void* snx_workspace(size_t bytes, int slot, void* stream);
/* as snx_workspace; a newly taken buffer is zero-filled on `stream` first */
void* snx_workspace_zeroed(size_t bytes, int slot, void* stream);
/* stream-ordered release of the calling thread's workspaces on `stream` and
 * of those that ended threads left on it */
void snx_release_workspaces(void* stream);
/* workspaces held now, by live threads and left by ended ones (for tests) */
long snx_workspace_count(void);
/* the current device's static scratch array (noalloc.hip) when `bytes` fit
 * in it, else NULL with the error text set (prefixed by `who`) */
void* snx_noalloc_scratch(size_t bytes, const char* who);
void snx_clear_error(void);
int snx_launch_check(const char* kernel);

/* kinds of snx_k_finalize_scale */
enum {
    SNX_SCALE_SYM127 = 0,   /* int8 sym: max/127 (quantize_int8.c:52-59) */
    SNX_SCALE_SYM7 = 1,     /* int4 sym: max/7   (quantize_int8.c:198-205) */
    SNX_SCALE_ASYM255 = 2,  /* int8 asym: (max-min)/255, zp (quantize_int8.c:102-117) */
    SNX_SCALE_FP8_240 = 3,  /* per-tensor fp8: max/240 (build-defined) */
    SNX_SCALE_MODELZOO = 4  /* model-zoo int8 multiplier 127/max (weights.c:233-240) */
};

/* Scale record written by snx_k_finalize_scale (device memory, 4 floats):
 * [0] scale, [1] 1/scale, [2] zero point (as float), [3] 1.0 if degenerate. */
#define SNX_SCALE_REC 4

/* number of partial blocks the reduction launchers use for n elements */
int snx_reduce_parts(size_t n);

int snx_k_absmax(const float* x, size_t n, float* part, int nparts, void* stream);
int snx_k_minmax(const float* x, size_t n, float* part, int nparts, void* stream);
int snx_k_finalize_scale(const float* part, int nparts, int kind, const float* x,
                         float* rec, float* scale_out, void* stream);

int snx_k_quant_int8_sym(const float* x, int8_t* q, size_t n, const float* rec, void* stream);
int snx_k_dequant_int8_sym(const int8_t* q, float* y, size_t n, float scale, void* stream);
int snx_k_quant_int8_asym(const float* x, int8_t* q, size_t n, const float* rec, void* stream);
int snx_k_dequant_int8_asym(const int8_t* q, float* y, size_t n, float scale, int32_t zp,
                            void* stream);
int snx_k_quant_int4_sym(const float* x, uint8_t* p, size_t n, const float* rec, void* stream);
int snx_k_dequant_int4_sym(const uint8_t* p, float* y, size_t n, float scale, void* stream);
/* fmt 0 = E4M3, 1 = E5M2; rec == NULL encodes x as is, else x * rec[1] */
int snx_k_fp8_encode(const float* x, uint8_t* c, size_t n, int fmt, const float* rec,
                     void* stream);
int snx_k_fp8_decode(const uint8_t* c, float* y, size_t n, int fmt, void* stream);

/* rne: 0 = roundf (the reference), 1 = ties to even */
int snx_k_quant_int8_rows(const float* x, int8_t* q, float* scales, size_t rows, size_t cols,
                          int rne, void* stream);
/* layer_kernels.hip: out[c][r] = in[r][c] (in is rows x cols); fp32 -> bf16 RNE */
int snx_k_transpose_f32(const float* in, float* out, size_t rows, size_t cols, void* stream);
int snx_k_f32_to_bf16(const float* x, uint16_t* y, size_t n, void* stream);

/* mx_kernels.hip (f: element format 0 e4m3, 1 e5m2, 2 e3m2, 3 e2m3, 4 e2m1) */
int snx_mx_scale_host(uint32_t peak_bits, int f, int tensor);
int snx_k_mx_quant_blocks(const float* x, uint8_t* packed, int8_t* scales, size_t rows,
                          size_t cols, int bs, int f, void* stream);
int snx_k_mx_dequant_blocks(const uint8_t* packed, const int8_t* scales, float* y, size_t rows,
                            size_t cols, int bs, int f, void* stream);
int snx_mx_tensor_parts(size_t n);
int snx_k_mx_tensor_stats(const float* x, size_t n, uint32_t* part, int nparts, void* stream);
int snx_k_mx_quant_tensor(const float* x, uint8_t* packed, size_t n, int s, int f, void* stream);
int snx_k_mxfp4_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                     void* out, int y_f32, size_t M, size_t N, size_t K, void* stream);
/* LDS-staged MXFP4 GEMM (256 x 224 tiles): K % 256 == 0, 4-byte aligned scales */
int snx_k_mxfp4_gemm_tiled(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                           void* out, int y_f32, size_t M, size_t N, size_t K, void* st);
/* the same with one exponent per operand (sA[0], sW[0]; NVFP4's default):
 * their sum split between the operands as k_mx_expand_scales splits it */
int snx_k_mxfp4_gemm_tiled_pt(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                              void* out, int y_f32, size_t M, size_t N, size_t K, void* st);
int snx_k_mx_dequant_tensor(const uint8_t* packed, float* y, size_t n, int s, int f, void* stream);
/* reference MXFP8 blocks (f 0 e4m3, 1 e5m2) -> matrix-core-decodable codes and
 * exponents; *rounded (device, may be NULL) counts elements that rounded */
/* block-32 exponents of a GEMM operand from a block of 32 * rep (rep > 0) or
 * a per-tensor exponent (rep == 0: operand `which` 0 = A / 1 = W takes its
 * share of sA[0] + sW[0]) */
int snx_k_mx_expand_scales(const int8_t* src, const int8_t* sA, const int8_t* sW, int8_t* dst,
                           size_t rows, size_t kb32, unsigned rep, int which, void* stream);
int snx_k_mx_to_mfma(const uint8_t* in, const int8_t* sin, uint8_t* out, int8_t* sout,
                     size_t nblocks, int f, unsigned int* rounded, void* stream);
/* MXFP8 / MXFP6 GEMM on matrix-core-decodable operands; mf the MFMA element
 * format (0 e4m3, 1 e5m2, 2 e2m3, 3 e3m2); K % 128 == 0 */
int snx_k_mx8_gemm(const uint8_t* A, const int8_t* sA, const uint8_t* W, const int8_t* sW,
                   void* out, int y_f32, int mf, size_t M, size_t N, size_t K, void* stream);

/* model-zoo int8 codes with the multiplier in rec[0] (weights.c:242-247) */
int snx_k_quant_int8_modelzoo(const float* x, int8_t* q, size_t n, const float* rec,
                              void* stream);
/* the same rule (roundf) on bf16 rows */
/* per-token int8 of bf16 rows in one pass (row in registers; cols % 8 == 0,
 * cols <= 8192, x 16-byte and q 8-byte aligned, else the two-pass kernel) */
int snx_k_quant_rows_bf16_fast(const uint16_t* x, int8_t* q, float* scales, size_t rows, size_t cols,
                               void* stream);
/* partial max|x| of bf16 values / per-tensor scaled e4m3 codes of bf16 values
 * (value / rec[0]) */
int snx_k_absmax_bf16(const uint16_t* x, size_t n, float* part, int nparts, void* stream);
int snx_k_fp8_encode_bf16(const uint16_t* x, uint8_t* c, size_t n, const float* rec, void* stream);
/* the same from the nparts partial maxima of snx_k_absmax_bf16, the scale
 * (max/240) computed in every block and written to *scale_out; n % 8 == 0,
 * x 16-byte and c 8-byte aligned */
int snx_k_fp8_encode_bf16_pt(const uint16_t* x, uint8_t* c, size_t n, const float* part, int nparts,
                             float* scale_out, void* stream);
int snx_k_quant_int8_rows_bf16(const uint16_t* x, int8_t* q, float* scales, size_t rows,
                               size_t cols, void* stream);
int snx_k_fake_quant(const float* x, float* y, size_t n, float scale, int bits, void* stream);
int snx_k_awq_quantize(const float* w, int8_t* q, float* scales, size_t rows, size_t cols,
                       size_t group, void* stream);
/* q may be NULL (bits > 8 store no codes); zeros may be NULL */
int snx_k_gptq_quantize(const float* w, int8_t* q, float* scales, int32_t* zeros,
                        size_t rows, size_t cols, size_t group, int bits, int sym,
                        void* stream);
int snx_k_awq_scale_weights(float* w, const float* act, float* scale_out, size_t rows,
                            size_t cols, void* stream);
int snx_k_gptq_hessian(float* h, const float* act, size_t n, size_t dim, void* stream);
/* out[0] = scale, out[1] = zero (int32 bits) */
int snx_k_gptq_block(float* w, const float* h_inv, float* qw, float* out, size_t n,
                     int bits, int sym, void* stream);

int snx_k_w4_awq_quantize(const float* w, uint32_t* qw, uint16_t* scales, uint32_t* qzeros,
                          size_t N, size_t K, int group, void* stream);
int snx_k_w4_gptq_quantize(const float* w, const int32_t* g_idx, size_t G, uint32_t* qw,
                           uint16_t* scales, size_t N, size_t K, void* stream);

/* ---- linears (gemv_kernels.hip, gemm_kernels.hip) ---- */
/* bias (fp32 [N] or NULL) is added to the fp32 result of every linear below */
int snx_k_w8_gemv(const float* x, const int8_t* q, const float* s, float* y, const float* bias,
                  size_t M, size_t N, size_t K, void* stream);
/* y_f32: 1 -> fp32 output, 0 -> bf16.  perm (uint16 [K], may be NULL): the
 * weight columns are stored in that order (M <= 4 only, see small_ok). */
int snx_k_w4a16_gemv(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                     const uint32_t* qzeros, const uint16_t* perm, void* y, const float* bias,
                     int y_f32, size_t M, size_t N, size_t K, int group, void* stream);
size_t snx_w4a16_small_lds(size_t M, size_t K, int perm);
int snx_w4a16_small_ok(size_t M, size_t K, int group, int perm);
/* the M = 1 streaming decode kernel applies (group 128, K = 2048 T <= 16384,
 * scales 16-byte and qzeros 4-byte aligned); perm may be given */
int snx_w4a16_gemv1_ok(size_t M, size_t K, int group, const void* scales, const void* qzeros);
int snx_w4a16_gemv1_swiglu_ok(size_t F, size_t K, int group, const void* scales, const void* qzeros);
int snx_k_w4a16_gemv1_swiglu(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                             const uint32_t* qzeros, const float* bias, uint16_t* out, size_t F,
                             size_t K, int group, void* st);
/* split-K decode (5 <= M <= 16): K span per workgroup (0 = unsupported),
 * partials part [K/kspan][M][N] fp32, then the ordered reduction */
int snx_w4a16_splitk_span(size_t M, size_t K, int group);
int snx_k_w4a16_splitk(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                       const uint32_t* qzeros, float* part, size_t M, size_t N, size_t K,
                       int group, int kspan, void* stream);
int snx_k_w4a16_reduce(const float* part, void* y, int y_f32, int S, size_t MN, size_t N,
                       const float* bias, void* stream);
/* xs[m][k'] = x[m][perm[k']] (bf16), perm entries < K */
int snx_k_gather_cols(const uint16_t* x, const uint16_t* perm, uint16_t* xs, size_t M, size_t K,
                      void* stream);
/* qs[n] column k' = qw[n] column perm[k'] (packed uint4 words) */
int snx_k_w4_permute_cols(const uint32_t* qw, const uint16_t* perm, uint32_t* qs, size_t N,
                          size_t K, void* stream);
/* any group size / g_idx, any M: reference-layout fallback */
/* 2 <= M <= 16 decode GEMV (group 128, K = 1024 .. 4096 in steps of 1024): one
 * persistent workgroup per CU; perm != NULL gathers x[m][perm[k]] (M <= 8). */
size_t snx_w4a16_mt_lds(size_t M, size_t K, int perm);
int snx_w4a16_mt_ok(size_t M, size_t K, int group, int perm);
int snx_k_w4a16_gemv_mt(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                        const uint32_t* qzeros, const uint16_t* perm, void* y, const float* bias,
                        int y_f32, size_t M, size_t N, size_t K, void* stream);
int snx_k_w4a16_generic(const uint16_t* x, const uint32_t* qw, const uint16_t* scales,
                        const uint32_t* qzeros, const int32_t* g_idx, size_t G, void* y,
                        const float* bias, int y_f32, size_t M, size_t N, size_t K, int group,
                        void* stream);
int snx_w4a16_gemv_supported(size_t M, size_t N, size_t K, int group);

/* W4A16 prefill GEMM (w4_gemm_kernels.hip): activations prepared once
 * (k-slot order + fp32 sums per 128 columns, xs [K/128][Mp]), then the GEMM. */
size_t snx_w4_prep_rows(size_t M);
int snx_w4a16_gemm_ok(size_t M, size_t N, size_t K, int group);
int snx_k_w4_prep_x(const uint16_t* x, uint16_t* xp, float* xs, size_t M, size_t K, size_t Mp,
                    void* stream);
/* K spans the GEMM splits M x N x K into (1, 2 or 4: with few tiles), and
 * the partials / counters workspaces a call with `splits` > 1 takes (the
 * counters zero when taken; every call leaves them zero) */
int snx_w4a16_gemm_splits(size_t M, size_t N, size_t K);
size_t snx_w4a16_gemm_part_bytes(size_t M, size_t N, int splits);
size_t snx_w4a16_gemm_cnt_bytes(size_t M, size_t N);
int snx_k_w4a16_gemm(const uint16_t* xp, const float* xs, const uint32_t* qw,
                     const uint16_t* scales, const uint32_t* qzeros, void* y, const float* bias,
                     int y_f32, size_t M, size_t N, size_t K, int group, size_t Mp, int splits,
                     void* part, uint32_t* cnt, void* stream);

/* SwiGLU step: out [T][F] = bf16(silu(gu[:, :F]) * gu[:, F:]), F % 8 == 0 */
/* SwiGLU then per-token int8 of the bf16 result (F % 8 == 0, F <= 32768) */
int snx_k_silu_mul_quant_int8(const uint16_t* gu, int8_t* q, float* scales, size_t T, size_t F,
                              void* stream);
int snx_k_silu_mul(const uint16_t* gu, uint16_t* out, size_t T, size_t F, void* stream);
/* the fused SwiGLU rule on fp32 gate/up rows [T][2F] -> bf16 [T][F] */
int snx_k_silu_mul_f32(const float* gu, uint16_t* out, size_t T, size_t F, void* stream);
/* the prefill GEMM with the SwiGLU epilogue: qw is the stacked [2F][K]
 * gate/up projection, out bf16 [M][F], bias fp32 [2F] or NULL */
int snx_k_w4a16_gemm_swiglu(const uint16_t* xp, const float* xs, const uint32_t* qw,
                            const uint16_t* scales, const uint32_t* qzeros, uint16_t* out,
                            const float* bias, size_t M, size_t F, size_t K, int group, size_t Mp,
                            void* stream);
/* the same GEMM writing its SwiGLU rows as the down projection's prepared
 * input: out_xp [M][F] in the prep pass's slot order, out_xs [F / 128][Mp]
 * step sums (F % 128 == 0) */
int snx_k_w4a16_gemm_swiglu_prep(const uint16_t* xp, const float* xs, const uint32_t* qw,
                                 const uint16_t* scales, const uint32_t* qzeros, uint16_t* out_xp,
                                 float* out_xs, const float* bias, size_t M, size_t F, size_t K, int group,
                                 size_t Mp, void* stream);

int snx_k_i8_gemm(const int8_t* A, const int8_t* W, const float* sA, const float* sW,
                  int32_t* c_i32, uint16_t* out_bf16, const float* bias, size_t M, size_t N,
                  size_t K, void* stream);
int snx_k_fp8_gemm(const uint8_t* A, const uint8_t* W, const float* sA, const float* sW,
                   uint16_t* out_bf16, const float* bias, size_t M, size_t N, size_t K,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif
