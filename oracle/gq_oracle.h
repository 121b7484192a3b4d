/*
 * gq_oracle.h -- CPU restatement of GRETA CORE's quantized-weight matrix path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links or calls this
 * code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use
 * it, and only as the checker / CPU baseline.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the leaatimberini/gretacore-v3 tree).  Pinning of each function:
 *   gqo_fp16_to_fp32      exhaustive 2^16 check against CpuReference::half_to_float
 *                         (compiled from the reference) and against numpy float16.
 *   gqo_float_to_half     exhaustive-sample check against numpy's RNE float16.
 *   gqo_dequant_q8_0      GGUF closed form d*q; one-hot / d=1 special cases.
 *   gqo_dequant_q4_0      GGUF closed form (q-8)*d; all-8 -> zeros; d=1 ints.
 *   gqo_dequant_q4_k      bit-exact against dequantize_q4_k_block compiled from
 *                         the reference sources (oracle/_ref), plus code-range and
 *                         d=1,dmin=0 invariants.
 *   gqo_dequant_q4_k_ggml invariants (d=1,dmin=0 -> integer codes x nibble) and a
 *                         hand-built block; "parity unpinned" against ggml itself
 *                         (ggml is not vendored in the reference).
 *   gqo_dequant_q6_k      bit-exact against dequantize_q6_k_block from oracle/_ref.
 *   gqo_gemm_ref          CpuReference::gemm known answer 19/22/43/50.
 *   gqo_gemv / gqo_gemm   brute force on tiny shapes in numpy, one-hot columns.
 *   gqo_requant_int8/int4 closed-form invariants (|q|<=127 / [-8,7], error<=s/2).
 */
#ifndef GQ_ORACLE_H
#define GQ_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (reference weight_loader.cpp:15-33) plus one variant id. */
enum {
  GQO_F32 = 0,
  GQO_F16 = 1,
  GQO_Q4_0 = 2,
  GQO_Q8_0 = 8,
  GQO_Q4_K = 12,      /* reference (GRETA) Q4_K nibble / scale layout */
  GQO_Q6_K = 14,
  GQO_Q4_K_GGML = 112, /* llama.cpp canonical Q4_K layout */
  GQO_Q6_K_GGML = 114  /* llama.cpp canonical Q6_K layout */
};

float gqo_fp16_to_fp32(uint16_t h);
uint16_t gqo_float_to_half(float f);
uint16_t gqo_fp32_to_fp16_trunc(float f);
/* Array forms of the two conversions above. */
void gqo_fp16_to_fp32_n(const uint16_t *h, size_t n, float *out);
void gqo_fp32_to_fp16_trunc_n(const float *f, size_t n, uint16_t *out);

size_t gqo_block_elems(int fmt);
size_t gqo_block_bytes(int fmt);

/* Dequantize n_blocks consecutive GGUF blocks of `fmt` into fp32. */
int gqo_dequant(int fmt, const uint8_t *blocks, size_t n_blocks, float *out);

/* y[b][n] = sum_k x[b][k] * W[n][k], W = dequant(w) (row-major GGUF, N rows of
 * K elements), accumulated in double, stored as float.  threads<=0: all. */
int gqo_gemv(int fmt, const uint8_t *w, const float *x, float *y, int N, int K,
             int B, int threads);

/* C[m][n] = sum_k A[m][k] * W[n][k] (fp64 accumulate). */
int gqo_gemm(int fmt, const uint8_t *w, const float *A, float *C, int M, int N,
             int K, int threads);

/* CpuReference::gemm: C = A[M][K] * B[K][N], fp64 accumulate. */
void gqo_gemm_ref(const float *A, const float *B, float *C, int M, int N, int K);

/* Reference INT8 requant (weight_loader.cpp:780-802). */
void gqo_requant_int8(const float *w, size_t n, int8_t *q, float *scales);
/* Reference INT4 requant + pack (weight_loader.cpp:920-957). */
void gqo_requant_int4(const float *w, size_t n, uint8_t *packed, float *scales);
/* Reference per-head scales (weight_loader.cpp:972-998). */
void gqo_head_scales(const float *w, uint32_t num_heads, uint32_t head_dim,
                     uint32_t dim, float *h_scales);
/* Reference GQA K/V transpose [D][KV] -> [KV][D] (weight_loader.cpp:877-918). */
void gqo_gqa_transpose(const float *in, uint32_t model_dim, uint32_t kv_dim,
                       float *out);

/* Reference INT8 / INT4 weight-only GEMV/GEMM math (gemm_kernels.hip:594-634,
 * 640-740, 763-817, 820-908): y[m][n] = sum_k x[m][k]*(q[n][k]*s[idx]) (x head
 * scale), idx = (n*K)/gs + k/gs on the GEMV route (gemv_route != 0: M <= 32
 * or force_gemv) and (n*K + k)/gs on the MFMA route (M > 32). */
void gqo_gemm_int8_wt(const float *x, const int8_t *q, const float *s, float *y,
                      int M, int N, int K, int gs, int gemv_route);
void gqo_gemm_int4_wt(const float *x, const uint8_t *packed, const float *s,
                      const float *head_scales, float *y, int M, int N, int K,
                      int gs, int head_dim, int gemv_route);

/* RMS normalisation of fused_rmsnorm_qkv_gemv_kernel_f16
 * (src/rt/backend/hip/kernels/fused_compute_kernels.hip:36-87), in fp64:
 * out[b][k] = x[b][k] / sqrt(sum_k x^2 / K + eps) * gamma[k]. */
void gqo_rmsnorm(const float *x, const float *gamma, int rows, int K, float eps, double *out);
/* silu(g) * u of fused_ffn_front_gemv_kernel_f16 (fused_compute_kernels.hip:162-241),
 * silu(g) = g / (1 + exp(-g)), in fp64. */
void gqo_swiglu(const double *g, const double *u, size_t n, double *out);

/* Per-32 activation quantization used by the int8-MFMA Q8_0 path:
 * d = amax/127, inv = d>1e-9 ? 1/d : 0, q = round(a*inv) (half away). */
void gqo_quantize_act_q8(const float *a, int M, int K, int8_t *q, float *d);
/* C[m][n] = sum_blk dA[m][blk]*dW[n][blk]*sum_{k in blk} qa*qw (exact ints,
 * fp64 scale products) for Q8_0 weights. */
int gqo_gemm_q8_i8(const uint8_t *w, const int8_t *qa, const float *da,
                   float *C, int M, int N, int K, int threads);

#ifdef __cplusplus
}
#endif
#endif
