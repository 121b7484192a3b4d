/*
 * gq.h -- C ABI of the MI355X-native GGUF quantized-weight matrix path
 * (libgq.so).  Plain pointers and sizes only; device pointers are HIP device
 * memory, `stream` is a hipStream_t passed as void* (NULL = default stream).
 * Every entry point returns a gq status (0 = GQ_OK) and launches
 * asynchronously on `stream` unless stated otherwise.
 *
 * Reference interfaces replaced (paths relative to leaatimberini/gretacore-v3):
 *   - src/rt/backend/hip/include/gcore/rt/hip/kernels/gemm_kernels.hpp:43-57
 *       launch_gemm_mfma_int8_wt_fp32_acc32 / launch_gemm_mfma_int4_wt_fp32_acc32
 *       -> gq_launch_gemm_mfma_int8_wt_fp32_acc32 / ..._int4_... (same args)
 *       and, for GGUF-native weights, gq_gemv / gq_gemm.
 *   - src/compute/src/greta_compute_hip.cpp:148-374 GretaCompute::gemm routing
 *       (M <= 32 -> GEMV kernel, else MFMA GEMM) -> gq_matmul.
 *   - src/inference/src/weight_loader.cpp:91-156, 703-712 (CPU dequant at load)
 *       -> gq_dequant_gguf (device, bit-exact) and gq_repack (GGUF -> T16).
 *   - src/inference/src/weight_loader.cpp:825-1008 load_tensor_int4 upload
 *       (requant to INT4 + hipMemcpy) -> gq_repack_host / gq_repack + upload of
 *       the GGUF blocks themselves (see gq_gguf.h for the loader ABI).
 */
#ifndef GQ_H
#define GQ_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GQ_ABI_VERSION 1

/* status codes */
#define GQ_OK 0
#define GQ_ERR_INVALID_ARGS 1 /* null pointer, bad shape, size out of range */
#define GQ_ERR_UNSUPPORTED 2  /* unknown format / dtype / batch */
#define GQ_ERR_HIP 3          /* a HIP call or kernel launch failed */
#define GQ_ERR_WORKSPACE 4    /* workspace missing or too small */
#define GQ_ERR_NO_DEVICE 5    /* no usable GPU */

/* weight formats: GGML type ids (weight_loader.cpp:15-33) + Q4_K / Q6_K variants */
#define GQ_FMT_Q4_0 2
#define GQ_FMT_Q8_0 8
#define GQ_FMT_Q4_K 12       /* reference (GRETA) Q4_K layout, weight_loader.cpp:125-156 */
#define GQ_FMT_Q6_K 14       /* reference Q6_K layout, weight_loader.cpp:158-177 */
#define GQ_FMT_Q4_K_GGML 112 /* llama.cpp canonical Q4_K layout */
#define GQ_FMT_Q6_K_GGML 114 /* llama.cpp canonical Q6_K layout */
/* accepted by gq_dequant_gguf only (loader conversions) */
#define GQ_FMT_F16 1         /* one "block" = one fp16 value (weight_loader.cpp:91-110) */
/* Q6_K (both layouts): T16 repack, dequant, gq_gemv (int8 matrix-core
   kernel at batch 1..2, fp16 above) and gq_gemm for K <= 4096 (skinny kernel,
   any M); gq_gemv_multi / gq_gemv_swiglu run their fallback for it (RMSNorm,
   one gq_gemv per matrix); gq_gemm with longer K and gq_gemv_prep / prepped
   return GQ_ERR_UNSUPPORTED for it (gq_matmul then runs 16-row GEMV batches). */

/* activation / output dtypes */
#define GQ_DT_F32 0
#define GQ_DT_F16 1
#define GQ_DT_BF16 2

/* limits checked by every entry point */
#define GQ_MAX_DIM (1u << 24) /* N, K, M */
#define GQ_MAX_BATCH 16       /* gq_gemv batch (decode) */

int gq_abi_version(void);
const char *gq_status_string(int status);
/* Last HIP error text seen by this thread (empty if none). */
const char *gq_last_error(void);

/* ---- sizes ---------------------------------------------------------------- */
/* GGUF bytes of an N x K tensor (weight_loader.cpp:457-463 sizing). */
size_t gq_gguf_bytes(int fmt, size_t N, size_t K);
/* Bytes of the repacked (T16) tensor.  Equal to the GGUF size whenever N is a
 * multiple of 16 and K a multiple of 128 (Q4_0/Q8_0) or 256 (Q4_K). */
int gq_packed_size(int fmt, size_t N, size_t K, size_t *bytes);

/* ---- load-time repack ----------------------------------------------------- */
/* Host: GGUF rows (N x K, row-major blocks) -> T16 layout; no GPU needed. */
int gq_repack_host(int fmt, const void *gguf, size_t N, size_t K, void *packed);
/* Host: inverse of gq_repack_host (T16 -> GGUF bytes of the same format). */
int gq_unpack_host(int fmt, const void *packed, size_t N, size_t K, void *gguf);
/* Device: same as gq_repack_host on device buffers. */
int gq_repack(int fmt, const void *d_gguf, size_t N, size_t K, void *d_packed, void *stream);
/* Device, one slice of rows: d_gguf_rows holds the GGUF rows [row0, row0 +
 * rows) of an N x K tensor; their T16 tiles are written into d_packed, the
 * whole tensor's buffer (gq_packed_size(N, K) bytes).  row0 is a multiple of
 * 16 and rows is too unless the slice ends the tensor (the last tile's padding
 * rows are then zeroed).  Slices may run in any order; together they give
 * gq_repack's result.  Lets a loader repack a tensor while later slices are
 * still in flight from the host (replaces the whole-tensor hipMemcpy of
 * src/inference/src/weight_loader.cpp:532-534). */
int gq_repack_rows(int fmt, const void *d_gguf_rows, size_t N, size_t K, size_t row0, size_t rows,
                   void *d_packed, void *stream);

/* ---- dequantization (bit-exact with the reference semantics) -------------- */
/* n_blocks raw GGUF blocks -> fp32 (n_blocks * 32 or * 256 values; F16:
 * n_blocks values).  Formats: Q4_0, Q8_0, Q4_K, Q4_K_GGML, Q6_K, F16. */
int gq_dequant_gguf(int fmt, const void *d_blocks, size_t n_blocks, float *d_out, void *stream);
/* T16 tensor -> fp32 [N][K]. */
int gq_dequant_packed(int fmt, const void *d_packed, size_t N, size_t K, float *d_out, void *stream);

/* ---- load-time conversions of the reference loader (all bit-exact) -------- */
/* fp32 -> fp16 with the reference's truncating rule (weight_loader.cpp:112-123):
 * mantissa truncated, below the normal range -> signed zero, above -> Inf. */
int gq_convert_f32_to_f16(const float *d_in, size_t n, uint16_t *d_out, void *stream);
/* GQA K/V transpose (weight_loader.cpp:634-658, 739-781, 877-918): in is
 * [model_dim][kv_dim] (kv contiguous), out [kv_dim][model_dim]; elem_bytes 2 or
 * 4; out must not alias in. */
int gq_transpose_kv(int elem_bytes, const void *d_in, size_t model_dim, size_t kv_dim, void *d_out,
                    void *stream);
/* INT8 requant per 32 of the flat tensor (weight_loader.cpp:780-802):
 * scales[ceil(n/32)], q[n]. */
int gq_requant_int8(const float *d_w, size_t n, int8_t *d_q, float *d_scales, void *stream);
/* INT4 requant + pack (weight_loader.cpp:920-957): packed[ceil(n/2)], scales[ceil(n/32)]. */
int gq_requant_int4(const float *d_w, size_t n, uint8_t *d_packed, float *d_scales, void *stream);
/* Per-head max |w| (weight_loader.cpp:972-998): out[h] over the head_dim rows of
 * dim values of head h, 1.0 if <= 1e-9.  Requires num_heads*head_dim*dim <= n. */
int gq_head_scales(const float *d_w, size_t n, uint32_t num_heads, uint32_t head_dim, uint32_t dim,
                   float *d_out, void *stream);
/* Q8_0 blocks -> int8 q[32 * n_blocks] + fp32 scales[n_blocks]
 * (weight_loader.cpp:703-712). */
int gq_split_q8_0(const void *d_blocks, size_t n_blocks, int8_t *d_q, float *d_scales, void *stream);

/* ---- decode GEMV: y[b][n] = sum_k x[b][k] * W[n][k], 1 <= batch <= 16 ------- */
/* Workspace bytes needed by gq_gemv for (fmt, K, batch). */
size_t gq_gemv_workspace_bytes(int fmt, size_t K, int batch);
/* x f32 [batch][K], y f32 [batch][N].  workspace may be NULL: the library then
 * uses a per-device buffer it owns (allocated on first use; not for use under
 * stream capture).  Concurrent calls that share a workspace race. */
int gq_gemv(int fmt, const void *d_packed, const float *d_x, float *d_y, size_t N, size_t K, int batch,
            void *d_workspace, size_t workspace_bytes, void *stream);
/* Launch plan of gq_gemv for a shape (no GPU needed): row tiles per
 * workgroup, waves per workgroup (K split) and the most K chunks one wave
 * streams.  Environment overrides for tuning: GQ_GEMV_R, GQ_GEMV_KSPLIT. */
int gq_gemv_plan(int fmt, size_t N, size_t K, int batch, int *row_tiles_per_wg, int *ksplit,
                 int *chunks_per_wave);
/* Split form: prepare x once (gq_gemv_prep) and run several GEMVs that share
 * it (q/k/v, gate/up) with gq_gemv_prepped. */
int gq_gemv_prep(int fmt, const float *d_x, size_t K, int batch, void *d_workspace, size_t workspace_bytes,
                 void *stream);
int gq_gemv_prepped(int fmt, const void *d_packed, const void *d_workspace, float *d_y, size_t N, size_t K,
                    int batch, void *stream);

/* ---- fused decode GEMVs (batch 1..4) ----------------------------------------
 * Quantized counterparts of the reference's fp16 fused kernels
 * (src/rt/backend/hip/kernels/fused_compute_kernels.hip:22-243,
 * launch_fused_rmsnorm_qkv_gemv_f16 / launch_fused_ffn_front_f16), in one
 * launch each.  When gamma is not NULL, x is first RMS-normalised per batch row:
 * xn = x * (1 / sqrt(sum(x^2) / K + eps)) * gamma (gamma has K values).
 *
 * gq_gemv_multi: y[i] [batch][N[i]] = W_i xn for n_mats (1..4) matrices of one
 * format sharing K and x (e.g. q, k, v with GQA shapes). */
int gq_gemv_multi(int fmt, int n_mats, const void *const *d_packed, const size_t *N, size_t K, const float *d_x,
                  float *const *d_y, int batch, const float *d_gamma, float eps, void *stream);
/* Q6_K, and shapes whose activation staging does not fit one fused launch
 * (batch 3..4 with K beyond about 14000, or K too long for a wave's chunk list), run as a
 * fallback: x RMS-normalised into the library's workspace (when gamma is
 * given), one gq_gemv per matrix, and for gq_gemv_swiglu an elementwise
 * silu(gate) * up -- the same results within the GEMV bound, in 2-4 launches.
 * The fallback's normalised x and gate / up rows live in the library's default
 * workspace, which is allocated (after a device synchronisation) when a call
 * first needs more of it: under HIP graph capture, run such a shape once
 * before capturing.  Launch plan of gq_gemv_multi (row tiles per workgroup,
 * waves, chunks per wave); (0, 0, 0) when the call takes the fallback. */
int gq_gemv_multi_plan(int fmt, int n_mats, const size_t *N, size_t K, int batch, int *row_tiles_per_wg,
                       int *ksplit, int *chunks_per_wave);
/* gq_gemv_swiglu: y [batch][N] = silu(W_gate xn) * (W_up xn), silu(g) = g / (1 + e^-g)
 * (the FFN front of launch_fused_ffn_front_f16). */
int gq_gemv_swiglu(int fmt, const void *d_gate, const void *d_up, size_t N, size_t K, const float *d_x, float *d_y,
                   int batch, const float *d_gamma, float eps, void *stream);
/* Launch plan of gq_gemv_swiglu (waves, chunks per wave); (0, 0) for the fallback. */
int gq_gemv_swiglu_plan(int fmt, size_t N, size_t K, int batch, int *ksplit, int *chunks_per_wave);

/* ---- prefill GEMM: C[m][n] = sum_k A[m][k] * W[n][k] ------------------------ */
/* A is [M][K] of a_dtype (GQ_DT_BF16 / F16 / F32), C is [M][N] of c_dtype
 * (GQ_DT_F32 or GQ_DT_BF16).  Computes on f16 MFMA (v_mfma_f32_32x32x16_f16)
 * with fp32 accumulation, weights dequantized into fp16 fragments.  Few rows
 * (M <= 256 where the grid stays within one workgroup per CU, or two for K
 * beyond 4096) run on a skinny kernel that splits K over the waves of a
 * workgroup; small tiled grids split K over 2 or 4 wave groups of a
 * workgroup. */
size_t gq_gemm_workspace_bytes(int fmt, size_t M, size_t K);
int gq_gemm(int fmt, const void *d_packed, const void *d_a, int a_dtype, void *d_c, int c_dtype, size_t M,
            size_t N, size_t K, void *d_workspace, size_t workspace_bytes, void *stream);

/* gq_gemm without a workspace and without any allocation: no counterpart in
 * the reference; for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  The
 * activation conversion uses a library-owned device array of
 * gq_gemm_static_max_bytes() (64 MiB) per GPU, held until the process ends;
 * shapes whose conversion needs more (gq_gemm_workspace_bytes(fmt, M, K) >
 * that) return GQ_ERR_WORKSPACE.  Every call on one GPU shares that array:
 * calls that overlap on one GPU (other streams, other threads) race. */
size_t gq_gemm_static_max_bytes(void);
int gq_gemm_static(int fmt, const void *d_packed, const void *d_a, int a_dtype, void *d_c, int c_dtype, size_t M,
                   size_t N, size_t K, void *stream);

/* Q8_0 x int8 activations (int8 MFMA): activations quantized per 32-block with
 * the reference's INT8 rule (d = amax/127, q = round(a / d)).  d_qa int8
 * [M][K] (16-byte aligned), d_da f32 [M][K/32], d_c f32 [M][N]. */
int gq_quantize_act_q8(const void *d_a, int a_dtype, size_t M, size_t K, int8_t *d_q, float *d_d,
                       void *stream);
int gq_gemm_q8_i8(const void *d_packed_q8, const int8_t *d_qa, const float *d_da, float *d_c, size_t M,
                  size_t N, size_t K, void *stream);

/* ---- GretaCompute::gemm routing for GGUF-native B (greta_compute_hip.cpp:148)
 * M <= 16 -> GEMV kernels, otherwise gq_gemm.  A f32 [M][K], C f32. */
int gq_matmul(int fmt, const void *d_packed, const float *d_a, float *d_c, size_t M, size_t N, size_t K,
              void *stream);

/* ---- reference-format launchers (drop-in for gemm_kernels.hpp:43-57) ------- */
/* INT8 weight-only: b int8 [N][K], scales f32 [N*K/group_size]. */
int gq_launch_gemm_mfma_int8_wt_fp32_acc32(void *stream, const float *a, const int8_t *b, float *c,
                                            const float *scales, uint32_t M, uint32_t N, uint32_t K,
                                            uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t group_size);
/* INT4 weight-only: b packed nibbles [N][K/2] (even k low, two's complement),
 * optional head_scales [N/head_dim]; a is f32, or f16 when is_fp16_a != 0. */
int gq_launch_gemm_mfma_int4_wt_fp32_acc32(void *stream, const void *a, const int8_t *b, float *c,
                                            const float *scales, const float *head_scales, uint32_t M,
                                            uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc,
                                            uint32_t group_size, uint32_t head_dim, int is_fp16_a,
                                            int force_gemv);

/* ---- FP16 weights --------------------------------------------------------
 * The reference's FP16 route: GretaCompute::gemm with FP16 B
 * (greta_compute_hip.cpp:361-371) -> launch_gemm_mixed_f16f32 /
 * launch_gemm_mfma_mixed_f16f32 (gemm_kernels.hpp:30-44, gemm_kernels.hip:
 * 294-358, 387-523): C[M][N] = A[M][K] W^T, A fp32, W fp16 row-major N x K
 * (GGUF F16 tensors, e.g. a dequantized lm_head), C fp32.  Here on the fp16
 * matrix cores in batches of up to 16 rows of A (fp32 accumulation; A rounded
 * to fp16 after a per-window power-of-two scaling) when K % 32 == 0 and d_w and
 * d_a are 16-byte aligned; any other K or alignment runs a plain fp32-accumulating
 * kernel (fp32 A times the fp16 weight, as the reference's VALU route).  Rows of
 * A beyond 16 take further launches, each streaming W again. */
int gq_gemm_f16w(const void *d_w, const float *d_a, float *d_c, size_t M, size_t N, size_t K, void *stream);
/* The two reference launchers under their argument lists; lda must be K and
 * ldc N (what GretaCompute::gemm passes), ldb is ignored as in the reference. */
int gq_launch_gemm_mixed_f16f32(void *stream, const float *a, const void *b, float *c, uint32_t M, uint32_t N,
                                uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc);
int gq_launch_gemm_mfma_mixed_f16f32(void *stream, const float *a, const void *b, float *c, uint32_t M, uint32_t N,
                                     uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc);

#ifdef __cplusplus
}
#endif
#endif
