// gq_internal.h -- shared declarations of the libgq implementation files.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/gq.h"
#include "gq_device.h"
#include "gq_layout.h"
#include "gq_repack_impl.h"

#define GQ_CHECK(cond, code) \
  do {                       \
    if (!(cond)) return (code); \
  } while (0)
#define GQ_TRY(expr)          \
  do {                        \
    int _st = (expr);         \
    if (_st != GQ_OK) return _st; \
  } while (0)

// Records the HIP error (if any) of the last launch and maps it to a status.
int gq_last_launch(void);
int gq_hip_status(hipError_t e);

// Validates (fmt, N, K): known format, K a multiple of the block size, sizes
// within GQ_MAX_DIM.
static inline int gq_check_shape(int fmt, size_t N, size_t K) {
  if (!gq_fmt_valid(fmt)) return GQ_ERR_UNSUPPORTED;
  if (N > GQ_MAX_DIM || K > GQ_MAX_DIM) return GQ_ERR_INVALID_ARGS;
  if (K % gq_block_elems(fmt)) return GQ_ERR_INVALID_ARGS;
  return GQ_OK;
}

static inline size_t gq_align256(size_t v) { return (v + 255) & ~(size_t)255; }
// padded K of the T16 layout
static inline size_t gq_kpad(int fmt, size_t K) { return gq_chunks(fmt, K) * gq_chunk_k(fmt); }
// GEMV workspace (batch > 4): int8 limbs [B][2][Kp] then a zero region of Kp
// bytes, then per (batch row, 32-block) float4 (s, S, s / 254, 0).
static inline size_t gq_xl_bytes(int fmt, size_t K, int B) {
  return gq_align256(((size_t)2 * B + 1) * gq_kpad(fmt, K));
}
static inline size_t gq_scl_bytes(int fmt, size_t K, int B) {
  return gq_align256((size_t)B * (gq_kpad(fmt, K) / 32) * 16);
}

// Zero-fills n floats with a kernel (no memset node, so it is safe to capture).
int gq_fill_zero(float *p, size_t n, hipStream_t s);
int gq_launch_prep_x(int fmt, const float *x, void *ws, int B, int K, hipStream_t s);

// fp16 batch GEMV (gq_gemv_h.hip)
int gq_gemv_h_min(void);
int gq_gemv_h_plan(int fmt, size_t N, size_t K, int nb, int *R_out, int *ks_out, int *cpw_out);
int gq_gemv_h1_plan(int fmt, size_t N, size_t K, int nb, int *R_out, int *ks_out, int *cpw_out);
int gq_launch_gemv_h(int fmt, const void *packed, const float *x, float *y, int N, int K, int nb, hipStream_t s);

// skinny GEMM for M <= 256 (gq_gemv_h.hip); A fp16 in the B fragments' order
// (k_a_to_f16 with the 4-bit permutation for Q4_0 / Q4_K); rs: per-row
// factors applied to C (NULL: none)
int gq_gemm_skinny_plan(int fmt, size_t M, size_t N, size_t K, int *ct_out, int *nck_out);
int gq_launch_gemm_skinny(int fmt, const void *packed, const _Float16 *a16, int lda, void *c, const float *rs,
                          int cbf16, int M, int N, int K, hipStream_t s);

// load-time conversions (gq_loadconv.hip)
int gq_launch_dequant_q6_k(const void *blocks, size_t n_blocks, float *out, int ggml, hipStream_t s);
int gq_launch_f16_to_f32(const void *in, size_t n, float *out, hipStream_t s);

// Library-owned per-device workspace (grown on demand, never shrunk).
int gq_default_workspace(size_t bytes, void **ptr);
// Compute units of the current device (cached per device; 0 without a device).
int gq_device_cus(void);
