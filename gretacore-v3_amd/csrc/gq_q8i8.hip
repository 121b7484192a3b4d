// gq_q8i8.hip -- Q8_0 weights x per-32 int8-quantized activations on the int8
// MFMA (v_mfma_i32_32x32x32_i8).  One 32-element block is one MFMA: the exact
// int32 block dot product is scaled by d_a[m][blk] * d_w[n][blk] in fp32 and
// accumulated.  Parity oracle: exact integer block sums with fp64 scale
// products (oracle gqo_gemm_q8_i8).
#include "gq_internal.h"

namespace {

// Workgroup = 4 waves = 64 x 64 of C; each wave owns one 32 x 32 tile and reads
// its operands straight from global memory (L2-resident across the grid).
__global__ void __launch_bounds__(256)
k_gemm_q8_i8(const uint8_t *__restrict__ w, size_t sc_off, const int8_t *__restrict__ qa,
             const float *__restrict__ da, float *__restrict__ c, int M, int N, int K, int C) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 64 + 32 * (wave >> 1), n0 = blockIdx.x * 64 + 32 * (wave & 1);
  const int nb = K / 32;
  const int hl = lane >> 5;           // which 16-byte half of the block
  int am = m0 + (lane & 31);
  if (am >= M) am = M - 1;            // clamped rows are never stored
  int bn = n0 + (lane & 31);
  const bool nvalid = bn < N;
  if (!nvalid) bn = N - 1;
  gq_f16v acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0.f;
  const gq_i16v zero = {};
  for (int blk = 0; blk < nb; ++blk) {
    gq_i4 af = *reinterpret_cast<const gq_i4 *>(qa + (size_t)am * K + blk * 32 + 16 * hl);
    gq_i4 bf = *reinterpret_cast<const gq_i4 *>(w + gq_q8_0_half_off(bn, blk, hl, C));
    float dw = gq_h2f(*reinterpret_cast<const uint16_t *>(w + sc_off + gq_q4_0_d_off(bn, blk, C)));
    gq_i16v D = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, zero, 0, 0, 0);
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      int m = m0 + 8 * (v >> 2) + 4 * hl + (v & 3);
      if (m >= M) m = M - 1;
      float s = da[(size_t)m * nb + blk] * dw;
      acc[v] += s * (float)D[v];
    }
  }
  if (!nvalid) return;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    int m = m0 + 8 * (v >> 2) + 4 * hl + (v & 3);
    if (m < M) c[(size_t)m * N + n0 + (lane & 31)] = acc[v];
  }
}

}  // namespace

extern "C" int gq_gemm_q8_i8(const void *packed, const int8_t *qa, const float *da, float *c, size_t M, size_t N,
                             size_t K, void *stream) {
  GQ_TRY(gq_check_shape(GQ_FMT_Q8_0, N, K));
  GQ_CHECK(M <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(packed && qa && da && c, GQ_ERR_INVALID_ARGS);
  if (M == 0 || N == 0) return GQ_OK;
  GQ_CHECK(K > 0, GQ_ERR_INVALID_ARGS);
  const int C = (int)gq_chunks(GQ_FMT_Q8_0, K);
  dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
  hipLaunchKernelGGL(k_gemm_q8_i8, grid, dim3(256), 0, (hipStream_t)stream, (const uint8_t *)packed,
                     gq_sc_plane_offset(GQ_FMT_Q8_0, N, K), qa, da, c, (int)M, (int)N, (int)K, C);
  return gq_last_launch();
}
