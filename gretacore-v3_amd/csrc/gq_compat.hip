// gq_compat.hip -- the reference's INT8 / INT4 weight-only launchers, with the
// same arguments, for callers that keep the reference's requantized weight
// formats (weight_loader.cpp:668-1008):
//   launch_gemm_mfma_int8_wt_fp32_acc32  gemm_kernels.hip:742-760
//   launch_gemm_mfma_int4_wt_fp32_acc32  gemm_kernels.hip:910-942
// Semantics: c[m][n] = (sum_k a[m][k] * (w[n][k] * s[(n*K + k)/gs])) * h[n/hd]
// with fp32 accumulation, written in the mathematical ("row") layout
// c[m*ldc + n].  Rows of a are lda apart.  M, N or K == 0 returns at once.
//
// One wave per output row n: lanes stream the row's weights with 16-byte loads
// (16 int8 / 32 nibbles per lane per step) and accumulate all M activation
// rows at once (M <= 32 per pass), reducing with DPP-backed shuffles.
#include "gq_internal.h"

namespace {

GQ_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename TA>
GQ_DEV float ld_a(const TA *p) { return (float)*p; }

template <int MB, typename TA, bool INT4>
__global__ void __launch_bounds__(256)
k_compat_gemv(const TA *__restrict__ a, const uint8_t *__restrict__ b, float *__restrict__ c,
              const float *__restrict__ scales, const float *__restrict__ head_scales, int M, int N, int K,
              int lda, int ldc, int gs, int head_dim, int m_base) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= N) return;
  const int mcount = min(MB, M - m_base);
  float acc[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) acc[i] = 0.f;
  const size_t row_elems = (size_t)n * K;
  // lane covers 16 consecutive k per step; the wave covers 1024 k per step
  for (int k0 = lane * 16; k0 < K; k0 += 1024) {
    float wv[16];
    if (k0 + 16 <= K && (K % 16) == 0) {
      if constexpr (INT4) {
        gq_u2 p = gq_ld8(b + (row_elems + k0) / 2);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          uint32_t byte = (p[e >> 3] >> (8 * ((e >> 1) & 3))) & 0xFFu;
          int v = (e & 1) ? (int)(byte >> 4) : (int)(byte & 15u);
          v = (v ^ 8) - 8;
          wv[e] = (float)v;
        }
      } else {
        gq_u4 p = gq_ld16(b + row_elems + k0);
#pragma unroll
        for (int e = 0; e < 16; ++e) wv[e] = (float)(int8_t)((p[e >> 2] >> (8 * (e & 3))) & 0xFFu);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) wv[e] = wv[e] * (scales ? scales[(row_elems + k0 + e) / gs] : 1.0f);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        int k = k0 + e;
        float v = 0.f;
        if (k < K) {
          size_t idx = row_elems + k;
          int q;
          if constexpr (INT4) {
            uint32_t byte = b[idx / 2];
            q = (idx & 1) ? (int)(byte >> 4) : (int)(byte & 15u);
            q = (q ^ 8) - 8;
          } else {
            q = (int8_t)b[idx];
          }
          v = (float)q * (scales ? scales[idx / gs] : 1.0f);
        }
        wv[e] = v;
      }
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if (i >= mcount) break;
      const TA *ar = a + (size_t)(m_base + i) * lda;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        int k = k0 + e;
        float x = k < K ? ld_a(ar + k) : 0.f;
        acc[i] += x * wv[e];
      }
    }
  }
  float h = (head_scales && head_dim > 0) ? head_scales[n / head_dim] : 1.0f;
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    if (i >= mcount) break;
    float s = wave_sum(acc[i]);
    if (lane == 0) c[(size_t)(m_base + i) * ldc + n] = s * h;
  }
}

// Streaming form for K % 16 == 0 and group sizes that are multiples of 16 (a
// lane's 16 k then share one scale): a wave takes RW = 4 rows and walks K in
// 1024-k segments, 16 k per lane; per segment it loads the MB activation rows'
// 16 values once (float4 loads) for all its rows, each row's 16 weights with
// one 16- (INT8) or 8-byte (INT4) load and one scale, and accumulates
// s * sum(q * x) in fp32.  The sum over a lane's 16 terms is then scaled once
// where the reference scales each weight: the result differs only by fp32
// rounding order.
template <int MB, int RW, typename TA, bool INT4>
__global__ void __launch_bounds__(256)
k_compat_gemv_seg(const TA *__restrict__ a, const uint8_t *__restrict__ b, float *__restrict__ c,
                  const float *__restrict__ scales, const float *__restrict__ head_scales, int M, int N, int K,
                  int lda, int ldc, int gs, int head_dim) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = ((int)blockIdx.x * 4 + wave) * RW;
  if (n0 >= N) return;
  const int m_base = (int)blockIdx.y * MB;
  const int mcount = min(MB, M - m_base);
  float acc[RW][MB];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[r][i] = 0.f;
  const TA *arow[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) arow[i] = a + (size_t)(m_base + (i < mcount ? i : 0)) * lda;
#pragma unroll 2
  for (int k0 = 16 * lane; k0 < K; k0 += 1024) {
    float xv[MB][16];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      if constexpr (sizeof(TA) == 4) {
        const gq_f4 *p = reinterpret_cast<const gq_f4 *>(reinterpret_cast<const float *>(arow[i]) + k0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const gq_f4 v = p[q];
          xv[i][4 * q] = v[0];
          xv[i][4 * q + 1] = v[1];
          xv[i][4 * q + 2] = v[2];
          xv[i][4 * q + 3] = v[3];
        }
      } else {
        const gq_half8 *p = reinterpret_cast<const gq_half8 *>(reinterpret_cast<const _Float16 *>(arow[i]) + k0);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const gq_half8 v = p[q];
#pragma unroll
          for (int e = 0; e < 8; ++e) xv[i][8 * q + e] = (float)v[e];
        }
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = n0 + r < N ? n0 + r : N - 1;  // (rows past N are computed, never stored)
      const size_t idx = (size_t)n * K + k0;
      float wv[16];
      if constexpr (INT4) {
        const gq_u2 p = gq_ld8(b + idx / 2);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t byte = (p[e >> 3] >> (8 * ((e >> 1) & 3))) & 0xFFu;
          const int v = (int)((e & 1) ? (byte >> 4) : (byte & 15u));
          wv[e] = (float)((v ^ 8) - 8);
        }
      } else {
        const gq_u4 p = gq_ld16(b + idx);
#pragma unroll
        for (int e = 0; e < 16; ++e) wv[e] = (float)(int8_t)((p[e >> 2] >> (8 * (e & 3))) & 0xFFu);
      }
      const float sc = scales ? scales[idx / gs] : 1.0f;
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) d += xv[i][e] * wv[e];
        acc[r][i] += sc * d;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = n0 + r;
    const float h = (head_scales && head_dim > 0 && n < N) ? head_scales[n / head_dim] : 1.0f;
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const float sum = wave_sum(acc[r][i]);
      if (lane == 0 && n < N && i < mcount) c[(size_t)(m_base + i) * ldc + n] = sum * h;
    }
  }
}

template <typename TA, bool INT4>
int launch_compat(hipStream_t s, const TA *a, const uint8_t *b, float *c, const float *sc, const float *hs, int M,
                  int N, int K, int lda, int ldc, int gs, int hd) {
  const bool seg = K % 16 == 0 && (!sc || gs % 16 == 0) && lda % (sizeof(TA) == 4 ? 4 : 8) == 0 &&
                   (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0;
  if (seg) {
    // MB activation rows per pass (the passes re-read the weights)
    const int mb = M >= 4 ? 4 : M >= 2 ? 2 : 1;
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + mb - 1) / mb));
    if (mb == 4)
      hipLaunchKernelGGL((k_compat_gemv_seg<4, 4, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda,
                         ldc, gs, hd);
    else if (mb == 2)
      hipLaunchKernelGGL((k_compat_gemv_seg<2, 4, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda,
                         ldc, gs, hd);
    else
      hipLaunchKernelGGL((k_compat_gemv_seg<1, 4, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda,
                         ldc, gs, hd);
    return gq_last_launch();
  }
  dim3 grid((unsigned)((N + 3) / 4));
  for (int m = 0; m < M; m += 8)
    hipLaunchKernelGGL((k_compat_gemv<8, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda, ldc,
                       gs, hd, m);
  return gq_last_launch();
}

}  // namespace

extern "C" int gq_launch_gemm_mfma_int8_wt_fp32_acc32(void *stream, const float *a, const int8_t *b, float *c,
                                                       const float *scales, uint32_t M, uint32_t N, uint32_t K,
                                                       uint32_t lda, uint32_t ldb, uint32_t ldc,
                                                       uint32_t group_size) {
  (void)ldb;
  if (M == 0 || N == 0 || K == 0) return GQ_OK;
  GQ_CHECK(a && b && c, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(!scales || group_size > 0, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(M <= GQ_MAX_DIM && N <= GQ_MAX_DIM && K <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  return launch_compat<float, false>((hipStream_t)stream, a, (const uint8_t *)b, c, scales, nullptr, (int)M, (int)N,
                                     (int)K, (int)(lda ? lda : K), (int)(ldc ? ldc : N), (int)group_size, 0);
}

extern "C" int gq_launch_gemm_mfma_int4_wt_fp32_acc32(void *stream, const void *a, const int8_t *b, float *c,
                                                       const float *scales, const float *head_scales, uint32_t M,
                                                       uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                                                       uint32_t ldc, uint32_t group_size, uint32_t head_dim,
                                                       int is_fp16_a, int force_gemv) {
  (void)ldb;
  (void)force_gemv;  // one kernel serves both of the reference's routes
  if (M == 0 || N == 0 || K == 0) return GQ_OK;
  GQ_CHECK(a && b && c, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(!scales || group_size > 0, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(M <= GQ_MAX_DIM && N <= GQ_MAX_DIM && K <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  hipStream_t s = (hipStream_t)stream;
  const int ld = (int)(lda ? lda : K), lc = (int)(ldc ? ldc : N);
  if (is_fp16_a)
    return launch_compat<_Float16, true>(s, (const _Float16 *)a, (const uint8_t *)b, c, scales, head_scales, (int)M,
                                         (int)N, (int)K, ld, lc, (int)group_size, (int)head_dim);
  return launch_compat<float, true>(s, (const float *)a, (const uint8_t *)b, c, scales, head_scales, (int)M, (int)N,
                                    (int)K, ld, lc, (int)group_size, (int)head_dim);
}
