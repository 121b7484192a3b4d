// gq_compat.hip -- the reference's INT8 / INT4 weight-only launchers, with the
// same arguments, for callers that keep the reference's requantized weight
// formats (weight_loader.cpp:668-1008):
//   launch_gemm_mfma_int8_wt_fp32_acc32  gemm_kernels.hip:742-760
//   launch_gemm_mfma_int4_wt_fp32_acc32  gemm_kernels.hip:910-942
// Semantics: c[m][n] = (sum_k a[m][k] * (w[n][k] * s[idx(n, k)])) * h[n/hd]
// with fp32 accumulation, written in the mathematical ("row") layout
// c[m*ldc + n].  Rows of a are lda apart.  M, N or K == 0 returns at once.
//
// Up to 32 rows (and with force_gemv) the GEMV in fp32, as the reference's
// GEMV kernels; above, the reference's MFMA route on fp16 operands through
// gq_gemm (compat_gemm_route).
#include "gq_internal.h"

namespace {

// Scale of weight (n, k).  The reference's two routes index the per-group
// scales differently: its GEMV kernels (M <= 32 or force_gemv) take
// s_row = scales + (n*K)/gs and s_row[k/gs] (gemm_kernels.hip:610,615 and
// 781,796-797), its MFMA kernels (M > 32) scales[(n*K + k)/gs]
// (gemm_kernels.hip:717, 886).  srow selects the first form; the two agree
// whenever K % gs == 0.
GQ_DEV size_t scale_idx(size_t n, size_t K, size_t k, int gs, int srow) {
  return srow ? (n * K) / (size_t)gs + k / (size_t)gs : (n * K + k) / (size_t)gs;
}
// The same with the row's part computed once: for row n, q0 = (n K) / gs and
// r0 = (n K) % gs; a lane's index for k is then q0 + k / gs (srow) or
// q0 + (r0 + k) / gs, one 32-bit division -- a shift where gs is a power of
// two (gsh >= 0) -- instead of a 64-bit division per load.
struct RowScale {
  size_t q0;
  uint32_t r0;
};
GQ_DEV RowScale row_scale(size_t n, size_t K, int gs) {
  const size_t nk = n * K;
  return RowScale{nk / (size_t)gs, (uint32_t)(nk % (size_t)gs)};
}
GQ_DEV int gs_shift(int gs) { return (gs & (gs - 1)) == 0 ? __builtin_ctz((unsigned)gs) : -1; }
GQ_DEV size_t scale_idx_row(RowScale rsc, uint32_t k, int gs, int gsh, int srow) {
  const uint32_t x = srow ? k : rsc.r0 + k;
  return rsc.q0 + (gsh >= 0 ? x >> gsh : x / (uint32_t)gs);
}

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
              int lda, int ldc, int gs, int srow, int head_dim, int m_base) {
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
      for (int e = 0; e < 16; ++e) wv[e] = wv[e] * (scales ? scales[scale_idx(n, K, k0 + e, gs, srow)] : 1.0f);
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
          v = (float)q * (scales ? scales[scale_idx(n, K, k, gs, srow)] : 1.0f);
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
                  int lda, int ldc, int gs, int srow, int head_dim) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
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
  const int gsh = gs_shift(gs);
  RowScale rsc[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) rsc[r] = row_scale((size_t)(n0 + r < N ? n0 + r : N - 1), (size_t)K, gs);
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
      const float sc = scales ? scales[scale_idx_row(rsc[r], (uint32_t)k0, gs, gsh, srow)] : 1.0f;
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

// One-row-per-wave form with the activations in LDS (fp32, all of K for MB
// rows, staged once per workgroup of 16 waves): the activation traffic per
// workgroup is K * MB * 4 bytes for 16 rows instead of per wave.  Each lane
// takes 16 k per 1024-k segment; its weights for all segments are requested
// up front (at most NSEG segments).  The LDS holds 16-byte chunks at
// c ^ ((c >> 4) & 3) so the four 16-byte reads of a lane's 16 values hit 16
// different bank groups across each 16 lanes.
template <int MB, int NSEG, typename TA, bool INT4, int RW = 1>
__global__ void __launch_bounds__(1024)
k_compat_gemv_lds(const TA *__restrict__ a, const uint8_t *__restrict__ b, float *__restrict__ c,
                  const float *__restrict__ scales, const float *__restrict__ head_scales, int M, int N, int K,
                  int lda, int ldc, int gs, int srow, int head_dim) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];
  gq_f4 *xs = reinterpret_cast<gq_f4 *>(lds_raw);  // [MB][K / 4] chunks, swizzled
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m_base = (int)blockIdx.y * MB;
  const int mcount = min(MB, M - m_base);
  const int n0 = ((int)blockIdx.x * 16 + __builtin_amdgcn_readfirstlane(wave)) * RW;
  const int nseg = (K + 1023) / 1024;
  const int gsh = gs_shift(gs);
  // weights and scales of every segment of the wave's RW rows first (clamped,
  // unconditional; a row past N is computed, never stored)
  gq_u4 w8[RW][INT4 ? 1 : NSEG];
  gq_u2 w4[RW][INT4 ? NSEG : 1];
  float sc[RW][NSEG];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int nr = n0 + r < N ? n0 + r : N - 1;
    const RowScale rsc = row_scale((size_t)nr, (size_t)K, gs);
#pragma unroll
    for (int it = 0; it < NSEG; ++it) {
      int k0 = 16 * lane + 1024 * it;
      k0 = k0 < K ? k0 : K - 16;
      const size_t idx = (size_t)nr * K + k0;
      if constexpr (INT4) w4[r][it] = gq_ld8(b + idx / 2);
      else w8[r][it] = gq_ld16(b + idx);
      sc[r][it] = scales ? scales[scale_idx_row(rsc, (uint32_t)k0, gs, gsh, srow)] : 1.0f;
    }
  }
  // activations -> LDS
  const int nchunk = K / 4;
  for (int i = (int)threadIdx.x; i < MB * nchunk; i += 1024) {
    const int row = i / nchunk, ch = i % nchunk;
    gq_f4 v = gq_f4{0.f, 0.f, 0.f, 0.f};
    if (row < mcount) {
      const TA *src = a + (size_t)(m_base + row) * lda + 4 * ch;
      if constexpr (sizeof(TA) == 4) {
        v = *reinterpret_cast<const gq_f4 *>(src);
      } else {
        const _Float16 *h = reinterpret_cast<const _Float16 *>(src);
        v = gq_f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
      }
    }
    xs[row * nchunk + (ch ^ ((ch >> 4) & 3))] = v;
  }
  __syncthreads();
  float acc[RW][MB];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[r][i] = 0.f;
#pragma unroll
  for (int it = 0; it < NSEG; ++it) {
    const int k0 = 16 * lane + 1024 * it;
    if (it < nseg && k0 < K) {
      float xv[MB][16];
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int ch = k0 / 4 + j;
          const gq_f4 x4 = xs[i * nchunk + (ch ^ ((ch >> 4) & 3))];
          xv[i][4 * j] = x4[0];
          xv[i][4 * j + 1] = x4[1];
          xv[i][4 * j + 2] = x4[2];
          xv[i][4 * j + 3] = x4[3];
        }
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        float wv[16];
        if constexpr (INT4) {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const uint32_t byte = (w4[r][it][e >> 3] >> (8 * ((e >> 1) & 3))) & 0xFFu;
            const int v = (int)((e & 1) ? (byte >> 4) : (byte & 15u));
            wv[e] = (float)((v ^ 8) - 8);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e) wv[e] = (float)(int8_t)((w8[r][it][e >> 2] >> (8 * (e & 3))) & 0xFFu);
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 16; ++e) d += xv[i][e] * wv[e];
          acc[r][i] += sc[r][it] * d;
        }
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
                  int N, int K, int lda, int ldc, int gs, int srow, int hd) {
  const bool seg = K % 16 == 0 && (!sc || gs % 16 == 0) && lda % (sizeof(TA) == 4 ? 4 : 8) == 0 &&
                   (uintptr_t)a % 16 == 0 && (uintptr_t)b % 16 == 0;
  // activations staged in LDS per 16-row workgroup (K <= 16384), else read
  // per wave (4096 x 4096 M = 1 / 8: 5.9 / 14.2 us against 7.5 / 20)
  if (seg && K <= 16384) {
    const int mb = (M >= 4 && K <= 4096) ? 4 : (M >= 2 && K <= 8192) ? 2 : 1;
    const size_t lds = (size_t)mb * K * 4;
    // INT4, one activation row, tall matrices: two rows per wave (twice the
    // weight bytes in flight per wave; 14336 x 4096: 14.3 -> 13.5 us) while
    // the grid keeps a workgroup per CU
    const bool rw2 = INT4 && mb == 1 && K <= 4096 && N >= 8192;
    dim3 grid((unsigned)((N + (rw2 ? 31 : 15)) / (rw2 ? 32 : 16)), (unsigned)((M + mb - 1) / mb));
    if (rw2) {
      hipLaunchKernelGGL((k_compat_gemv_lds<1, 4, TA, INT4, 2>), grid, dim3(1024), lds, s, a, b, c, sc, hs, M, N, K,
                         lda, ldc, gs, srow, hd);
      return gq_last_launch();
    }
#define GQ_LDS_L(MBV, NS)                                                                                       \
  hipLaunchKernelGGL((k_compat_gemv_lds<MBV, NS, TA, INT4>), grid, dim3(1024), lds, s, a, b, c, sc, hs, M, N, K, \
                     lda, ldc, gs, srow, hd)
    const int nseg = (K + 1023) / 1024;
    if (mb == 4) GQ_LDS_L(4, 4);
    else if (mb == 2) { if (nseg <= 4) GQ_LDS_L(2, 4); else GQ_LDS_L(2, 8); }
    else { if (nseg <= 4) GQ_LDS_L(1, 4); else if (nseg <= 8) GQ_LDS_L(1, 8); else GQ_LDS_L(1, 16); }
#undef GQ_LDS_L
    return gq_last_launch();
  }
  if (seg) {
    // MB activation rows per pass (the passes re-read the weights)
    const int mb = M >= 4 ? 4 : M >= 2 ? 2 : 1;
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + mb - 1) / mb));
    if (mb == 4)
      hipLaunchKernelGGL((k_compat_gemv_seg<4, 4, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda,
                         ldc, gs, srow, hd);
    else if (mb == 2)
      hipLaunchKernelGGL((k_compat_gemv_seg<2, 4, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda,
                         ldc, gs, srow, hd);
    else
      hipLaunchKernelGGL((k_compat_gemv_seg<1, 4, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda,
                         ldc, gs, srow, hd);
    return gq_last_launch();
  }
  dim3 grid((unsigned)((N + 3) / 4));
  for (int m = 0; m < M; m += 8)
    hipLaunchKernelGGL((k_compat_gemv<8, TA, INT4>), grid, dim3(256), 0, s, a, b, c, sc, hs, M, N, K, lda, ldc,
                       gs, srow, hd, m);
  return gq_last_launch();
}

// Reference INT8 / INT4 rows -> GGUF Q8_0 / Q4_0 blocks for the MFMA GEMM
// route, one thread per 32-block: d = fp16(s * h) (the group's scale times the
// row's head scale), INT8 codes as they are, INT4 codes q (two's complement,
// even k in the low nibble) as q + 8 in Q4_0's order (low nibbles k 0..15,
// high nibbles k 16..31).  gs % 32 == 0 and K % 32 == 0 (host-checked).
template <bool INT4>
__global__ void __launch_bounds__(256)
k_compat_to_gguf(const uint8_t *__restrict__ b, const float *__restrict__ scales, const float *__restrict__ hs,
                 uint8_t *__restrict__ out, int N, int K, int gs, int head_dim) {
  const size_t blk = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t nblk = (size_t)N * (K / 32);
  if (blk >= nblk) return;
  const int n = (int)(blk / (size_t)(K / 32));
  const size_t e0 = blk * 32;  // first element (n * K + 32 j)
  float sc = scales ? scales[e0 / gs] : 1.0f;
  if (hs && head_dim > 0) sc *= hs[n / head_dim];
  const uint16_t d = __builtin_bit_cast(uint16_t, (_Float16)sc);
  if constexpr (INT4) {
    uint8_t *o = out + blk * 18;
    o[0] = (uint8_t)(d & 0xFF);
    o[1] = (uint8_t)(d >> 8);
    const uint8_t *p = b + e0 / 2;
    uint8_t u[32];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint8_t byte = p[j];
      u[2 * j] = (uint8_t)(((byte & 15) ^ 8));      // q + 8 for q in -8..7
      u[2 * j + 1] = (uint8_t)(((byte >> 4) ^ 8));
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) o[2 + j] = (uint8_t)(u[j] | (u[j + 16] << 4));
  } else {
    uint8_t *o = out + blk * 34;
    o[0] = (uint8_t)(d & 0xFF);
    o[1] = (uint8_t)(d >> 8);
    const uint8_t *p = b + e0;
#pragma unroll
    for (int j = 0; j < 32; ++j) o[2 + j] = p[j];
  }
}

// The reference's MFMA route (M > 32 without force_gemv: gemm_kernels.hip:
// 910-942, 742-760) computes on fp16 operands (A and w * s rounded to fp16);
// here the weights become Q8_0 / Q4_0 blocks (d = fp16(s * h)), are repacked
// into T16 and go through gq_gemm.  Needs lda == K, ldc == N, K % 32 == 0 and
// gs % 32 == 0; the library's per-device workspace holds the converted
// weights (the launchers have no workspace argument).  GQ_ERR_UNSUPPORTED
// when a condition fails (the caller then runs the GEMV).
template <bool INT4>
int compat_gemm_route(hipStream_t s, const void *a, int a_dtype, const uint8_t *b, float *c, const float *sc,
                      const float *hs, int M, int N, int K, int lda, int ldc, int gs, int hd) {
  if (M <= 32 || lda != K || ldc != N || K % 32 || (sc && gs % 32)) return GQ_ERR_UNSUPPORTED;
  const int fmt = INT4 ? GQ_FMT_Q4_0 : GQ_FMT_Q8_0;
  const size_t nblk = (size_t)N * (K / 32);
  const size_t gguf = gq_align256(nblk * (INT4 ? 18 : 34));
  const size_t packed = gq_align256(gq_packed_bytes(fmt, N, K));
  const size_t gws = gq_gemm_workspace_bytes(fmt, M, K);
  void *ws = nullptr;
  GQ_TRY(gq_default_workspace(gguf + packed + gws, &ws));
  uint8_t *wg = (uint8_t *)ws, *wp = wg + gguf, *wa = wp + packed;
  hipLaunchKernelGGL((k_compat_to_gguf<INT4>), dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, b, sc, hs, wg,
                     N, K, gs, hd);
  GQ_TRY(gq_last_launch());
  GQ_TRY(gq_repack(fmt, wg, N, K, wp, s));
  return gq_gemm(fmt, wp, a, a_dtype, c, GQ_DT_F32, M, N, K, wa, gws, s);
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
  const int ld = (int)(lda ? lda : K), lc = (int)(ldc ? ldc : N);
  const int r = compat_gemm_route<false>((hipStream_t)stream, a, GQ_DT_F32, (const uint8_t *)b, c, scales, nullptr,
                                         (int)M, (int)N, (int)K, ld, lc, (int)group_size, 0);
  if (r != GQ_ERR_UNSUPPORTED) return r;
  // past the MFMA route's conditions the GEMV computes the MFMA route's scale
  // index for M > 32
  return launch_compat<float, false>((hipStream_t)stream, a, (const uint8_t *)b, c, scales, nullptr, (int)M, (int)N,
                                     (int)K, ld, lc, (int)group_size, M <= 32 ? 1 : 0, 0);
}

extern "C" int gq_launch_gemm_mfma_int4_wt_fp32_acc32(void *stream, const void *a, const int8_t *b, float *c,
                                                       const float *scales, const float *head_scales, uint32_t M,
                                                       uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                                                       uint32_t ldc, uint32_t group_size, uint32_t head_dim,
                                                       int is_fp16_a, int force_gemv) {
  (void)ldb;
  if (M == 0 || N == 0 || K == 0) return GQ_OK;
  GQ_CHECK(a && b && c, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(!scales || group_size > 0, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(M <= GQ_MAX_DIM && N <= GQ_MAX_DIM && K <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  // the reference addresses row n at byte n*(K/2) (gemm_kernels.hip:781, 859)
  // while its loader packs the flat tensor (weight_loader.cpp:920-957): the
  // two agree only for even K
  GQ_CHECK(K % 2 == 0, GQ_ERR_UNSUPPORTED);
  hipStream_t s = (hipStream_t)stream;
  const int ld = (int)(lda ? lda : K), lc = (int)(ldc ? ldc : N);
  const int srow = (force_gemv || M <= 32) ? 1 : 0;  // the GEMV route's scale index
  if (!force_gemv) {  // the reference's MFMA route for M > 32
    const int r = compat_gemm_route<true>(s, a, is_fp16_a ? GQ_DT_F16 : GQ_DT_F32, (const uint8_t *)b, c, scales,
                                          head_scales, (int)M, (int)N, (int)K, ld, lc, (int)group_size,
                                          (int)head_dim);
    if (r != GQ_ERR_UNSUPPORTED) return r;
  }
  if (is_fp16_a)
    return launch_compat<_Float16, true>(s, (const _Float16 *)a, (const uint8_t *)b, c, scales, head_scales, (int)M,
                                         (int)N, (int)K, ld, lc, (int)group_size, srow, (int)head_dim);
  return launch_compat<float, true>(s, (const float *)a, (const uint8_t *)b, c, scales, head_scales, (int)M, (int)N,
                                    (int)K, ld, lc, (int)group_size, srow, (int)head_dim);
}
