// gq_gemv.hip -- decode GEMV (batch 1..16) over T16-repacked GGUF weights.
//
// Replaces gemv_int8_wt_kernel / gemv_int4_wt_kernel
// (src/rt/backend/hip/kernels/gemm_kernels.hip:594-634, 763-817) for
// GGUF-native weights: y[b][n] = sum_k x[b][k] * W[n][k].
//
// Design (CDNA4, wave64):
//  * One workgroup per 16-row tile; its KSPLIT waves split the K axis and meet
//    in LDS at the end.  Each wave first issues the loads of ALL its chunks
//    (one dwordx4 per lane per chunk: 1 KiB per wave, fully coalesced), so the
//    whole weight stream is in flight at once, then consumes them in order.
//  * Weights become fp16 MFMA operands without any float math: a 4-bit (or
//    offset 8-bit) code placed in the low bits of an fp16 is the subnormal
//    value code * 2^-24, which the matrix cores multiply exactly.  So a
//    canonical Q4 word turns into four operand pairs with one shift and one AND
//    each.  The 2^-24 is folded into the final store; the GGUF offsets (q - 8,
//    q - 128) are applied per block as d * 8 * S with S = sum of x over the
//    block.  Q4_K folds its 6-bit sub-block scale into the code
//    (sc * q <= 945 still fits the subnormal mantissa) and gets
//    sum_j m_j * S_j from one extra MFMA per super-block.
//  * Dot products run on v_mfma_f32_16x16x32_f16 with A = activations (rows =
//    batch rows) and B = the weight tile (cols = 16 weight rows).  The fp32
//    activation is split into fp16 hi + lo rows (x = hi + lo to ~2^-22), so no
//    precision is lost to fp16; hi and lo ride in spare MFMA rows.
//  * Batch <= 2 (decode): each wave converts its own K slice of the fp32
//    activations into LDS (hi/lo rows + block sums) -- no separate kernel.
//    Batch 3..16: a small prep kernel writes the same data to a workspace once
//    and the GEMV reads its operands from there (L2-resident).
#include <stdlib.h>

#include "gq_internal.h"

namespace {

constexpr float kTwo24 = 16777216.0f;

template <int FMT>
struct Fmt;
template <>
struct Fmt<GQ_FMT_Q4_0> {
  static constexpr int CK = 128, QB = 1024, SB = 128, MAXC = 8;
};
template <>
struct Fmt<GQ_FMT_Q8_0> {
  static constexpr int CK = 128, QB = 2048, SB = 128, MAXC = 8;
};
template <>
struct Fmt<GQ_FMT_Q4_K> {
  static constexpr int CK = 256, QB = 2048, SB = 256, MAXC = 4;
};

// weight registers of one chunk
template <int FMT>
struct Chunk;
template <>
struct Chunk<GQ_FMT_Q4_0> {
  gq_u4 q;
  gq_u2 d;
};
template <>
struct Chunk<GQ_FMT_Q8_0> {
  gq_u4 q0, q1;
  gq_u2 d;
};
template <>
struct Chunk<GQ_FMT_Q4_K> {
  gq_u4 qa, qb, meta;
};

template <int FMT>
GQ_DEV void load_chunk(const uint8_t *qp, const uint8_t *sp, int r, Chunk<FMT> &ch) {
  if constexpr (FMT == GQ_FMT_Q4_0) {
    ch.q = gq_ld16(qp);
    ch.d = gq_ld8(sp + 8 * r);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    ch.q0 = gq_ld16(qp);
    ch.q1 = gq_ld16(qp + 1024);
    ch.d = gq_ld8(sp + 8 * r);
  } else {
    ch.qa = gq_ld16(qp);
    ch.qb = gq_ld16(qp + 1024);
    ch.meta = gq_ld16(sp + 16 * r);
  }
}

// canonical Q4 word -> 4 subnormal-code operand pairs (value q * 2^-24)
GQ_DEV gq_half8 q4_codes(uint32_t w) {
  gq_u4 t;
#pragma unroll
  for (int s = 0; s < 4; ++s) t[s] = (w >> (4 * s)) & 0x000F000Fu;
  return __builtin_bit_cast(gq_half8, t);
}
// canonical Q4 word -> codes sc * q (value sc * q * 2^-24, exact)
GQ_DEV gq_half8 q4_scaled_codes(uint32_t w, uint32_t sc) {
  gq_u4 t;
#pragma unroll
  for (int s = 0; s < 4; ++s) t[s] = __umul24((w >> (4 * s)) & 0x000F000Fu, sc);
  return __builtin_bit_cast(gq_half8, t);
}
// 8 int8 -> codes q + 128 (value (q + 128) * 2^-24)
GQ_DEV gq_half8 q8_codes(uint32_t w0, uint32_t w1) {
  uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  gq_u4 t;
  t[0] = __builtin_amdgcn_perm(0u, u0, 0x04010400u);
  t[1] = __builtin_amdgcn_perm(0u, u0, 0x04030402u);
  t[2] = __builtin_amdgcn_perm(0u, u1, 0x04010400u);
  t[3] = __builtin_amdgcn_perm(0u, u1, 0x04030402u);
  return __builtin_bit_cast(gq_half8, t);
}

GQ_DEV float h16lo(uint32_t v) { return (float)__builtin_bit_cast(gq_half2, v)[0]; }
GQ_DEV float h16hi(uint32_t v) { return (float)__builtin_bit_cast(gq_half2, v)[1]; }


// ---------------------------------------------------------------------------
// Fused path (batch NB <= 2): each wave stages its own K slice of the fp32
// activations in LDS: rows 2b (hi) and 2b+1 (lo), row stride `stride` halves,
// then the per-32-block sums (fp32; Q4_K: fp16 (hi, lo) pairs).
// ---------------------------------------------------------------------------
struct XlLayout {
  int lk, stride, sf_off, wave_bytes;
};
__host__ __device__ inline XlLayout xl_layout(int lk, int nb) {
  XlLayout L;
  L.lk = lk;
  L.stride = lk + 8;
  L.sf_off = 2 * nb * L.stride * 2;
  L.wave_bytes = (L.sf_off + nb * (lk / 32) * 4 + 15) & ~15;
  return L;
}

template <int FMT, int NB, int KSPLIT>
__global__ void __launch_bounds__(64 * KSPLIT)
k_gemv_xl(const uint8_t *__restrict__ w, size_t sc_off, const float *__restrict__ x, float *__restrict__ y, int N,
          int K, int C) {
  using F = Fmt<FMT>;
  constexpr int LKMAX = F::CK * F::MAXC;
  constexpr int TPR = LKMAX / 8 / 64;  // 8-element tasks per batch row per lane
  extern __shared__ __attribute__((aligned(16))) unsigned char gq_dyn_lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const size_t t = blockIdx.x;
  const int c0 = (C * wave) / KSPLIT, c1 = (C * (wave + 1)) / KSPLIT;
  const int nck = c1 - c0;  // <= F::MAXC (host-checked)
  const int k0 = c0 * F::CK, LK = nck * F::CK;
  const XlLayout L = xl_layout(F::CK * ((C + KSPLIT - 1) / KSPLIT), NB);
  unsigned char *lds = gq_dyn_lds + (size_t)wave * L.wave_bytes;
  _Float16 *xs = reinterpret_cast<_Float16 *>(lds);
  float *sf = reinterpret_cast<float *>(lds + L.sf_off);
  const int nblk = L.lk / 32;

  // 1. activation loads first (so waiting for them never waits for weights)
  // Loads are unconditional (out-of-range ones read a clamped valid address
  // and are discarded) so the compiler can count outstanding loads exactly and
  // start on chunk 0 as soon as it lands.
  float4 xv[NB * TPR][2];
  bool xin[NB * TPR];
#pragma unroll
  for (int i = 0; i < NB * TPR; ++i) {
    const int b = i / TPR, e8 = lane + 64 * (i % TPR), k = k0 + 8 * e8;
    xin[i] = 8 * e8 < LK && k < K;
    const float4 *p = reinterpret_cast<const float4 *>(x + (size_t)b * K + (xin[i] ? k : 0));
    xv[i][0] = p[0];
    xv[i][1] = p[1];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weights
  // 2. weight loads for every chunk of this wave
  Chunk<FMT> ch[F::MAXC];
  const uint8_t *qp = w + (t * (size_t)C + c0) * F::QB + 16 * lane;
  const uint8_t *sp = w + sc_off + (t * (size_t)C + c0) * F::SB;
#pragma unroll
  for (int i = 0; i < F::MAXC; ++i) {
    const int ii = i < nck ? i : nck - 1;
    load_chunk<FMT>(qp + (size_t)ii * F::QB, sp + (size_t)ii * F::SB, r, ch[i]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 3. hi/lo split + block sums into LDS
#pragma unroll
  for (int i = 0; i < NB * TPR; ++i) {
    const int b = i / TPR, e8 = lane + 64 * (i % TPR);
    float v[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                  xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = xin[i] ? v[e] : 0.f;
    gq_half8 hi, lo;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hi[e] = (_Float16)v[e];
      lo[e] = (_Float16)(v[e] - (float)hi[e]);
      s += v[e];
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if (8 * e8 < LK) {
      *reinterpret_cast<gq_half8 *>(xs + (2 * b) * L.stride + 8 * e8) = hi;
      *reinterpret_cast<gq_half8 *>(xs + (2 * b + 1) * L.stride + 8 * e8) = lo;
      if ((lane & 3) == 0) {
        const int blk = b * nblk + (e8 >> 2);
        if constexpr (FMT == GQ_FMT_Q4_K) {
          const _Float16 shh = (_Float16)s;
          const gq_half2 pr = {shh, (_Float16)(s - (float)shh)};
          reinterpret_cast<uint32_t *>(sf)[blk] = gq_h2_bits(pr);
        } else {
          sf[blk] = s;
        }
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();

  // 4. consume the chunks.  A rows >= 2NB read real (finite) data: they only
  // feed D rows that are never used, so no masking is needed.
  const int ar = r & (2 * NB - 1);
  const gq_f4 zero4 = {0.f, 0.f, 0.f, 0.f};
  float acc[2 * NB], cor[NB];
#pragma unroll
  for (int v = 0; v < 2 * NB; ++v) acc[v] = 0.f;
#pragma unroll
  for (int u = 0; u < NB; ++u) cor[u] = 0.f;

  if constexpr (FMT == GQ_FMT_Q4_0 || FMT == GQ_FMT_Q8_0) {
    const _Float16 *xa = xs + ar * L.stride + 8 * g;
#pragma unroll
    for (int i = 0; i < F::MAXC; ++i) {
      if (i >= nck) break;
      gq_f4 D[4];
      float sblk[NB][4];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const gq_f4 s4 = *reinterpret_cast<const gq_f4 *>(sf + u * nblk + 4 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) sblk[u][j] = s4[j];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        gq_half8 b;
        if constexpr (FMT == GQ_FMT_Q4_0) {
          b = q4_codes(ch[i].q[j]);
        } else {
          const gq_u4 &qq = (j < 2) ? ch[i].q0 : ch[i].q1;
          b = q8_codes(qq[2 * (j & 1)], qq[2 * (j & 1) + 1]);
        }
        const gq_half8 a = *reinterpret_cast<const gq_half8 *>(xa + i * 128 + 32 * j);
        D[j] = gq_mfma16(a, b, zero4);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float d = (j & 1) ? h16hi(ch[i].d[j >> 1]) : h16lo(ch[i].d[j >> 1]);
#pragma unroll
        for (int v = 0; v < 2 * NB; ++v) acc[v] += d * D[j][v];
#pragma unroll
        for (int u = 0; u < NB; ++u) cor[u] += d * sblk[u][j];
      }
    }
  } else {
    const _Float16 *xa = xs + ar * L.stride + 64 * g;
    const uint32_t *sh = reinterpret_cast<const uint32_t *>(sf);
    const bool hirow = !(ar & 1);
#pragma unroll
    for (int i = 0; i < F::MAXC; ++i) {
      if (i >= nck) break;
      const uint32_t m0w = ch[i].meta[0];
      const float d = h16lo(m0w), dmin = h16hi(m0w);
      uint32_t sc0, m0, sc1, m1;
      gq_q4k_codes(ch[i].meta[1], ch[i].meta[2], ch[i].meta[3], g, sc0, m0, sc1, m1);
      gq_f4 D1 = zero4;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        const int h = tt >> 2;
        const uint32_t word = h ? ch[i].qb[tt & 3] : ch[i].qa[tt & 3];
        const gq_half8 b = q4_scaled_codes(word, h ? sc1 : sc0);
        const gq_half8 a = *reinterpret_cast<const gq_half8 *>(xa + i * 256 + 32 * h + 8 * (tt & 3));
        D1 = gq_mfma16(a, b, D1);
      }
      // min term: A = (S_hi, S_lo) of sub-blocks 2g, 2g+1 on hi rows
      const gq_u2 sp2 = *reinterpret_cast<const gq_u2 *>(sh + (ar >> 1) * nblk + 8 * i + 2 * g);
      gq_u4 at = {0u, 0u, 0u, 0u};
      at[0] = hirow ? ((sp2[0] & 0xFFFFu) | (sp2[1] << 16)) : 0u;
      at[1] = hirow ? ((sp2[0] >> 16) | (sp2[1] & 0xFFFF0000u)) : 0u;
      const gq_u4 bmt = {m0 | (m1 << 16), m0 | (m1 << 16), 0u, 0u};
      const gq_f4 D2 =
          gq_mfma16(__builtin_bit_cast(gq_half8, at), __builtin_bit_cast(gq_half8, bmt), zero4);
#pragma unroll
      for (int v = 0; v < 2 * NB; ++v) acc[v] += d * D1[v] - dmin * D2[v];
    }
  }

  constexpr float OFF = (FMT == GQ_FMT_Q4_0) ? 8.f : (FMT == GQ_FMT_Q8_0) ? 128.f : 0.f;
  float part[NB];
#pragma unroll
  for (int u = 0; u < NB; ++u) part[u] = kTwo24 * (acc[2 * u] + acc[2 * u + 1]) - OFF * cor[u];
  if constexpr (KSPLIT > 1) {
    __shared__ float red[KSPLIT][NB][16];
    if (g == 0) {
#pragma unroll
      for (int u = 0; u < NB; ++u) red[wave][u][r] = part[u];
    }
    __syncthreads();
    if (wave != 0 || g != 0) return;
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      float s = 0.f;
#pragma unroll
      for (int q = 0; q < KSPLIT; ++q) s += red[q][u][r];
      part[u] = s;
    }
  } else if (g != 0) {
    return;
  }
  const size_t row = t * 16 + r;
  if (row < (size_t)N) {
#pragma unroll
    for (int u = 0; u < NB; ++u) y[(size_t)u * N + row] = part[u];
  }
}

// ---------------------------------------------------------------------------
// Workspace path (batch 3..16): operands from the prepared buffers
//   xq [2B][Kp] fp16 (rows 2b hi, 2b+1 lo), sf [B][Kp/32] f32,
//   sh [B][Kp/32] fp16 (hi, lo) sums (Q4_K).
// D rows: lane (g, r) holds rows 16mt + 4g + v, i.e. batch 8mt + 2g + v/2.
// ---------------------------------------------------------------------------
template <int FMT, int MT, int KSPLIT>
__global__ void __launch_bounds__(64 * KSPLIT)
k_gemv_xg(const uint8_t *__restrict__ w, size_t sc_off, const _Float16 *__restrict__ xq,
          const float *__restrict__ sfq, const uint32_t *__restrict__ shq, float *__restrict__ y, int N, int C,
          int Kp, int nb) {
  using F = Fmt<FMT>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const size_t t = blockIdx.x;
  const int c0 = (C * wave) / KSPLIT, c1 = (C * (wave + 1)) / KSPLIT;
  const int nck = c1 - c0;
  const int nsub = Kp / 32;

  Chunk<FMT> ch[F::MAXC];
  const uint8_t *qp = w + (t * (size_t)C + c0) * F::QB + 16 * lane;
  const uint8_t *sp = w + sc_off + (t * (size_t)C + c0) * F::SB;
#pragma unroll
  for (int i = 0; i < F::MAXC; ++i) {
    const int ii = i < nck ? i : nck - 1;
    load_chunk<FMT>(qp + (size_t)ii * F::QB, sp + (size_t)ii * F::SB, r, ch[i]);
  }

  // per-lane operand rows (rows >= 2nb read a valid row; their D rows are unused)
  const _Float16 *xa[MT];
  int ar[MT], bs[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = 16 * mt + r;
    ar[mt] = row < 2 * nb ? row : row % (2 * nb);
    xa[mt] = xq + (size_t)ar[mt] * Kp + (FMT == GQ_FMT_Q4_K ? 64 : 8) * g;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = 8 * mt + 2 * g + u;
      bs[mt][u] = b < nb ? b : 0;
    }
  }
  const gq_f4 zero4 = {0.f, 0.f, 0.f, 0.f};
  gq_f4 acc[MT];
  float cor[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = zero4;
    cor[mt][0] = cor[mt][1] = 0.f;
  }

#pragma unroll
  for (int i = 0; i < F::MAXC; ++i) {
    if (i >= nck) break;
    const int c = c0 + i;
    if constexpr (FMT == GQ_FMT_Q4_0 || FMT == GQ_FMT_Q8_0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        gq_half8 b;
        if constexpr (FMT == GQ_FMT_Q4_0) {
          b = q4_codes(ch[i].q[j]);
        } else {
          const gq_u4 &qq = (j < 2) ? ch[i].q0 : ch[i].q1;
          b = q8_codes(qq[2 * (j & 1)], qq[2 * (j & 1) + 1]);
        }
        const float d = (j & 1) ? h16hi(ch[i].d[j >> 1]) : h16lo(ch[i].d[j >> 1]);
        const int blk = 4 * c + j;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const gq_half8 a = *reinterpret_cast<const gq_half8 *>(xa[mt] + blk * 32);
          acc[mt] += d * gq_mfma16(a, b, zero4);
#pragma unroll
          for (int u = 0; u < 2; ++u) cor[mt][u] += d * sfq[(size_t)bs[mt][u] * nsub + blk];
        }
      }
    } else {
      const uint32_t m0w = ch[i].meta[0];
      const float d = h16lo(m0w), dmin = h16hi(m0w);
      uint32_t sc0, m0, sc1, m1;
      gq_q4k_codes(ch[i].meta[1], ch[i].meta[2], ch[i].meta[3], g, sc0, m0, sc1, m1);
      gq_f4 D1[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) D1[mt] = zero4;
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        const int h = tt >> 2;
        const uint32_t word = h ? ch[i].qb[tt & 3] : ch[i].qa[tt & 3];
        const gq_half8 b = q4_scaled_codes(word, h ? sc1 : sc0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const gq_half8 a = *reinterpret_cast<const gq_half8 *>(xa[mt] + c * 256 + 32 * h + 8 * (tt & 3));
          D1[mt] = gq_mfma16(a, b, D1[mt]);
        }
      }
      const gq_u4 bmt = {m0 | (m1 << 16), m0 | (m1 << 16), 0u, 0u};
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bool hirow = !(ar[mt] & 1);
        const gq_u2 sp2 = *reinterpret_cast<const gq_u2 *>(shq + (size_t)(ar[mt] >> 1) * nsub + 8 * c + 2 * g);
        gq_u4 at = {0u, 0u, 0u, 0u};
        at[0] = hirow ? ((sp2[0] & 0xFFFFu) | (sp2[1] << 16)) : 0u;
        at[1] = hirow ? ((sp2[0] >> 16) | (sp2[1] & 0xFFFF0000u)) : 0u;
        const gq_f4 D2 =
            gq_mfma16(__builtin_bit_cast(gq_half8, at), __builtin_bit_cast(gq_half8, bmt), zero4);
        acc[mt] += d * D1[mt] - dmin * D2;
      }
    }
  }

  constexpr float OFF = (FMT == GQ_FMT_Q4_0) ? 8.f : (FMT == GQ_FMT_Q8_0) ? 128.f : 0.f;
  float part[MT][2];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int u = 0; u < 2; ++u)
      part[mt][u] = kTwo24 * (acc[mt][2 * u] + acc[mt][2 * u + 1]) - OFF * cor[mt][u];
  if constexpr (KSPLIT > 1) {
    __shared__ float red[KSPLIT][MT * 2][64];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int u = 0; u < 2; ++u) red[wave][mt * 2 + u][lane] = part[mt][u];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < KSPLIT; ++q) s += red[q][mt * 2 + u][lane];
        part[mt][u] = s;
      }
  }
  const size_t row = t * 16 + r;
  if (row >= (size_t)N) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = 8 * mt + 2 * g + u;
      if (b < nb) y[(size_t)b * N + row] = part[mt][u];
    }
}

// GQ_GEMV_KSPLIT=1|2|4|8|16 overrides the K-split heuristic (for tuning).
int env_ksplit() {
  const char *e = getenv("GQ_GEMV_KSPLIT");
  return e ? atoi(e) : 0;
}

// K-split: enough waves to cover the chip (~4 per SIMD), each wave holding at
// most MAXC chunks in registers.
template <int FMT>
int pick_ksplit(size_t tiles, int C) {
  using F = Fmt<FMT>;
  int ks = 1;
  while (ks < 16 && (C + ks - 1) / ks > F::MAXC) ks *= 2;
  while (ks < 16 && tiles * ks < 4096 && 2 * ks <= C) ks *= 2;
  int e = env_ksplit();
  if (e == 1 || e == 2 || e == 4 || e == 8 || e == 16)
    if ((C + e - 1) / e <= F::MAXC) ks = e;
  return ks;
}

template <int FMT, int NB>
int launch_xl(const void *packed, const float *x, float *y, int N, int K, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K);
  const size_t tiles = gq_tiles(N);
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const int ks = pick_ksplit<FMT>(tiles, C);
  const size_t lds = (size_t)ks * xl_layout(Fmt<FMT>::CK * ((C + ks - 1) / ks), NB).wave_bytes;
  const uint8_t *w = (const uint8_t *)packed;
#define GQ_LAUNCH_KS(KS)                                                                                  \
  hipLaunchKernelGGL((k_gemv_xl<FMT, NB, KS>), dim3((unsigned)tiles), dim3(64 * KS), lds, s, w, sc_off, x, y, \
                     N, K, C)
  switch (ks) {
  case 1: GQ_LAUNCH_KS(1); break;
  case 2: GQ_LAUNCH_KS(2); break;
  case 4: GQ_LAUNCH_KS(4); break;
  case 8: GQ_LAUNCH_KS(8); break;
  default: GQ_LAUNCH_KS(16); break;
  }
#undef GQ_LAUNCH_KS
  return gq_last_launch();
}

template <int FMT, int MT>
int launch_xg(const void *packed, const void *ws, float *y, int N, int K, int nb, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K);
  const int Kp = (int)gq_kpad(FMT, K);
  const size_t tiles = gq_tiles(N);
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const _Float16 *xq = (const _Float16 *)ws;
  const float *sf = (const float *)((const uint8_t *)ws + gq_xq_bytes(FMT, K, nb));
  const uint32_t *sh = (const uint32_t *)((const uint8_t *)ws + gq_xq_bytes(FMT, K, nb) + gq_sf_bytes(FMT, K, nb));
  const int ks = pick_ksplit<FMT>(tiles, C);
  const uint8_t *w = (const uint8_t *)packed;
#define GQ_LAUNCH_KS(KS)                                                                                     \
  hipLaunchKernelGGL((k_gemv_xg<FMT, MT, KS>), dim3((unsigned)tiles), dim3(64 * KS), 0, s, w, sc_off, xq, sf, sh, \
                     y, N, C, Kp, nb)
  switch (ks) {
  case 1: GQ_LAUNCH_KS(1); break;
  case 2: GQ_LAUNCH_KS(2); break;
  case 4: GQ_LAUNCH_KS(4); break;
  case 8: GQ_LAUNCH_KS(8); break;
  default: GQ_LAUNCH_KS(16); break;
  }
#undef GQ_LAUNCH_KS
  return gq_last_launch();
}

template <int FMT>
int launch_gemv(const void *packed, const float *x, const void *ws, float *y, int N, int K, int nb, hipStream_t s) {
  if (x) return nb == 1 ? launch_xl<FMT, 1>(packed, x, y, N, K, s) : launch_xl<FMT, 2>(packed, x, y, N, K, s);
  if (nb <= 8) return launch_xg<FMT, 1>(packed, ws, y, N, K, nb, s);
  return launch_xg<FMT, 2>(packed, ws, y, N, K, nb, s);
}

int dispatch(int fmt, const void *packed, const float *x, const void *ws, float *y, int N, int K, int nb,
             hipStream_t s) {
  switch (fmt) {
  case GQ_FMT_Q4_0: return launch_gemv<GQ_FMT_Q4_0>(packed, x, ws, y, N, K, nb, s);
  case GQ_FMT_Q8_0: return launch_gemv<GQ_FMT_Q8_0>(packed, x, ws, y, N, K, nb, s);
  default: return launch_gemv<GQ_FMT_Q4_K>(packed, x, ws, y, N, K, nb, s);
  }
}

}  // namespace

// batch sizes whose activations are staged in-kernel (no workspace)
static inline bool gq_gemv_fused(int batch) { return batch <= 2; }

extern "C" size_t gq_gemv_workspace_bytes(int fmt, size_t K, int batch) {
  if (!gq_fmt_valid(fmt) || batch < 1 || batch > GQ_MAX_BATCH || K > GQ_MAX_DIM) return 0;
  return gq_xq_bytes(fmt, K, batch) + gq_sf_bytes(fmt, K, batch) + gq_sq_bytes(fmt, K, batch);
}

extern "C" int gq_gemv_prep(int fmt, const float *x, size_t K, int batch, void *ws, size_t ws_bytes,
                            void *stream) {
  GQ_TRY(gq_check_shape(fmt, 0, K));
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(x && ws, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(ws_bytes >= gq_gemv_workspace_bytes(fmt, K, batch), GQ_ERR_WORKSPACE);
  if (K == 0) return GQ_OK;
  return gq_launch_prep_x(fmt, x, ws, batch, (int)K, (hipStream_t)stream);
}

extern "C" int gq_gemv_prepped(int fmt, const void *packed, const void *ws, float *y, size_t N, size_t K,
                               int batch, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(packed && ws && y, GQ_ERR_INVALID_ARGS);
  if (N == 0) return GQ_OK;
  if (K == 0) return gq_fill_zero(y, N * batch, (hipStream_t)stream);
  return dispatch(gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt, packed, nullptr, ws, y, (int)N, (int)K, batch,
                  (hipStream_t)stream);
}

extern "C" int gq_gemv(int fmt, const void *packed, const float *x, float *y, size_t N, size_t K, int batch,
                       void *ws, size_t ws_bytes, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(packed && x && y, GQ_ERR_INVALID_ARGS);
  if (N == 0) return GQ_OK;
  if (K == 0) return gq_fill_zero(y, N * batch, (hipStream_t)stream);
  if (gq_gemv_fused(batch))
    return dispatch(gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt, packed, x, nullptr, y, (int)N, (int)K, batch,
                    (hipStream_t)stream);
  size_t need = gq_gemv_workspace_bytes(fmt, K, batch);
  if (!ws) {
    GQ_TRY(gq_default_workspace(need, &ws));
    ws_bytes = need;
  }
  GQ_TRY(gq_gemv_prep(fmt, x, K, batch, ws, ws_bytes, stream));
  return gq_gemv_prepped(fmt, packed, ws, y, N, K, batch, stream);
}
