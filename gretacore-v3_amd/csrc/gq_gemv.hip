// gq_gemv.hip -- decode GEMV (batch 1..16) over T16-repacked GGUF weights.
//
// Replaces gemv_int8_wt_kernel / gemv_int4_wt_kernel
// (src/rt/backend/hip/kernels/gemm_kernels.hip:594-634, 763-817) for
// GGUF-native weights: y[b][n] = sum_k x[b][k] * W[n][k].
//
// Design (CDNA4, wave64):
//  * One workgroup per 16-row tile; its KSPLIT waves split the K axis and meet
//    in LDS at the end.  Each lane streams its tile's chunks with one dwordx4
//    load per chunk (1 KiB per wave, fully coalesced) and dequantizes in
//    registers into fp16 MFMA operands (exact small integers, no rounding).
//  * The dot products run on v_mfma_f32_16x16x32_f16 with A = activations
//    (rows = batch rows) and B = the weight tile (cols = 16 weight rows).  The
//    activation is split into fp16 hi + lo rows (x = hi + lo to ~2^-22), so the
//    fp16 operands lose no precision; hi and lo ride in spare MFMA rows.
//  * Per-block fp16 scales are applied in fp32 to each block's MFMA result
//    (Q4_0, Q8_0).  Q4_K folds the 6-bit sub-block scale into the operand
//    (sc*q <= 945 is exact in fp16), accumulates one super-block per MFMA
//    chain, and gets sum_j m_j * S_j (S_j = sub-block sums of x) from one extra
//    MFMA: y += d*D1 - dmin*D2.
#include "gq_internal.h"

namespace {

constexpr int kPF = 4;  // chunks whose loads are issued together per wave

template <int MT>
struct XRows {
  const _Float16 *p[MT];
  bool v[MT];
};

template <int MT>
GQ_DEV void load_xfrags(const XRows<MT> &xr, int k, gq_half8 (&a)[MT]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    gq_half8 z = {};
    a[mt] = xr.v[mt] ? *reinterpret_cast<const gq_half8 *>(xr.p[mt] + k) : z;
  }
}

template <int FMT, int MT, int KSPLIT>
__global__ void __launch_bounds__(64 * KSPLIT)
k_gemv_t16(const uint8_t *__restrict__ w, size_t sc_off, const _Float16 *__restrict__ xq,
           const uint32_t *__restrict__ sq, float *__restrict__ y, int N, int C, int Kp, int nb) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, r = lane & 15;
  const size_t t = blockIdx.x;
  const int c0 = (C * wave) / KSPLIT, c1 = (C * (wave + 1)) / KSPLIT;

  XRows<MT> xr;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    int row = 16 * mt + r;
    xr.v[mt] = row < 2 * nb;
    xr.p[mt] = xq + (size_t)(xr.v[mt] ? row : 0) * Kp;
  }
  gq_f4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = gq_f4{0.f, 0.f, 0.f, 0.f};
  const gq_f4 zero4 = {0.f, 0.f, 0.f, 0.f};

  if constexpr (FMT == GQ_FMT_Q4_0) {
    const uint8_t *qp = w + t * (size_t)C * 1024 + 16 * lane;
    const uint8_t *dp = w + sc_off + t * (size_t)C * 128 + 8 * r;
    for (int cb = c0; cb < c1; cb += kPF) {
      gq_u4 q[kPF];
      gq_u2 dd[kPF];
#pragma unroll
      for (int p = 0; p < kPF; ++p)
        if (cb + p < c1) {
          q[p] = gq_ld16(qp + (size_t)(cb + p) * 1024);
          dd[p] = gq_ld8(dp + (size_t)(cb + p) * 128);
        }
#pragma unroll
      for (int p = 0; p < kPF; ++p)
        if (cb + p < c1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            gq_half8 b;
            gq_q4word_to_h8<8>(q[p][j], b);
            float d = gq_scale_h2f((j & 1) ? (dd[p][j >> 1] >> 16) : dd[p][j >> 1]);
            gq_half8 a[MT];
            load_xfrags<MT>(xr, (cb + p) * 128 + 32 * j + 8 * g, a);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              gq_f4 D = gq_mfma16(a[mt], b, zero4);
              acc[mt] += d * D;
            }
          }
        }
    }
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    const uint8_t *qp = w + t * (size_t)C * 2048 + 16 * lane;
    const uint8_t *dp = w + sc_off + t * (size_t)C * 128 + 8 * r;
    for (int cb = c0; cb < c1; cb += kPF) {
      gq_u4 q0[kPF], q1[kPF];
      gq_u2 dd[kPF];
#pragma unroll
      for (int p = 0; p < kPF; ++p)
        if (cb + p < c1) {
          q0[p] = gq_ld16(qp + (size_t)(cb + p) * 2048);
          q1[p] = gq_ld16(qp + (size_t)(cb + p) * 2048 + 1024);
          dd[p] = gq_ld8(dp + (size_t)(cb + p) * 128);
        }
#pragma unroll
      for (int p = 0; p < kPF; ++p)
        if (cb + p < c1) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const gq_u4 &qq = (j < 2) ? q0[p] : q1[p];
            gq_half8 b;
            gq_i8x8_to_h8(qq[2 * (j & 1)], qq[2 * (j & 1) + 1], b);
            float d = gq_scale_h2f((j & 1) ? (dd[p][j >> 1] >> 16) : dd[p][j >> 1]);
            gq_half8 a[MT];
            load_xfrags<MT>(xr, (cb + p) * 128 + 32 * j + 8 * g, a);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              gq_f4 D = gq_mfma16(a[mt], b, zero4);
              acc[mt] += d * D;
            }
          }
        }
    }
  } else {  // Q4_K (both GGUF variants share the repacked form)
    const uint8_t *qp = w + t * (size_t)C * 2048 + 16 * lane;
    const uint8_t *mp = w + sc_off + t * (size_t)C * 256 + 16 * r;
    const int nsub = Kp / 32;
    // sub-block sums of x: only the hi row (even xrow) of each batch row
    const uint32_t *sqr[MT];
    bool sv[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      int row = 16 * mt + r;
      sv[mt] = (row < 2 * nb) && !(row & 1);
      sqr[mt] = sq + (size_t)(sv[mt] ? (row >> 1) : 0) * nsub;
    }
    for (int cb = c0; cb < c1; cb += 2) {
      gq_u4 qa[2], qb[2], meta[2];
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (cb + p < c1) {
          qa[p] = gq_ld16(qp + (size_t)(cb + p) * 2048);
          qb[p] = gq_ld16(qp + (size_t)(cb + p) * 2048 + 1024);
          meta[p] = gq_ld16(mp + (size_t)(cb + p) * 256);
        }
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (cb + p < c1) {
          const int s = cb + p;
          float d = gq_scale_h2f(meta[p][0] & 0xFFFFu), dmin = gq_scale_h2f(meta[p][0] >> 16);
          uint32_t sc0, m0, sc1, m1;
          gq_q4k_codes(meta[p][1], meta[p][2], meta[p][3], g, sc0, m0, sc1, m1);
          _Float16 hs0 = (_Float16)(float)sc0, hs1 = (_Float16)(float)sc1;
          _Float16 hn0 = (_Float16)(-1024.0f * (float)sc0), hn1 = (_Float16)(-1024.0f * (float)sc1);
          gq_f4 D1[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) D1[mt] = zero4;
#pragma unroll
          for (int tt = 0; tt < 8; ++tt) {
            const int h = tt >> 2;
            uint32_t word = h ? qb[p][tt & 3] : qa[p][tt & 3];
            gq_half2 sc2 = h ? gq_half2{hs1, hs1} : gq_half2{hs0, hs0};
            gq_half2 ns2 = h ? gq_half2{hn1, hn1} : gq_half2{hn0, hn0};
            gq_half8 b;
            gq_q4word_scaled_h8(word, sc2, ns2, b);
            gq_half8 a[MT];
            load_xfrags<MT>(xr, s * 256 + 32 * (2 * g + h) + 8 * (tt & 3), a);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) D1[mt] = gq_mfma16(a[mt], b, D1[mt]);
          }
          // min term: sum over sub-blocks of m_j * S_j via one MFMA
          gq_half8 bm = {};
          bm[0] = (_Float16)(float)m0;
          bm[1] = (_Float16)(float)m1;
          bm[2] = bm[0];
          bm[3] = bm[1];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            gq_half8 am = {};
            if (sv[mt]) {
              gq_u2 sp = gq_ld8(sqr[mt] + (size_t)s * 8 + 2 * g);  // (Sh,Sl) of 2g, 2g+1
              gq_half2 s0 = gq_bits_h2(sp[0]), s1 = gq_bits_h2(sp[1]);
              am[0] = s0[0];
              am[1] = s1[0];
              am[2] = s0[1];
              am[3] = s1[1];
            }
            gq_f4 D2 = gq_mfma16(am, bm, zero4);
            acc[mt] += d * D1[mt] - dmin * D2;
          }
          (void)nsub;
        }
    }
  }

  // combine the KSPLIT partial sums and write y
  if constexpr (KSPLIT > 1) {
    __shared__ float red[KSPLIT][MT * 4][64];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[wave][mt * 4 + v][lane] = acc[mt][v];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < KSPLIT; ++q) s += red[q][mt * 4 + v][lane];
        acc[mt][v] = s;
      }
  }
  const size_t row = t * 16 + r;
  if (row >= (size_t)N) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      int b = 8 * mt + 2 * g + u;
      if (b < nb) y[(size_t)b * N + row] = acc[mt][2 * u] + acc[mt][2 * u + 1];
    }
}

template <int FMT, int MT>
int launch_gemv_fmt(const void *packed, const void *ws, float *y, int N, int K, int nb, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K);
  const int Kp = (int)gq_kpad(FMT, K);
  const size_t tiles = gq_tiles(N);
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const _Float16 *xq = (const _Float16 *)ws;
  const uint32_t *sq = gq_fmt_is_q4k(FMT) ? (const uint32_t *)((const uint8_t *)ws + gq_xq_bytes(FMT, K, nb))
                                          : nullptr;
  // enough waves to cover the chip: ~2048+ waves, at least one chunk each
  int ks = 1;
  while (ks < 16 && tiles * ks < 2048 && 2 * ks <= C) ks *= 2;
  const uint8_t *w = (const uint8_t *)packed;
#define GQ_LAUNCH_KS(KS)                                                                              \
  hipLaunchKernelGGL((k_gemv_t16<FMT, MT, KS>), dim3((unsigned)tiles), dim3(64 * KS), 0, s, w, sc_off, \
                     xq, sq, y, N, C, Kp, nb)
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
int launch_gemv(const void *packed, const void *ws, float *y, int N, int K, int nb, hipStream_t s) {
  if (nb <= 8) return launch_gemv_fmt<FMT, 1>(packed, ws, y, N, K, nb, s);
  return launch_gemv_fmt<FMT, 2>(packed, ws, y, N, K, nb, s);
}

}  // namespace

extern "C" size_t gq_gemv_workspace_bytes(int fmt, size_t K, int batch) {
  if (!gq_fmt_valid(fmt) || batch < 1 || batch > GQ_MAX_BATCH || K > GQ_MAX_DIM) return 0;
  return gq_xq_bytes(fmt, K, batch) + gq_sq_bytes(fmt, K, batch);
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
  if (K == 0) return hipMemsetAsync(y, 0, N * batch * sizeof(float), (hipStream_t)stream) == hipSuccess
                         ? GQ_OK
                         : GQ_ERR_HIP;
  hipStream_t s = (hipStream_t)stream;
  switch (fmt) {
  case GQ_FMT_Q4_0: return launch_gemv<GQ_FMT_Q4_0>(packed, ws, y, (int)N, (int)K, batch, s);
  case GQ_FMT_Q8_0: return launch_gemv<GQ_FMT_Q8_0>(packed, ws, y, (int)N, (int)K, batch, s);
  default: return launch_gemv<GQ_FMT_Q4_K>(packed, ws, y, (int)N, (int)K, batch, s);
  }
}

extern "C" int gq_gemv(int fmt, const void *packed, const float *x, float *y, size_t N, size_t K, int batch,
                       void *ws, size_t ws_bytes, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(packed && x && y, GQ_ERR_INVALID_ARGS);
  if (N == 0) return GQ_OK;
  size_t need = gq_gemv_workspace_bytes(fmt, K, batch);
  if (!ws) {
    GQ_TRY(gq_default_workspace(need, &ws));
    ws_bytes = need;
  }
  GQ_TRY(gq_gemv_prep(fmt, x, K, batch, ws, ws_bytes, stream));
  return gq_gemv_prepped(fmt, packed, ws, y, N, K, batch, stream);
}
