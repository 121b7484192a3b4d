// gq_gemv_h.hip -- decode GEMV for batch 5..16 on the fp16 matrix cores.
//
// The int8 GEMV (gq_gemv.hip) applies the weight and activation scales per
// (row, 32-block, batch row); with a wide batch that VALU work outgrows the
// weight stream.  Here the weights are dequantized once per weight with the
// block scale folded in -- (q - 8) * d (Q4_0), q * d (Q8_0),
// d * sc * q - dmin * m (Q4_K), each rounded once to fp16 as the reference's
// MFMA path does (__float2half(w * s), gemm_kernels.hip:820-908) -- and fed to
// v_mfma_f32_16x16x32_f16 as the B operand, whose 16 columns are the 16 rows of
// a T16 row tile; the A operand's 16 rows are the batch rows of x, rounded to
// fp16 (rows >= batch are zero).  The MFMA accumulates across blocks in fp32,
// so no per-block work remains.
//
// A wave takes its K slice in groups of NCK chunks: it issues every weight
// load of the group, converts the activations of its MFMA k-positions to fp16
// registers (shared by the R row tiles of the workgroup), and consumes the
// chunks as they arrive.  The KSPLIT waves' partial sums are reduced in LDS.
#include <stdlib.h>

#include "gq_internal.h"

namespace {

template <int FMT>
struct HFmt;
template <>
struct HFmt<GQ_FMT_Q4_0> {
  static constexpr int CK = 128, QB = 1024, SB = 128, STEPS = 2, NCK = 4;
};
template <>
struct HFmt<GQ_FMT_Q8_0> {
  static constexpr int CK = 128, QB = 2048, SB = 128, STEPS = 2, NCK = 4;
};
template <>
struct HFmt<GQ_FMT_Q4_K> {
  static constexpr int CK = 256, QB = 2048, SB = 256, STEPS = 4, NCK = 2;
};

template <int FMT>
struct HChunk;
template <>
struct HChunk<GQ_FMT_Q4_0> {
  gq_u4 q;  // steps 0, 1: 8-byte code groups
  uint32_t d;
};
template <>
struct HChunk<GQ_FMT_Q8_0> {
  gq_u4 q0, q1;
  uint32_t d;
};
template <>
struct HChunk<GQ_FMT_Q4_K> {
  gq_u4 qa, qb;
  gq_u4 meta;
};

template <int FMT>
GQ_DEV void load_hchunk(const uint8_t *qp, const uint8_t *sp, uint32_t qo, uint32_t so, HChunk<FMT> &ch) {
  if constexpr (FMT == GQ_FMT_Q4_0) {
    ch.q = gq_ld16_nt(qp + qo);
    ch.d = gq_ld4_nt(sp + so);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    ch.q0 = gq_ld16_nt(qp + qo);
    ch.q1 = gq_ld16_nt(qp + 1024 + qo);
    ch.d = gq_ld4_nt(sp + so);
  } else {
    ch.qa = gq_ld16_nt(qp + qo);
    ch.qb = gq_ld16_nt(qp + 1024 + qo);
    ch.meta = gq_ld16_nt(sp + so);
  }
}

// 4 byte values u (0..255) -> 2 fp16 pairs holding (1024 + u)
GQ_DEV void magic4(uint32_t u, gq_half2 &lo, gq_half2 &hi) {
  lo = gq_bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
  hi = gq_bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
}

GQ_DEV gq_half2 splat_h(uint32_t b16) { return gq_bits_h2((b16 & 0xFFFFu) * 0x10001u); }

// The 16 weights a lane holds for MFMA step m -> fp16 B fragments (slots
// 0..7, 8..15).  j is the lane's 32-block within the chunk.
template <int FMT>
GQ_DEV void dequant_step(const HChunk<FMT> &c, int m, int j, gq_half8 &o0, gq_half8 &o1) {
  uint32_t regs[4];
  gq_half2 off, sc2, nsc2, d2, mn2;
  if constexpr (FMT == GQ_FMT_Q4_0) {
    const uint32_t w0 = c.q[2 * m], w1 = c.q[2 * m + 1];
    regs[0] = w0 & 0x0F0F0F0Fu;
    regs[1] = (w0 >> 4) & 0x0F0F0F0Fu;
    regs[2] = w1 & 0x0F0F0F0Fu;
    regs[3] = (w1 >> 4) & 0x0F0F0F0Fu;
    off = gq_half2{(_Float16)-1032.0f, (_Float16)-1032.0f};
    d2 = splat_h(m ? (c.d >> 16) : c.d);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    const gq_u4 &q = m ? c.q1 : c.q0;
#pragma unroll
    for (int i = 0; i < 4; ++i) regs[i] = q[i] ^ 0x80808080u;
    off = gq_half2{(_Float16)-1152.0f, (_Float16)-1152.0f};
    d2 = splat_h(m ? (c.d >> 16) : c.d);
  } else {
    const gq_u4 &q = (m < 2) ? c.qa : c.qb;
    const uint32_t w0 = q[2 * (m & 1)], w1 = q[2 * (m & 1) + 1];
    regs[0] = w0 & 0x0F0F0F0Fu;
    regs[1] = (w0 >> 4) & 0x0F0F0F0Fu;
    regs[2] = w1 & 0x0F0F0F0Fu;
    regs[3] = (w1 >> 4) & 0x0F0F0F0Fu;
    const uint32_t mv[4] = {c.meta[0], c.meta[1], c.meta[2], c.meta[3]};
    uint32_t sc, mn;
    gq_q4k_meta_codes(mv, j, &sc, &mn);
    const float d = gq_h2f(mv[0] & 0xFFFFu), dmin = gq_h2f(mv[0] >> 16);
    const _Float16 hd = (_Float16)d;  // exact: d came from fp16 (NaN aside)
    const _Float16 hsc = (_Float16)(float)sc, hnsc = (_Float16)(-1024.0f * (float)sc);
    const _Float16 hmin = (_Float16)(-(dmin * (float)mn));
    sc2 = gq_half2{hsc, hsc};
    nsc2 = gq_half2{hnsc, hnsc};
    d2 = gq_half2{hd, hd};
    mn2 = gq_half2{hmin, hmin};
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    gq_half2 lo, hi;
    magic4(regs[q], lo, hi);
    if constexpr (FMT == GQ_FMT_Q4_K) {
      // (1024 + c) * sc - 1024 sc = c * sc exactly, then one rounding of
      // c * sc * d - dmin * m
      lo = __builtin_elementwise_fma(__builtin_elementwise_fma(lo, sc2, nsc2), d2, mn2);
      hi = __builtin_elementwise_fma(__builtin_elementwise_fma(hi, sc2, nsc2), d2, mn2);
    } else {
      lo = (lo + off) * d2;  // exact (q - bias), one rounding of the product
      hi = (hi + off) * d2;
    }
    gq_half8 &o = (q < 2) ? o0 : o1;
    const int b = 4 * (q & 1);
    o[b] = lo[0];
    o[b + 1] = lo[1];
    o[b + 2] = hi[0];
    o[b + 3] = hi[1];
  }
}

GQ_DEV gq_f4 mfma16h(const gq_half8 &a, const gq_half8 &b, const gq_f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 16 consecutive fp32 -> 2 fp16 A fragments (zeros where `in` is false)
GQ_DEV void x16_to_frags(const float *p, bool in, gq_half8 &f0, gq_half8 &f1) {
  gq_f4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = in ? *reinterpret_cast<const gq_f4 *>(p + 4 * i) : gq_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    f0[i] = (_Float16)v[i >> 2][i & 3];
    f1[i] = (_Float16)v[2 + (i >> 2)][i & 3];
  }
}

template <int FMT, int R, int KSPLIT>
__global__ void __launch_bounds__(64 * KSPLIT)
k_gemv_h(const uint8_t *__restrict__ w, size_t sc_off, const float *__restrict__ x, float *__restrict__ y, int N,
         int K, int C, int nb) {
  using F = HFmt<FMT>;
  constexpr int NCK = F::NCK;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const size_t tile0 = (size_t)blockIdx.x * R;
  const int ntiles = (int)gq_tiles(N);
  const int c0 = (C * wave) / KSPLIT, c1 = (C * (wave + 1)) / KSPLIT;
  const int nck = c1 - c0;  // chunks of this wave, consumed in groups of NCK

  const uint32_t qlane = 16u * (uint32_t)lane;
  const uint32_t slane = (FMT == GQ_FMT_Q4_K) ? 16u * (uint32_t)r : 8u * (uint32_t)r + 4u * (uint32_t)(g >> 1);
  size_t tbase[R];
#pragma unroll
  for (int rt = 0; rt < R; ++rt) {
    const size_t t = (tile0 + rt < (size_t)ntiles) ? tile0 + rt : (size_t)ntiles - 1;
    tbase[rt] = t * (size_t)C;
  }
  const bool brow = r < nb;
  const float *xr = x + (size_t)(brow ? r : 0) * K;

  gq_f4 acc[R];
#pragma unroll
  for (int rt = 0; rt < R; ++rt) acc[rt] = gq_f4{0.f, 0.f, 0.f, 0.f};

  for (int gb = 0; gb == 0 || gb < nck; gb += NCK) {
    const int ng = nck - gb < NCK ? nck - gb : NCK;  // chunks in this group (may be 0)
    // ---- weight loads of the group (clamped, unconditional): surplus loads
    // re-read the group's last chunk (chunk c0 when the wave has none: c0 < C
    // always holds), never outside the tensor
    HChunk<FMT> ch[R][NCK];
#pragma unroll
    for (int i = 0; i < NCK; ++i) {
      const int ci = c0 + gb + (i < ng ? i : (ng > 0 ? ng - 1 : 0));
#pragma unroll
      for (int rt = 0; rt < R; ++rt)
        load_hchunk<FMT>(w + (tbase[rt] + ci) * F::QB, w + sc_off + (tbase[rt] + ci) * F::SB, qlane, slane,
                         ch[rt][i]);
    }
    // ---- activations: lane (g, row b = r) keeps x[b][k] for the k of its
    // MFMA slots: per step m, 16 consecutive k at 64 m + 32 (g >> 1) + 16 (g & 1)
    gq_half8 xa[NCK][F::STEPS][2];
#pragma unroll
    for (int i = 0; i < NCK; ++i) {
      const int ci = c0 + gb + (i < ng ? i : (ng > 0 ? ng - 1 : 0));
#pragma unroll
      for (int m = 0; m < F::STEPS; ++m) {
        const int k = ci * F::CK + 64 * m + 32 * (g >> 1) + 16 * (g & 1);
        const bool in = brow && k < K;  // K % 32 == 0: a 16-run is wholly in or out
        x16_to_frags(xr + (in ? k : 0), in, xa[i][m][0], xa[i][m][1]);
      }
    }
    // ---- consume
#pragma unroll
    for (int i = 0; i < NCK; ++i) {
      if (i < ng)
#pragma unroll
        for (int m = 0; m < F::STEPS; ++m)
#pragma unroll
          for (int rt = 0; rt < R; ++rt) {
            gq_half8 b0, b1;
            dequant_step<FMT>(ch[rt][i], m, 2 * m + (g >> 1), b0, b1);
            acc[rt] = mfma16h(xa[i][m][0], b0, acc[rt]);
            acc[rt] = mfma16h(xa[i][m][1], b1, acc[rt]);
          }
    }
  }

  // ---- reduce over the KSPLIT waves; D lane (g, r): batch rows 4g..4g+3, column r
  if constexpr (KSPLIT > 1) {
    __shared__ gq_f4 red[KSPLIT][R][64];
#pragma unroll
    for (int rt = 0; rt < R; ++rt) red[wave][rt][lane] = acc[rt];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int rt = 0; rt < R; ++rt) {
      gq_f4 s = red[0][rt][lane];
#pragma unroll
      for (int q = 1; q < KSPLIT; ++q) {
        const gq_f4 v = red[q][rt][lane];
        s[0] += v[0];
        s[1] += v[1];
        s[2] += v[2];
        s[3] += v[3];
      }
      acc[rt] = s;
    }
  }
#pragma unroll
  for (int rt = 0; rt < R; ++rt) {
    const size_t row = (tile0 + rt) * 16 + r;
    if (row >= (size_t)N) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int b = 4 * g + v;
      if (b < nb) y[(size_t)b * N + row] = acc[rt][v];
    }
  }
}

int env_int(const char *name) {
  const char *e = getenv(name);
  return e ? atoi(e) : 0;
}

}  // namespace

// Launch plan of the fp16 batch GEMV: R (1 or 2) row tiles per workgroup and
// KSPLIT (1..8) waves.  chunks_per_wave may exceed NCK: the kernel then
// consumes them in groups.
int gq_gemv_h_plan(int fmt, size_t N, size_t K, int *R_out, int *ks_out, int *cpw_out) {
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt;
  const int nck = f == GQ_FMT_Q4_K ? HFmt<GQ_FMT_Q4_K>::NCK : f == GQ_FMT_Q8_0 ? HFmt<GQ_FMT_Q8_0>::NCK
                                                                                : HFmt<GQ_FMT_Q4_0>::NCK;
  const int C = (int)gq_chunks(f, K);
  const size_t tiles = gq_tiles(N);
  // two row tiles per workgroup while that still leaves >= 256 workgroups
  int R = (tiles + 1) / 2 >= 256 ? 2 : 1;
  const int er = env_int("GQ_GEMV_H_R");
  if (er == 1 || er == 2) R = er;
  // fewest waves (at most 8: a wave keeps ~200 VGPRs) such that each holds at
  // most NCK chunks; past that a wave consumes its chunks in groups of NCK
  int ks = 1;
  while (ks < 8 && (C + ks - 1) / ks > nck) ks *= 2;
  const int e = env_int("GQ_GEMV_H_KSPLIT");
  if (e == 1 || e == 2 || e == 4 || e == 8) ks = e;
  *R_out = R;
  *ks_out = ks;
  *cpw_out = (C + ks - 1) / ks;
  return GQ_OK;
}

namespace {
template <int FMT, int R>
int launch_h_r(const void *packed, const float *x, float *y, int N, int K, int nb, int ks, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K);
  const size_t wgs = (gq_tiles(N) + R - 1) / R;
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const uint8_t *w = (const uint8_t *)packed;
#define GQ_LAUNCH_H(KS)                                                                                            \
  hipLaunchKernelGGL((k_gemv_h<FMT, R, KS>), dim3((unsigned)wgs), dim3(64 * KS), 0, s, w, sc_off, x, y, N, K, C, \
                     nb)
  switch (ks) {
  case 1: GQ_LAUNCH_H(1); break;
  case 2: GQ_LAUNCH_H(2); break;
  case 4: GQ_LAUNCH_H(4); break;
  default: GQ_LAUNCH_H(8); break;
  }
#undef GQ_LAUNCH_H
  return gq_last_launch();
}

template <int FMT>
int launch_h(const void *packed, const float *x, float *y, int N, int K, int nb, hipStream_t s) {
  int R, ks, cpw;
  GQ_TRY(gq_gemv_h_plan(FMT, N, K, &R, &ks, &cpw));
  if (R == 2) return launch_h_r<FMT, 2>(packed, x, y, N, K, nb, ks, s);
  return launch_h_r<FMT, 1>(packed, x, y, N, K, nb, ks, s);
}
}  // namespace

int gq_launch_gemv_h(int fmt, const void *packed, const float *x, float *y, int N, int K, int nb, hipStream_t s) {
  switch (gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt) {
  case GQ_FMT_Q4_0: return launch_h<GQ_FMT_Q4_0>(packed, x, y, N, K, nb, s);
  case GQ_FMT_Q8_0: return launch_h<GQ_FMT_Q8_0>(packed, x, y, N, K, nb, s);
  default: return launch_h<GQ_FMT_Q4_K>(packed, x, y, N, K, nb, s);
  }
}
