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
// The activations are staged once per workgroup, window by window, as fp16 A
// fragments in LDS and shared by the workgroup's row tiles (k_gemv_h below).
#include <stdlib.h>

#include <type_traits>

#include "gq_internal.h"

namespace {

template <int FMT>
struct HFmt;
template <>
struct HFmt<GQ_FMT_Q4_0> {
  static constexpr int CK = 128, QB = 1024, SB = 128, STEPS = 2;
};
template <>
struct HFmt<GQ_FMT_Q8_0> {
  static constexpr int CK = 128, QB = 2048, SB = 128, STEPS = 2;
};
template <>
struct HFmt<GQ_FMT_Q4_K> {
  static constexpr int CK = 256, QB = 2048, SB = 256, STEPS = 4;
};
template <>
struct HFmt<GQ_FMT_Q6_K> {
  static constexpr int CK = 256, QB = 3072, SB = 288, STEPS = 4;
};

// fp16 weights, row-major N x K (the reference's FP16 route, no T16 layout):
// a "chunk" is 128 k of one row tile, read straight from the 16 rows
template <>
struct HFmt<GQ_FMT_F16> {
  static constexpr int CK = 128, STEPS = 2;
  [[maybe_unused]] static constexpr int QB = 0, SB = 0;  // (no T16 records or scale plane)
};

template <int FMT>
struct HChunk;
template <>
struct HChunk<GQ_FMT_F16> {
  gq_u4 q[4];  // step m: q[2m], q[2m + 1] = the lane's 16 fp16 weights (halves 0, 1)
};
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
template <>
struct HChunk<GQ_FMT_Q6_K> {
  gq_u4 qa, qb;  // low-nibble code groups, steps 0,1 and 2,3
  gq_u4 hi;      // high 2-bit fields, one word per step
  gq_u4 sc;      // the row's 16 int8 scales
  uint32_t d;    // the row's fp16 d (low half)
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
  } else if constexpr (FMT == GQ_FMT_Q4_K) {
    ch.qa = gq_ld16_nt(qp + qo);
    ch.qb = gq_ld16_nt(qp + 1024 + qo);
    ch.meta = gq_ld16_nt(sp + so);
  } else {  // Q6_K: so = 16 r
    ch.qa = gq_ld16_nt(qp + qo);
    ch.qb = gq_ld16_nt(qp + 1024 + qo);
    ch.hi = gq_ld16_nt(qp + 2048 + qo);
    ch.sc = gq_ld16_nt(sp + so);
    ch.d = gq_ld4_nt(sp + 256 + 4 * (so >> 5)) >> (16 * ((so >> 4) & 1));
  }
}

// Where a wave's chunks of one row tile come from: T16 records (chunk ci of
// the tile at q + ci * QB, its scales at s + ci * SB, this lane's offsets
// qo / so), or, for row-major fp16 weights, this lane's row (row tile rows
// past N read row N - 1, never stored) with the lane's k offset qo (bytes)
// and the row length K.
template <int FMT>
struct HSrc {
  const uint8_t *q, *s;
  uint32_t qo, so;
  int K;
};
template <int FMT>
GQ_DEV HSrc<FMT> hsrc(const uint8_t *w, size_t sc_off, size_t tile, int C, int N, int K, int lane) {
  const int g = lane >> 4, r = lane & 15;
  if constexpr (FMT == GQ_FMT_F16) {
    size_t n = tile * 16 + (size_t)r;
    n = n < (size_t)N ? n : (size_t)N - 1;
    return HSrc<FMT>{w + n * (size_t)K * 2, nullptr, 32u * (uint32_t)g, 0u, K};
  } else {
    using F = HFmt<FMT>;
    const uint32_t slane = (FMT == GQ_FMT_Q4_K || FMT == GQ_FMT_Q6_K) ? 16u * (uint32_t)r
                                                                      : 8u * (uint32_t)r + 4u * (uint32_t)(g >> 1);
    return HSrc<FMT>{w + tile * (size_t)C * F::QB, w + sc_off + tile * (size_t)C * F::SB, 16u * (uint32_t)lane,
                     slane, K};
  }
}

template <int FMT>
GQ_DEV void load_src(const HSrc<FMT> &src, int ci, HChunk<FMT> &ch) {
  if constexpr (FMT == GQ_FMT_F16) {
    // step m: k = 128 ci + 64 m + 16 g .. + 15 (K % 32 == 0: wholly in or out
    // of the row); a run past K reads the row's start and is zeroed
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t kb = 2u * (uint32_t)(128 * ci + 64 * m) + src.qo;  // byte offset in the row
      const bool in = kb < 2u * (uint32_t)src.K;
      const uint8_t *p = src.q + (in ? kb : 0u);
      gq_u4 a = gq_ld16_nt(p), b = gq_ld16_nt(p + 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[e] = in ? a[e] : 0u;
        b[e] = in ? b[e] : 0u;
      }
      ch.q[2 * m] = a;
      ch.q[2 * m + 1] = b;
    }
  } else {
    using F = HFmt<FMT>;
    load_hchunk<FMT>(src.q + (size_t)ci * F::QB, src.s + (size_t)ci * F::SB, src.qo, src.so, ch);
  }
}

// 4 byte values u (0..255) -> 2 fp16 pairs holding (1024 + u)
GQ_DEV void magic4(uint32_t u, gq_half2 &lo, gq_half2 &hi) {
  lo = gq_bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
  hi = gq_bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
}

GQ_DEV gq_half2 splat_h(uint32_t b16) { return gq_bits_h2((b16 & 0xFFFFu) * 0x10001u); }

// B fragment element e of a 4-bit format holds slot kQ4Perm[e]; elements with
// kQ4Div16 set are 16 x the weight
constexpr int kQ4Perm[8] = {0, 2, 4, 6, 1, 3, 5, 7};
constexpr bool kQ4Div16[8] = {false, false, true, true, false, false, true, true};
template <int FMT>
constexpr bool kNibOrder = FMT == GQ_FMT_Q4_0 || FMT == GQ_FMT_Q4_K;

GQ_DEV _Float16 bits_h(uint32_t b16) { return __builtin_bit_cast(_Float16, (uint16_t)(b16 & 0xFFFFu)); }

// The 16 weights a lane holds for MFMA step m -> fp16 B fragments (slots
// 0..7, 8..15; for the 4-bit formats in gq_nib_halves order).  g is the lane's
// 16-lane group: its 16 weights are half g & 1 of 32-block 2 m + (g >> 1) of
// the chunk (Q6_K: 16-element scale group 4 m + g).
template <int FMT>
GQ_DEV void dequant_step(const HChunk<FMT> &c, int m, int g, uint32_t mg, gq_half8 &o0, gq_half8 &o1) {
  if constexpr (FMT == GQ_FMT_F16) {
    o0 = __builtin_bit_cast(gq_half8, c.q[2 * m]);
    o1 = __builtin_bit_cast(gq_half8, c.q[2 * m + 1]);
    return;
  } else if constexpr (FMT == GQ_FMT_Q4_0 || FMT == GQ_FMT_Q4_K) {
    uint32_t w0, w1;
    gq_half2 a1, b1, a16, b16;  // (h * a + b) per pair; then * d2 + m2 (Q4_K)
    gq_half2 d2, m1, m16;
    if constexpr (FMT == GQ_FMT_Q4_0) {
      w0 = c.q[2 * m];
      w1 = c.q[2 * m + 1];
      // (q - 8) * d: the subtraction is exact, the product rounds once (and
      // 16 (q - 8) * d is 16 x that rounding)
      const _Float16 d = bits_h(m ? (c.d >> 16) : c.d);
      a1 = gq_half2{(_Float16)1.0f, (_Float16)1.0f};
      b1 = gq_half2{(_Float16)-1032.0f, (_Float16)-1032.0f};
      a16 = a1;
      b16 = gq_half2{(_Float16)-1152.0f, (_Float16)-1152.0f};
      d2 = gq_half2{d, d};
    } else {
      const gq_u4 &q = (m < 2) ? c.qa : c.qb;
      w0 = q[2 * (m & 1)];
      w1 = q[2 * (m & 1) + 1];
      // The lane's sub-blocks of steps 0..3 are 2 m + h (h = g >> 1): their
      // 6-bit scales are the low bits of the 4 bytes of meta word 1 + h, the
      // mins' low 2 bits the top bits of those bytes and their high 4 bits
      // nibble h of the bytes of meta word 3.  All four steps' factors are
      // decoded packed, two per instruction (the same values for every step
      // of a chunk, so the unrolled steps share them).
      const uint32_t h = (uint32_t)(g >> 1);
      const uint32_t wh = h ? c.meta[2] : c.meta[1];
      const uint32_t scb = wh & 0x3F3F3F3Fu;
      const uint32_t mnb = ((wh >> 6) & 0x03030303u) | (((c.meta[3] >> (4u * h)) & 0x0F0F0F0Fu) << 2);
      gq_half2 s01, s23, n01, n23;
      magic4(scb, s01, s23);
      magic4(mnb, n01, n23);
      const gq_half2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
      s01 = s01 + k1024;  // sc, exact
      s23 = s23 + k1024;
      n01 = n01 + k1024;  // m, exact
      n23 = n23 + k1024;
      // -(dmin m): the exact product rounded once, as (half)(-(float)dmin * m)
      const _Float16 ndmin = -bits_h(c.meta[0] >> 16);
      const gq_half2 nd2 = {ndmin, ndmin};
      const gq_half2 hm01 = n01 * nd2, hm23 = n23 * nd2;
      const gq_half2 k16 = {(_Float16)16.0f, (_Float16)16.0f};
      // (1024 + q) * sc - 1024 sc = q * sc exactly (<= 945; 16 q sc <= 15120,
      // a multiple of 16: exact too), then one rounding of q sc d - dmin m;
      // -1024 sc and 16 (-dmin m) are exact
      const gq_half2 sp = m < 2 ? s01 : s23, mp = m < 2 ? hm01 : hm23;
      const gq_half2 np = sp * k1024, mp16 = mp * k16;
      if (m & 1) {
        a1 = __builtin_shufflevector(sp, sp, 1, 1);
        b1 = __builtin_shufflevector(np, np, 1, 1);
        m1 = __builtin_shufflevector(mp, mp, 1, 1);
        m16 = __builtin_shufflevector(mp16, mp16, 1, 1);
      } else {
        a1 = __builtin_shufflevector(sp, sp, 0, 0);
        b1 = __builtin_shufflevector(np, np, 0, 0);
        m1 = __builtin_shufflevector(mp, mp, 0, 0);
        m16 = __builtin_shufflevector(mp16, mp16, 0, 0);
      }
      a16 = a1;
      b16 = b1;
      const _Float16 d = bits_h(c.meta[0]);
      d2 = gq_half2{d, d};
    }
#pragma unroll
    for (int hw = 0; hw < 2; ++hw) {
      gq_half2 p[4];
      gq_nib_halves(hw ? w1 : w0, mg, p);
      gq_half8 &o = hw ? o1 : o0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool x16 = q & 1;
        gq_half2 t;
        if constexpr (FMT == GQ_FMT_Q4_0) {
          t = (p[q] + (x16 ? b16 : b1)) * d2;
        } else {
          t = __builtin_elementwise_fma(__builtin_elementwise_fma(p[q], x16 ? a16 : a1, x16 ? b16 : b1), d2,
                                        x16 ? m16 : m1);
        }
        o[2 * q] = t[0];
        o[2 * q + 1] = t[1];
      }
    }
    return;
  } else {
  const int j = 2 * m + (g >> 1);
  (void)j;
  uint32_t regs[4];
  gq_half2 off, d2;
  if constexpr (FMT == GQ_FMT_Q6_K) {
    const gq_u4 &q = (m < 2) ? c.qa : c.qb;
    const uint32_t w0 = q[2 * (m & 1)], w1 = q[2 * (m & 1) + 1], hw = c.hi[m];
    regs[0] = w0 & 0x0F0F0F0Fu;
    regs[1] = (w0 >> 4) & 0x0F0F0F0Fu;
    regs[2] = w1 & 0x0F0F0F0Fu;
    regs[3] = (w1 >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int i = 0; i < 4; ++i) regs[i] |= ((hw >> (2 * i)) & 0x03030303u) << 4;  // codes 0..63
    // (c - 32) * (d * scale): the scale product rounded to fp16, then one
    // rounding of the exact (c - 32) * that
    const float sc = (float)(int8_t)((c.sc[m] >> (8 * g)) & 0xFFu);
    const _Float16 hs = (_Float16)((float)bits_h(c.d) * sc);
    off = gq_half2{(_Float16)-1056.0f, (_Float16)-1056.0f};
    d2 = gq_half2{hs, hs};
  } else {  // Q8_0
    const gq_u4 &q = m ? c.q1 : c.q0;
#pragma unroll
    for (int i = 0; i < 4; ++i) regs[i] = q[i] ^ 0x80808080u;
    off = gq_half2{(_Float16)-1152.0f, (_Float16)-1152.0f};
    d2 = splat_h(m ? (c.d >> 16) : c.d);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    gq_half2 lo, hi;
    magic4(regs[q], lo, hi);
    lo = (lo + off) * d2;  // exact (q - bias), one rounding of the product
    hi = (hi + off) * d2;
    gq_half8 &o = (q < 2) ? o0 : o1;
    const int b = 4 * (q & 1);
    o[b] = lo[0];
    o[b + 1] = lo[1];
    o[b + 2] = hi[0];
    o[b + 3] = hi[1];
  }
  }
}

GQ_DEV gq_f4 mfma16h(const gq_half8 &a, const gq_half8 &b, const gq_f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Largest (unsigned) value over each 32-lane half of the wave, every lane receiving its
// half's: quads (DPP lane ^ 1, ^ 2), 8-lane halves (row_half_mirror), 16-lane
// rows (row_mirror), then the two rows of the half (permlane16 swap returns
// the pair (own, partner) in some order).
GQ_DEV uint32_t max_half_wave(uint32_t v) {
  // (update_dpp with a zero old value and bound_ctrl: 0 is max's identity, so
  // each move fuses into the max as a DPP operand)
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, true));
  const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return max(s[0], s[1]);
}

// Activation range: each batch row's 256-k window (32 runs of 8, one per
// lane of a 32-lane half) is converted to fp16 after scaling by 2^s, s = 14 -
// floor(log2(max |x|)) over the window, clamped to [-100, 100] so both 2^s and
// 2^-s are normal floats: the window's largest entry lands in [2^14, 2^15),
// so no entry overflows fp16 and entries down to 2^-24 of the largest stay
// normal (also after the 1/16 of the 4-bit formats' high-nibble slots).  An
// all-zero window gets 2^100 (zeros stay zeros), one holding Inf or NaN
// 2^-100 (they stay Inf / NaN).  The window's dot products are multiplied by
// 2^-s (exact) as they are added to the fp32 accumulator.  `in` false: the
// run is outside the data (its values do not count).  Returns 2^s; *unscale
// receives 2^-s.
GQ_DEV float window_scale(const float (&xv)[8], bool in, float *unscale) {
  // (magnitudes compared as their bit patterns: monotonic for non-negative
  // floats, NaN above Inf)
  float am = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(xv[e]));
  const uint32_t eb = max_half_wave(in ? __float_as_uint(am) : 0u) >> 23;
  // biased exponent of 2^s: 127 + 14 - (eb - 127), clamped to 127 +- 100
  const uint32_t fe = (uint32_t)min(max(268 - (int)eb, 27), 227);
  *unscale = __uint_as_float((254u - fe) << 23);
  return __uint_as_float(fe << 23);
}

// 8 activations (one run) -> one fp16 A-fragment half, scaled by f, in the
// weights' slot order (4-bit formats: kQ4Perm, the kQ4Div16 slots divided by
// 16); zero when !in
template <int FMT>
GQ_DEV gq_u4 stage_run(const float (&xv)[8], float f, bool in) {
  gq_half8 h;
  const float f16 = f * 0.0625f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (kNibOrder<FMT>)
      h[e] = (_Float16)(xv[kQ4Perm[e]] * (kQ4Div16[e] ? f16 : f));
    else
      h[e] = (_Float16)(xv[e] * f);
  }
  gq_u4 hv = __builtin_bit_cast(gq_u4, h);
#pragma unroll
  for (int e = 0; e < 4; ++e) hv[e] = in ? hv[e] : 0u;
  return hv;
}

// Activation staging window: kWin consecutive k of every K part, converted to
// fp16 A fragments in LDS once per workgroup and shared by its TW row tiles.
constexpr int kWin = 256;

// Workgroup = TW row tiles x KS parts of K, one wave per (tile, part).  The
// waves of a part walk their K range window by window: weights are loaded two
// windows ahead into registers, the activations of the next window are loaded
// (fp32, coalesced runs of 8) while the current window is consumed, then
// converted into the other LDS buffer; one barrier per window.  A lane (g, r)
// of the A fragment for 64-k step m, half j holds x[r][64 m + 16 g + 8 j + 0..7]
// (4-bit formats: in kQ4Perm order, the kQ4Div16 elements divided by 16)
// (rows >= batch are zero), matching the weights dequant_step gives lane
// (g, r).  The KS parts' partial sums are reduced in LDS at the end.  MR
// activation rows are staged, as in k_gemv_h1 (MR = 8 up to batch 8: A rows
// 8..15 re-read rows 0..7, their D rows are never stored).
template <int FMT, int TW, int KS, int MR>
__global__ void __launch_bounds__(64 * TW * KS)
k_gemv_h(const uint8_t *__restrict__ w, size_t sc_off, const float *__restrict__ x, float *__restrict__ y, int N,
         int K, int C, int nb, int NI) {
  using F = HFmt<FMT>;
  static_assert(MR == 8 || MR == 16, "rows staged");
  constexpr int WC = kWin / F::CK;                   // chunks per window
  constexpr int NT = 64 * TW * KS;                   // threads
  constexpr int WB = kWin * 2 * MR;                  // LDS bytes per part and window: [kWin/64][2][4][MR][16]
  constexpr int RPT = (KS * MR * (kWin / 8)) / NT;   // x runs of 8 per thread per window
  static_assert(RPT >= 1 && RPT * NT == KS * MR * (kWin / 8), "runs must divide evenly");
  __shared__ __attribute__((aligned(16))) unsigned char xs[2][KS][WB];
  __shared__ __attribute__((aligned(16))) float xsc[2][KS * MR];  // 2^-s per (part, batch row) of a window
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tt = wave % TW, part = wave / TW;
  const int g = lane >> 4, r = lane & 15;
  const int ntiles = (int)gq_tiles(N);
  const size_t tile = (size_t)blockIdx.x * TW + tt;
  const HSrc<FMT> src = hsrc<FMT>(w, sc_off, tile < (size_t)ntiles ? tile : (size_t)ntiles - 1, C, N, K, lane);
  const int c0 = (C * part) / KS, c1 = (C * (part + 1)) / KS;  // this wave's chunks (c0 < c1: KS <= C)

  // weights of window `it` (chunks past the part re-read its last chunk)
  auto load_win = [&](int it, HChunk<FMT> (&ch)[WC]) {
#pragma unroll
    for (int j = 0; j < WC; ++j) {
      int ci = c0 + it * WC + j;
      ci = ci < c1 ? ci : c1 - 1;
      load_src<FMT>(src, ci, ch[j]);
    }
  };
  // activations: run u of this thread = (part p, batch row b, 8-run kr); its
  // source row, first k and end of K range are fixed, each window adds kWin
  gq_f4 xr[RPT][2];
  bool xin[RPT];
  const float *xsrc[RPT];
  int xk0[RPT], xk1[RPT];
  uint32_t xdst[RPT];
  int xsrow[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int run = (int)threadIdx.x + u * NT;
    const int kr = run & 31, b = (run >> 5) % MR, p = run / (32 * MR);
    xsrow[u] = p * MR + b;
    const int pc0 = (C * p) / KS, pc1 = (C * (p + 1)) / KS;
    xsrc[u] = x + (size_t)(b < nb ? b : 0) * K;
    xk0[u] = pc0 * F::CK + 8 * kr;
    xk1[u] = b < nb ? min(pc1 * F::CK, K) : 0;  // K % 32 == 0: a run is wholly in or out
    const int o = 8 * kr, m = o >> 6, gq = (o & 63) >> 4, j = (o & 15) >> 3;
    xdst[u] = (uint32_t)(p * WB + (((m * 2 + j) * 4 + gq) * MR + b) * 16);
  }
  auto load_x = [&](int it) {
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      // unconditional load from a clamped address, zeroed after: no branches
      const int k = xk0[u] + it * kWin;
      const bool in = k < xk1[u];
      const gq_f4 *src = reinterpret_cast<const gq_f4 *>(xsrc[u] + (in ? k : 0));
      xr[u][0] = src[0];
      xr[u][1] = src[1];
      xin[u] = in;
    }
  };
  // (a run's 32-lane half holds one (part, batch row) window: the window's
  // scale is reduced over it and lane 0 of the half records 2^-s)
  auto store_x = [&](int buf) {
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      const float xv[8] = {xr[u][0][0], xr[u][0][1], xr[u][0][2], xr[u][0][3],
                           xr[u][1][0], xr[u][1][1], xr[u][1][2], xr[u][1][3]};
      float us;
      const float f = window_scale(xv, xin[u], &us);  // (xin false: k past the part / K, or b >= batch)
      *reinterpret_cast<gq_u4 *>(&xs[buf][0][0] + xdst[u]) = stage_run<FMT>(xv, f, xin[u]);
      if ((lane & 31) == 0) xsc[buf][xsrow[u]] = us;
    }
  };

  const int nwin = ((c1 - c0) + WC - 1) / WC;  // this wave's windows (<= NI)
  const uint32_t mg = gq_nib_magic();
  HChunk<FMT> w0[WC], w1[WC], w2[WC];
  load_win(0, w0);
  load_win(1, w1);  // (a surplus re-read when NI == 1)
  load_x(0);
  store_x(0);
  __syncthreads();
  // acc, acc2: the sums of halves 0 and 1, unscaled (each window's chains
  // times the window's 2^-s)
  gq_f4 acc = gq_f4{0.f, 0.f, 0.f, 0.f}, acc2 = acc;
  // Window `it` (weights in cur).  PF: the activations of window it + 1 and
  // the weights of window it + 2 (into nxt, the buffer window it - 1
  // consumed) are requested first.  The three weight buffers rotate through the
  // roles by unrolling (no register copies).  The prefetch choices are
  // compile-time constants at every call, so no load sits under a branch (a
  // branch around a load makes the compiler wait for every load issued
  // before it).
  auto window = [&](int it, HChunk<FMT>(&cur)[WC], HChunk<FMT>(&nxt)[WC], auto pfw, auto pfx) {
    // (activations first: the wait for them before the staging below then
    // leaves the weight loads in flight)
    if constexpr (decltype(pfx)::value) load_x(it + 1);
    if constexpr (decltype(pfw)::value) load_win(it + 2, nxt);
    if (it < nwin) {
      const unsigned char *xb = xs[it & 1][part] + (g * MR + (r & (MR - 1))) * 16;  // this lane's A row
      gq_f4 wa = gq_f4{0.f, 0.f, 0.f, 0.f}, wb = wa;  // the window's chains of halves 0 and 1
#pragma unroll
      for (int j = 0; j < WC; ++j) {
        if (c0 + it * WC + j < c1) {
#pragma unroll
          for (int m = 0; m < F::STEPS; ++m) {
            const int ms = j * F::STEPS + m;
            const gq_half8 a0 = *reinterpret_cast<const gq_half8 *>(xb + (ms * 2 + 0) * 4 * MR * 16);
            const gq_half8 a1 = *reinterpret_cast<const gq_half8 *>(xb + (ms * 2 + 1) * 4 * MR * 16);
            gq_half8 b0, b1;
            dequant_step<FMT>(cur[j], m, g, mg, b0, b1);
            wa = mfma16h(a0, b0, wa);
            wb = mfma16h(a1, b1, wb);
          }
        }
      }
      // D rows 4g..4g+3 (MR = 8: A rows 8..15 are rows 0..7 again)
      const gq_f4 us = *reinterpret_cast<const gq_f4 *>(&xsc[it & 1][part * MR + ((4 * g) & (MR - 1))]);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        acc[v] = fmaf(wa[v], us[v], acc[v]);
        acc2[v] = fmaf(wb[v], us[v], acc2[v]);
      }
    }
    if constexpr (decltype(pfx)::value) store_x((it + 1) & 1);
    __syncthreads();
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  int it = 0;
  for (; it + 5 <= NI; it += 3) {
    window(it, w0, w2, T_{}, T_{});
    window(it + 1, w1, w0, T_{}, T_{});
    window(it + 2, w2, w1, T_{}, T_{});
  }
  // the last 1..4 windows, the buffer roles continuing the rotation
  switch (NI - it) {
  case 1:
    window(it, w0, w2, F_{}, F_{});
    break;
  case 2:
    window(it, w0, w2, F_{}, T_{});
    window(it + 1, w1, w0, F_{}, F_{});
    break;
  case 3:
    window(it, w0, w2, T_{}, T_{});
    window(it + 1, w1, w0, F_{}, T_{});
    window(it + 2, w2, w1, F_{}, F_{});
    break;
  default:
    window(it, w0, w2, T_{}, T_{});
    window(it + 1, w1, w0, T_{}, T_{});
    window(it + 2, w2, w1, F_{}, T_{});
    window(it + 3, w0, w2, F_{}, F_{});
    break;
  }
#pragma unroll
  for (int v = 0; v < 4; ++v) acc[v] += acc2[v];
  // ---- reduce over the KS parts (LDS reused); D lane (g, r): batch rows 4g..4g+3, column r
  if constexpr (KS > 1) {
    gq_f4 *red = reinterpret_cast<gq_f4 *>(&xs[0][0][0]);  // [KS][TW][64]
    red[(part * TW + tt) * 64 + lane] = acc;
    __syncthreads();
    if (part != 0) return;
    gq_f4 s = red[tt * 64 + lane];
#pragma unroll
    for (int q = 1; q < KS; ++q) {
      const gq_f4 v = red[(q * TW + tt) * 64 + lane];
      s[0] += v[0];
      s[1] += v[1];
      s[2] += v[2];
      s[3] += v[3];
    }
    acc = s;
  }
  const size_t row = tile * 16 + r;
  if (tile < (size_t)ntiles && row < (size_t)N) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int b = 4 * g + v;
      if (b < nb) y[(size_t)b * N + row] = acc[v];
    }
  }
}

// One-stage variant for K parts that fit: every wave issues the loads of ALL
// its chunks up front (like the int8 GEMV), the workgroup stages its whole
// activation range once (x loads are issued before the weight loads, so waiting
// for them never waits for a weight), one barrier, then each wave consumes its
// chunks in arrival order with no further synchronisation.  NCK (chunks per
// wave) and the LDS size KS * NCK * CK * 32 bytes are compile-time; the host
// picks this kernel only where both fit.
//
// MR (8 or 16) is the number of activation rows staged.  With MR = 8 (batch
// <= 8) the LDS holds half as much (two workgroups per CU) and the lanes of
// A rows 8..15 read rows 0..7 again: an A row only feeds the same row of D,
// and D rows >= batch are never stored.
template <int FMT, int TW, int KS, int NCK, int MR>
__global__ void __launch_bounds__(64 * TW * KS)
k_gemv_h1(const uint8_t *__restrict__ w, size_t sc_off, const float *__restrict__ x, float *__restrict__ y, int N,
          int K, int C, int nb) {
  using F = HFmt<FMT>;
  static_assert(MR == 8 || MR == 16, "rows staged");
  constexpr int NT = 64 * TW * KS;
  constexpr int PK = NCK * F::CK;                // k per part (padded)
  constexpr int PB = PK * 2 * MR;                // LDS bytes per part: [PK/64][2][4][MR][16]
  constexpr int NWIN = (PK + 255) / 256;         // 256-k windows per part (each with its own scale)
  constexpr int WC = 256 / F::CK;                // chunks per window
  constexpr int RPR = 32 * NWIN;                 // 8-element runs per (part, batch row), whole windows
  constexpr int RUNS = KS * MR * RPR;
  constexpr int RPT = (RUNS + NT - 1) / NT;
  constexpr bool kSkip = (RUNS % NT != 0) || (PK % 256 != 0);  // runs with nothing to store exist
  // (also the partial tiles' reduction [KS][TW][64] x 16 bytes at the end)
  constexpr int XSB = KS * PB > KS * TW * 64 * 16 ? KS * PB : KS * TW * 64 * 16;
  __shared__ __attribute__((aligned(16))) unsigned char xs[XSB];
  __shared__ __attribute__((aligned(16))) float xsc[KS * NWIN * MR];  // 2^-s per (part, window, batch row)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tt = wave % TW, part = wave / TW;
  const int g = lane >> 4, r = lane & 15;
  const int ntiles = (int)gq_tiles(N);
  const size_t tile = (size_t)blockIdx.x * TW + tt;
  const HSrc<FMT> src = hsrc<FMT>(w, sc_off, tile < (size_t)ntiles ? tile : (size_t)ntiles - 1, C, N, K, lane);
  const int c0 = (C * part) / KS, c1 = (C * (part + 1)) / KS;  // c0 < c1 (KS <= C)
  const int nck = c1 - c0;                                     // <= NCK (host-checked)

  // ---- 1. activation loads (the workgroup's whole range), then weights -------
  // run -> (part p, batch row b, run kr of the row's part); the 32 runs of a
  // window are one 32-lane half (RPR and NT are multiples of 32)
  gq_f4 xr[RPT][2];
  bool xin[RPT];
  uint32_t xdst[RPT];
  int xsi[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int run = (int)threadIdx.x + u * NT;
    const int kr = run % RPR, b = (run / RPR) % MR, p = run / (MR * RPR);
    const int pc0 = (C * p) / KS, pc1 = (C * (p + 1)) / KS;
    const int k = pc0 * F::CK + 8 * kr;
    const bool in = run < RUNS && b < nb && k < pc1 * F::CK && k < K;  // K % 32 == 0: runs are whole
    const gq_f4 *src = reinterpret_cast<const gq_f4 *>(x + (in ? (size_t)b * K + k : 0));
    xr[u][0] = src[0];
    xr[u][1] = src[1];
    xin[u] = in;
    const int o = 8 * kr, ms = o >> 6, gq = (o & 63) >> 4, j = (o & 15) >> 3;
    xdst[u] = (run < RUNS && o < PK) ? (uint32_t)(p * PB + (((ms * 2 + j) * 4 + gq) * MR + b) * 16) : 0xFFFFFFFFu;
    xsi[u] = run < RUNS ? (p * NWIN + kr / 32) * MR + b : -1;
  }
  __builtin_amdgcn_sched_barrier(0);
  HChunk<FMT> ch[NCK];
#pragma unroll
  for (int i = 0; i < NCK; ++i) {
    const int ci = c0 + i < c1 ? c0 + i : c1 - 1;  // surplus loads re-read the last chunk
    load_src<FMT>(src, ci, ch[i]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. activations -> scaled fp16 A fragments in LDS -------------------------
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const float xv[8] = {xr[u][0][0], xr[u][0][1], xr[u][0][2], xr[u][0][3],
                         xr[u][1][0], xr[u][1][1], xr[u][1][2], xr[u][1][3]};
    float us;
    const float f = window_scale(xv, xin[u], &us);  // (all lanes: a cross-lane reduction)
    if ((lane & 31) == 0 && xsi[u] >= 0) xsc[xsi[u]] = us;
    if (kSkip && xdst[u] == 0xFFFFFFFFu) continue;
    *reinterpret_cast<gq_u4 *>(xs + xdst[u]) = stage_run<FMT>(xv, f, xin[u]);
  }
  __syncthreads();

  // ---- 3. consume ------------------------------------------------------------------
  const uint32_t mg = gq_nib_magic();
  // this lane's A row: r (MR = 16) or r & 7 (MR = 8)
  const unsigned char *xb = xs + part * PB + (g * MR + (r & (MR - 1))) * 16;
  // acc, acc2: the sums of halves 0 and 1, unscaled; pa, pb: the previous
  // window's chains (window pw), added in times its 2^-s at the start of the
  // next window, when its MFMAs have finished
  gq_f4 acc = gq_f4{0.f, 0.f, 0.f, 0.f}, acc2 = acc, pa = acc, pb = acc;
  int pw = 0;
  auto fold = [&]() {
    // D rows 4g..4g+3 (MR = 8: A rows 8..15 are rows 0..7 again)
    const gq_f4 us = *reinterpret_cast<const gq_f4 *>(&xsc[(part * NWIN + pw) * MR + ((4 * g) & (MR - 1))]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc[v] = fmaf(pa[v], us[v], acc[v]);
      acc2[v] = fmaf(pb[v], us[v], acc2[v]);
    }
  };
  // one window: its chunks on two chains (halves 0 and 1 of each step)
  auto consume_win = [&](int wv, auto full) {
    fold();  // (a no-op before the first window: pa, pb are zero)
    gq_f4 wa = gq_f4{0.f, 0.f, 0.f, 0.f}, wb = wa;
#pragma unroll
    for (int jj = 0; jj < WC; ++jj) {
      const int i = wv * WC + jj;
      if (i >= NCK) break;
      if (!decltype(full)::value && i >= nck) break;
#pragma unroll
      for (int m = 0; m < F::STEPS; ++m) {
        const int ms = i * F::STEPS + m;
        const gq_half8 a0 = *reinterpret_cast<const gq_half8 *>(xb + (ms * 2 + 0) * 4 * MR * 16);
        const gq_half8 a1 = *reinterpret_cast<const gq_half8 *>(xb + (ms * 2 + 1) * 4 * MR * 16);
        gq_half8 b0, b1;
        dequant_step<FMT>(ch[i], m, g, mg, b0, b1);
        wa = mfma16h(a0, b0, wa);
        wb = mfma16h(a1, b1, wb);
      }
    }
    pa = wa;
    pb = wb;
    pw = wv;
  };
  if (nck == NCK) {
#pragma unroll
    for (int wv = 0; wv < NWIN; ++wv) consume_win(wv, std::true_type{});
  } else {
#pragma unroll
    for (int wv = 0; wv < NWIN; ++wv)
      if (wv * WC < nck) consume_win(wv, std::false_type{});
  }
  fold();
#pragma unroll
  for (int v = 0; v < 4; ++v) acc[v] += acc2[v];

  // ---- 4. reduce over the KS parts (LDS reused) ---------------------------------
  if constexpr (KS > 1) {
    __syncthreads();
    gq_f4 *red = reinterpret_cast<gq_f4 *>(xs);  // [KS][TW][64]
    red[(part * TW + tt) * 64 + lane] = acc;
    __syncthreads();
    if (part != 0) return;
    gq_f4 sum = red[tt * 64 + lane];
#pragma unroll
    for (int q = 1; q < KS; ++q) {
      const gq_f4 v = red[(q * TW + tt) * 64 + lane];
      sum[0] += v[0];
      sum[1] += v[1];
      sum[2] += v[2];
      sum[3] += v[3];
    }
    acc = sum;
  }
  const size_t row = tile * 16 + r;
  if (tile < (size_t)ntiles && row < (size_t)N) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int b = 4 * g + v;
      if (b < nb) y[(size_t)b * N + row] = acc[v];
    }
  }
}

// Skinny GEMM (M <= 256): C[m][n] = sum_k A[m][k] W[n][k] for few rows of A.
// The tiled GEMM walks K in 64-element steps, each waiting on loads requested a
// few steps earlier, on grids of few workgroups; here a workgroup takes CT row
// tiles of W (16 output columns each) and a block of 16 MT rows of A (64; 32
// in the 16-wave variant), and splits K over its KW waves (8; 16 for long K)
// like the GEMV: each wave requests all of its chunks
// (at most NCK) of the CT tiles up front, streams its A fragments straight
// from global memory (no LDS: no two waves share them) one 64-k step ahead,
// and issues MT x CT x 2 v_mfma_f32_16x16x32_f16 per step on weights
// dequantized once (dequant_step).  The KW partial tiles are added in LDS.
// A is fp16 [M][lda] in the B fragments' order: for the 4-bit formats each
// aligned run of 8 k holds slots kQ4Perm with the kQ4Div16 slots divided by 16
// (k_a_to_f16 with q4perm).  Rows >= M read row M - 1 and are not stored.
template <int FMT, int CT, int NCK, bool CBF16, int KW = 8, int MT = 4>
__global__ void __launch_bounds__(64 * KW) k_gemm_sk(const uint8_t *__restrict__ w, size_t sc_off,
                                                     const _Float16 *__restrict__ a16, int lda, void *__restrict__ c,
                                                     const float *__restrict__ rs, int M, int N, int C, int K) {
  using F = HFmt<FMT>;
  constexpr int NS = NCK * F::STEPS;  // 64-k steps per wave (static bound)
  __shared__ gq_f4 red[KW][CT * MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int ntiles = (int)gq_tiles(N);
  const int m0 = (int)blockIdx.y * 16 * MT;
  const int c0 = (C * wave) / KW, c1 = (C * (wave + 1)) / KW;
  const int nck = c1 - c0;  // <= NCK (host-checked); 0 when C < KW
  const int clast = nck > 0 ? c1 - 1 : c0;  // last chunk a load may name (c0 < C always)
  // weights: every chunk of the wave, tile by tile (surplus loads re-read the
  // last chunk)
  HChunk<FMT> ch[CT][NCK];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int t0 = (int)blockIdx.x * CT + ct;
    const HSrc<FMT> src = hsrc<FMT>(w, sc_off, (size_t)(t0 < ntiles ? t0 : ntiles - 1), C, N, K, lane);
#pragma unroll
    for (int i = 0; i < NCK; ++i) {
      const int ci = c0 + i <= clast ? c0 + i : clast;
      load_src<FMT>(src, ci, ch[ct][i]);
    }
  }
  // this lane's A rows: 16 mt + r of the block, k offset 16 g
  const _Float16 *arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = m0 + 16 * mt + r;
    arow[mt] = a16 + (size_t)(row < M ? row : M - 1) * lda + 16 * g;
  }
  // A fragments of step s: chunk s / STEPS of the wave, 64-k step s % STEPS,
  // halves j = 0, 1 (k + 8 j)
  auto load_a = [&](int s, gq_half8 (&af)[2][MT]) {
    const int i = s / F::STEPS, ci = c0 + i <= clast ? c0 + i : clast;
    const int k = ci * F::CK + 64 * (s % F::STEPS);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      af[0][mt] = *reinterpret_cast<const gq_half8 *>(arow[mt] + k);
      af[1][mt] = *reinterpret_cast<const gq_half8 *>(arow[mt] + k + 8);
    }
  };
  gq_f4 acc[CT][MT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[ct][mt] = gq_f4{0.f, 0.f, 0.f, 0.f};
  const uint32_t mg = gq_nib_magic();
  // A fragments requested AP steps ahead (ring of AP + 1; 2 and 3 measured no
  // faster)
  constexpr int AP = 1;
  gq_half8 abuf[AP + 1][2][MT];
#pragma unroll
  for (int s = 0; s < AP && s < NS; ++s) load_a(s, abuf[s]);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    if (s + AP < NS) load_a(s + AP, abuf[(s + AP) % (AP + 1)]);
    // keep the prefetch ahead of this step's work (the scheduler would
    // otherwise sink it below the MFMAs that wait on the current fragments)
    __builtin_amdgcn_sched_barrier(0);
    const int i = s / F::STEPS, m = s % F::STEPS;
    // steps past the wave's chunks multiply zeros (no branch: a branch here
    // makes the compiler wait for every load in flight)
    const uint32_t live = i < nck ? 0xFFFFFFFFu : 0u;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      gq_half8 b0, b1;
      dequant_step<FMT>(ch[ct][i], m, g, mg, b0, b1);
      gq_u4 u0 = __builtin_bit_cast(gq_u4, b0), u1 = __builtin_bit_cast(gq_u4, b1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        u0[e] &= live;
        u1[e] &= live;
      }
      b0 = __builtin_bit_cast(gq_half8, u0);
      b1 = __builtin_bit_cast(gq_half8, u1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[ct][mt] = mfma16h(abuf[s % (AP + 1)][0][mt], b0, acc[ct][mt]);
        acc[ct][mt] = mfma16h(abuf[s % (AP + 1)][1][mt], b1, acc[ct][mt]);
      }
    }
  }
  // partial tiles of the KW waves; wave p adds up pair p (and p + KW, ...)
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][ct * MT + mt][lane] = acc[ct][mt];
  __syncthreads();
  for (int p = wave; p < CT * MT; p += KW) {
    gq_f4 sum = red[0][p][lane];
#pragma unroll
    for (int q = 1; q < KW; ++q) {
      const gq_f4 v = red[q][p][lane];
      sum[0] += v[0];
      sum[1] += v[1];
      sum[2] += v[2];
      sum[3] += v[3];
    }
    const int ct = p / MT, mt = p % MT;
    const int t0 = (int)blockIdx.x * CT + ct;
    const int col = t0 * 16 + r;
    if (t0 >= ntiles || col >= N) continue;
    // row scales of the A conversion (powers of two; the buffer is padded past M)
    const gq_f4 rsv = rs ? *reinterpret_cast<const gq_f4 *>(rs + m0 + 16 * mt + 4 * g) : gq_f4{1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int row = m0 + 16 * mt + 4 * g + v;
      if (row >= M) continue;
      const float o = sum[v] * rsv[v];
      if constexpr (CBF16) {
        uint32_t u = __float_as_uint(o);
        uint16_t hb;
        if ((u & 0x7F800000u) == 0x7F800000u) {
          hb = (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
        } else {
          u += 0x7FFFu + ((u >> 16) & 1u);
          hb = (uint16_t)(u >> 16);
        }
        reinterpret_cast<uint16_t *>(c)[(size_t)row * N + col] = hb;
      } else {
        reinterpret_cast<float *>(c)[(size_t)row * N + col] = o;
      }
    }
  }
}

int env_int(const char *name) {
  const char *e = getenv(name);
  return e ? atoi(e) : 0;
}

}  // namespace

// Launch plan of the fp16 batch GEMV: TW (1, 2 or 4) row tiles and KS (1..8)
// parts of K per workgroup.  Wide matrices share each staged activation
// window across 4 (or 2) row tiles; K is split until the grid holds about
// 3584 waves (3.5 per SIMD; measured best on 14336 x 4096), at most 8 parts
// (the double-buffered windows take KS x 16 KiB of LDS), at most one part
// per chunk and at most 16 waves per workgroup.  chunks_per_wave is the
// longest part.
// Plan of the one-stage kernel (k_gemv_h1), or GQ_ERR_UNSUPPORTED where it does
// not apply: 16 waves per workgroup as TW row tiles x (16 / TW) K parts, the
// activations of all of K in LDS (MR rows x 2 bytes per k: 8 rows up to batch
// 8, else 16; at most 128 KiB) and each wave's chunks in registers
// (kH1MaxChunks).  Workgroups per CU: 2 with 8 rows (<= 64 KiB), else 1; TW is
// the largest that still gives every slot a workgroup, in one round.  Not for
// the register-heavy Q8_0 / Q6_K chunks.  GQ_GEMV_H1=0 turns the kernel off,
// =1 forces it wherever it fits.
int gq_gemv_h1_plan(int fmt, size_t N, size_t K, int nb, int *R_out, int *ks_out, int *cpw_out) {
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt;
  const int e = env_int("GQ_GEMV_H1");
  if (e == 0 && getenv("GQ_GEMV_H1")) return GQ_ERR_UNSUPPORTED;
  if (e != 1 && (f == GQ_FMT_Q8_0 || f == GQ_FMT_Q6_K)) return GQ_ERR_UNSUPPORTED;
  if (f == GQ_FMT_F16) return GQ_ERR_UNSUPPORTED;  // (its chunks spill the 16-wave workgroups)
  const int C = (int)gq_chunks(f, K);
  const int CK = f == GQ_FMT_Q4_K || f == GQ_FMT_Q6_K ? 256 : 128;
  const int maxc = f == GQ_FMT_Q4_0 || f == GQ_FMT_Q8_0 ? 8 : 4;
  const int mr = nb <= 8 ? 8 : 16;
  const size_t slots = 256 * (mr == 8 ? 2 : 1);
  const size_t tiles = gq_tiles(N);
  int tw = 8;
  while (tw > 1 && (tiles + tw - 1) / tw < slots * 7 / 8) tw /= 2;
  const int ks = 16 / tw;
  if (ks > C) return GQ_ERR_UNSUPPORTED;
  const int nck = (C + ks - 1) / ks;
  const int nckp = nck <= 1 ? 1 : nck <= 2 ? 2 : nck <= 4 ? 4 : nck <= 8 ? 8 : 16;
  if (nckp > maxc) return GQ_ERR_UNSUPPORTED;
  if ((size_t)ks * nckp * CK * 2 * mr > (mr == 8 ? 64 : 128) * 1024) return GQ_ERR_UNSUPPORTED;
  // a win on grids of up to 512 row tiles only: 4096 x 4096 batch 8 / 16 6.3 / 7.8
  // vs 6.8 / 9.1 us, 1024 x 4096 batch 8 5.5 vs 6.0 us; on 896 tiles (14336
  // rows) the windowed kernel's 4-tile workgroups are faster (Q4_K batch 5 / 8
  // 12.0 / 12.2 vs 12.9-13.3 / 13.4-13.5 us, Q4_0 batch 8 11.9 vs 12.4 us,
  // measured on two boxes)
  if (e != 1 && tiles > 512) return GQ_ERR_UNSUPPORTED;
  if (e != 1 && (tiles + tw - 1) / tw > slots) return GQ_ERR_UNSUPPORTED;
  *R_out = tw;
  *ks_out = ks;
  *cpw_out = nck;
  return GQ_OK;
}

int gq_gemv_h_plan(int fmt, size_t N, size_t K, int nb, int *R_out, int *ks_out, int *cpw_out) {
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt;
  const int C = (int)gq_chunks(f, K);
  const size_t tiles = gq_tiles(N);
  int tw = tiles >= 800 ? 4 : tiles >= 400 ? 2 : 1;
  const int er = env_int("GQ_GEMV_H_R");
  if (er == 1 || er == 2 || er == 4) tw = er;
  (void)nb;  // batch-independent (a 16-way split of 8-row windows measured slower than 8)
  // fp16 weights: 64 registers of weights per window and wave; at most 8
  // waves per workgroup, so the register budget holds them without spilling
  const int maxw = f == GQ_FMT_F16 ? 8 : 16;
  if (tw > maxw) tw = maxw;
  int ks = 1;
  while (ks < 8 && tiles * ks < 3584 && 2 * ks <= C && tw * ks < maxw) ks *= 2;
  const int e = env_int("GQ_GEMV_H_KSPLIT");
  if ((e == 1 || e == 2 || e == 4 || e == 8) && e <= C) ks = e;
  if (tw * ks > maxw) tw = maxw / ks > 0 ? maxw / ks : 1;
  *R_out = tw;
  *ks_out = ks;
  *cpw_out = (C + ks - 1) / ks;
  return GQ_OK;
}

namespace {
template <int FMT, int TW, int MR>
int launch_h_tw(const void *packed, const float *x, float *y, int N, int K, int nb, int ks, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K);
  const size_t wgs = (gq_tiles(N) + TW - 1) / TW;
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const uint8_t *w = (const uint8_t *)packed;
  constexpr int WC = kWin / HFmt<FMT>::CK;
  const int NI = ((C + ks - 1) / ks + WC - 1) / WC;
  // x runs must spread evenly over the threads (TW <= MR / 2)
#define GQ_LAUNCH_H(KS)                                                                                               \
  if constexpr (2 * TW <= MR && !(FMT == GQ_FMT_F16 && TW * KS > 8)) {                                               \
    hipLaunchKernelGGL((k_gemv_h<FMT, TW, KS, MR>), dim3((unsigned)wgs), dim3(64 * TW * KS), 0, s, w, sc_off, x, y, \
                       N, K, C, nb, NI);                                                                              \
  } else {                                                                                                            \
    return GQ_ERR_INVALID_ARGS;                                                                                       \
  }
  switch (ks) {
  case 1: GQ_LAUNCH_H(1); break;
  case 2: GQ_LAUNCH_H(2); break;
  case 4: GQ_LAUNCH_H(4); break;
  default:
    if constexpr (TW <= 2) { GQ_LAUNCH_H(8); }
    else return GQ_ERR_INVALID_ARGS;
    break;
  }
#undef GQ_LAUNCH_H
  return gq_last_launch();
}

// chunk registers a wave may hold in the one-stage kernel
template <int FMT>
constexpr int kH1MaxChunks = (FMT == GQ_FMT_Q4_0) ? 8 : (FMT == GQ_FMT_Q8_0) ? 8 : 4;

template <int FMT, int TW, int KS, int MR>
int launch_h1_nck(const void *packed, const float *x, float *y, int N, int K, int nb, int nck, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K);
  const size_t wgs = (gq_tiles(N) + TW - 1) / TW;
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const uint8_t *w = (const uint8_t *)packed;
  // instantiated only where the activations fit the LDS (KS * NCK * CK * 32 bytes)
#define GQ_LAUNCH_H1(NCK)                                                                                          \
  if constexpr (NCK <= kH1MaxChunks<FMT> && KS * NCK * HFmt<FMT>::CK * 2 * MR <= 128 * 1024) {                     \
    hipLaunchKernelGGL((k_gemv_h1<FMT, TW, KS, NCK, MR>), dim3((unsigned)wgs), dim3(64 * TW * KS), 0, s, w, sc_off, \
                       x, y, N, K, C, nb);                                                                         \
    return gq_last_launch();                                                                                       \
  }                                                                                                                \
  return GQ_ERR_INVALID_ARGS;
  if (nck <= 1) { GQ_LAUNCH_H1(1) }
  if (nck <= 2) { GQ_LAUNCH_H1(2) }
  if (nck <= 4) { GQ_LAUNCH_H1(4) }
  if (nck <= 8) { GQ_LAUNCH_H1(8) }
  return GQ_ERR_INVALID_ARGS;
#undef GQ_LAUNCH_H1
}

template <int FMT>
int launch_h(const void *packed, const float *x, float *y, int N, int K, int nb, hipStream_t s) {
  int tw, ks, cpw;
  if (gq_gemv_h1_plan(FMT, N, K, nb, &tw, &ks, &cpw) == GQ_OK) {
    if (nb <= 8) {
      if (tw == 1) return launch_h1_nck<FMT, 1, 16, 8>(packed, x, y, N, K, nb, cpw, s);
      if (tw == 2) return launch_h1_nck<FMT, 2, 8, 8>(packed, x, y, N, K, nb, cpw, s);
      if (tw == 4) return launch_h1_nck<FMT, 4, 4, 8>(packed, x, y, N, K, nb, cpw, s);
      return launch_h1_nck<FMT, 8, 2, 8>(packed, x, y, N, K, nb, cpw, s);
    }
    if (tw == 1) return launch_h1_nck<FMT, 1, 16, 16>(packed, x, y, N, K, nb, cpw, s);
    if (tw == 2) return launch_h1_nck<FMT, 2, 8, 16>(packed, x, y, N, K, nb, cpw, s);
    if (tw == 4) return launch_h1_nck<FMT, 4, 4, 16>(packed, x, y, N, K, nb, cpw, s);
    return launch_h1_nck<FMT, 8, 2, 16>(packed, x, y, N, K, nb, cpw, s);
  }
  GQ_TRY(gq_gemv_h_plan(FMT, N, K, nb, &tw, &ks, &cpw));
  if (nb <= 8) {
    if (tw == 4) return launch_h_tw<FMT, 4, 8>(packed, x, y, N, K, nb, ks, s);
    if (tw == 2) return launch_h_tw<FMT, 2, 8>(packed, x, y, N, K, nb, ks, s);
    return launch_h_tw<FMT, 1, 8>(packed, x, y, N, K, nb, ks, s);
  }
  if (tw == 4) return launch_h_tw<FMT, 4, 16>(packed, x, y, N, K, nb, ks, s);
  if (tw == 2) return launch_h_tw<FMT, 2, 16>(packed, x, y, N, K, nb, ks, s);
  return launch_h_tw<FMT, 1, 16>(packed, x, y, N, K, nb, ks, s);
}
}  // namespace

int gq_launch_gemv_h(int fmt, const void *packed, const float *x, float *y, int N, int K, int nb, hipStream_t s) {
  if (gq_fmt_is_q6k(fmt)) return launch_h<GQ_FMT_Q6_K>(packed, x, y, N, K, nb, s);
  switch (gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt) {
  case GQ_FMT_Q4_0: return launch_h<GQ_FMT_Q4_0>(packed, x, y, N, K, nb, s);
  case GQ_FMT_Q8_0: return launch_h<GQ_FMT_Q8_0>(packed, x, y, N, K, nb, s);
  default: return launch_h<GQ_FMT_Q4_K>(packed, x, y, N, K, nb, s);
  }
}

// ---- fp16 weights (row-major N x K): the reference's FP16 route ---------------
// C[M][N] = A[M][K] W^T with fp32 A, fp16 W and fp32 accumulation, batch
// GEMVs of up to 16 rows of A at a time on the fp16 batch kernels (the
// weights need no dequantization; A is rounded to fp16 after the per-window
// power-of-two scaling, as every batch GEMV here does).  Rows of A beyond 16
// take further launches (each re-reads W).
namespace {
// fp16 weights of any K or alignment (the matrix-core kernel needs K % 32 == 0
// and 16-byte rows): one workgroup of 4 waves per output column n, each wave
// one row of A, fp32 products of the fp32 activation and the fp16 weight
// summed over K (the reference's VALU route's arithmetic); rows of A beyond
// the grid's 4 * gridDim.y are taken in further strides
__global__ void __launch_bounds__(256) k_f16w_any(const _Float16 *__restrict__ w, const float *__restrict__ a,
                                                  float *__restrict__ c, int M, int N, int K) {
  const int n = blockIdx.x, lane = threadIdx.x & 63;
  const _Float16 *wr = w + (size_t)n * K;
  for (int m = blockIdx.y * 4 + (threadIdx.x >> 6); m < M; m += gridDim.y * 4) {
    const float *ar = a + (size_t)m * K;
    float sum = 0.f;
    for (int k = lane; k < K; k += 64) sum = fmaf(ar[k], (float)wr[k], sum);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
    if (lane == 0) c[(size_t)m * N + n] = sum;
  }
}
}  // namespace

extern "C" int gq_gemm_f16w(const void *w, const float *a, float *c, size_t M, size_t N, size_t K, void *stream) {
  GQ_CHECK(M <= GQ_MAX_DIM && N <= GQ_MAX_DIM && K <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(w && a && c, GQ_ERR_INVALID_ARGS);
  hipStream_t s = (hipStream_t)stream;
  if (M == 0 || N == 0) return GQ_OK;
  if (K == 0) return gq_fill_zero(c, M * N, s);
  // the matrix-core kernel's 16-element lane runs must not straddle rows, and
  // rows start 16-byte aligned; other shapes take the plain kernel
  if (K % 32 != 0 || (uintptr_t)w % 16 != 0 || (uintptr_t)a % 16 != 0) {
    const unsigned gy = (unsigned)((M + 3) / 4 < 65535 ? (M + 3) / 4 : 65535);
    hipLaunchKernelGGL(k_f16w_any, dim3((unsigned)N, gy), dim3(256), 0, s, (const _Float16 *)w, a, c, (int)M, (int)N,
                       (int)K);
    return gq_last_launch();
  }
  for (size_t m0 = 0; m0 < M; m0 += GQ_MAX_BATCH) {
    const int nb = (int)(M - m0 < (size_t)GQ_MAX_BATCH ? M - m0 : (size_t)GQ_MAX_BATCH);
    GQ_TRY(launch_h<GQ_FMT_F16>(w, a + m0 * K, c + m0 * N, (int)N, (int)K, nb, s));
  }
  return GQ_OK;
}

// The reference's two FP16-weight launchers under their argument lists
// (gemm_kernels.hpp:30-44): W is N x K (row stride K whatever ldb says, as the
// reference's kernels read b[n * K + k]); A rows at stride lda, C rows at
// stride ldc, both as GretaCompute::gemm passes them (K and N; other strides
// are refused).  The VALU launcher writes zeros for K == 0; the MFMA one
// returns at once when any dimension is zero (gemm_kernels.hip:347-358,
// 509-514).
extern "C" int gq_launch_gemm_mixed_f16f32(void *stream, const float *a, const void *b, float *c, uint32_t M,
                                           uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc) {
  (void)ldb;
  if (M == 0 || N == 0) return GQ_OK;
  GQ_CHECK(lda == K && ldc == N, GQ_ERR_UNSUPPORTED);
  return gq_gemm_f16w(b, a, c, M, N, K, stream);
}
extern "C" int gq_launch_gemm_mfma_mixed_f16f32(void *stream, const float *a, const void *b, float *c, uint32_t M,
                                                uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc) {
  (void)ldb;
  if (M == 0 || N == 0 || K == 0) return GQ_OK;
  GQ_CHECK(lda == K && ldc == N, GQ_ERR_UNSUPPORTED);
  return gq_gemm_f16w(b, a, c, M, N, K, stream);
}

// Skinny GEMM plan: M <= 256 (Q6_K: any M), a chunk list of at most 4 per wave
// of 8 (K <= 4096 for Q4_0 / Q8_0, 8192 for Q4_K; Q6_K 2, K <= 4096) or, for
// Q4_0 / Q4_K, 8 per wave of 16 (K <= 16384 / 32768; *nck_out = 16 + chunks), CT = 2 row tiles per workgroup where that
// still gives every CU a workgroup, and at most one workgroup per CU in all
// (two for the long-K form; each reads its 64 rows of A whole: measured slower
// than the tiled GEMM's K-group tiles beyond that).  GQ_ERR_UNSUPPORTED otherwise
// (the tiled GEMM takes the shape).  GQ_GEMM_SKINNY=0, or a tiled shape forced
// through GQ_GEMM_TILE, turns the kernel off.
int gq_gemm_skinny_plan(int fmt, size_t M, size_t N, size_t K, int *ct_out, int *nck_out) {
  const char *e = getenv("GQ_GEMM_SKINNY");
  if ((e && e[0] == '0') || getenv("GQ_GEMM_TILE")) return GQ_ERR_UNSUPPORTED;  // (a forced tiled shape)
  // Q6_K (no tiled GEMM; the alternative is the batch GEMV per 16 rows): any
  // M, at most 2 chunks per wave (K <= 4096; its chunks take 17 registers)
  const bool q6 = gq_fmt_is_q6k(fmt);
  if (M == 0 || (!q6 && M > 256) || N == 0 || K == 0) return GQ_ERR_UNSUPPORTED;
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : q6 ? GQ_FMT_Q6_K : fmt;
  const int C = (int)gq_chunks(f, K);
  const int nck = (C + 7) / 8;
  int nckp = nck <= 1 ? 1 : nck <= 2 ? 2 : nck <= 4 ? 4 : 0;
  if (q6 && nckp > 2) return GQ_ERR_UNSUPPORTED;
  const size_t tiles = gq_tiles(N), gy = (M + 63) / 64;
  const int cus0 = gq_device_cus();
  const size_t cus = cus0 > 0 ? (size_t)cus0 : 256;
  int ct = ((tiles + 1) / 2) * gy >= cus ? 2 : 1;
  size_t wgs = ((tiles + ct - 1) / ct) * gy;
  if (nckp == 0) {
    // long K: 16 waves (four per SIMD, so half the registers) on 32-row
    // blocks of A, one row tile, up to 8 chunks each for Q4_0 (K <= 16384)
    // and 4 for Q4_K (K <= 16384)
    const int n16 = (C + 15) / 16;
    if (q6 || f == GQ_FMT_Q8_0 || n16 > (f == GQ_FMT_Q4_0 ? 8 : 4)) return GQ_ERR_UNSUPPORTED;
    nckp = 16 + (n16 <= 4 ? 4 : 8);  // 16 + chunks: the 16-wave variant
    ct = 1;
    wgs = tiles * ((M + 31) / 32);
  }
  // (short K) more workgroups than CUs: the tiled GEMM's K-group shapes are
  // faster (4096 x 4096: 22-25 vs 29-36 us at 192 / 256 rows; 14336 x 4096:
  // 22-29 vs 30-35 us at 64 / 128 rows); up to one per CU the skinny kernel
  // is (4096 x 4096 at 64 / 128 rows: 15.6 / 17.5 vs 20-23 us)
  // (GQ_GEMM_SKINNY=2: up to two per CU, for tuning)
  const size_t lim = (nckp >= 16 || (e && e[0] == '2')) ? 2 * cus : cus;
  if (!q6 && wgs > lim) return GQ_ERR_UNSUPPORTED;
  *ct_out = ct;
  *nck_out = nckp;
  return GQ_OK;
}

namespace {
template <int FMT, int CT, bool CBF16>
int launch_sk(const void *packed, const _Float16 *a16, int lda, void *c, const float *rs, int M, int N, int K,
              int nck, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K);
  const dim3 grid((unsigned)((gq_tiles(N) + CT - 1) / CT), (unsigned)((M + 63) / 64));
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const uint8_t *w = (const uint8_t *)packed;
  if (nck > 16) {  // 16-wave variant (4-bit formats, one row tile, 32-row blocks)
    if constexpr (CT == 1 && (FMT == GQ_FMT_Q4_0 || FMT == GQ_FMT_Q4_K)) {
      const dim3 g2((unsigned)gq_tiles(N), (unsigned)((M + 31) / 32));
      if (nck == 20)
        hipLaunchKernelGGL((k_gemm_sk<FMT, 1, 4, CBF16, 16, 2>), g2, dim3(1024), 0, s, w, sc_off, a16, lda, c, rs, M, N,
                           C, K);
      else if constexpr (FMT == GQ_FMT_Q4_0)
        hipLaunchKernelGGL((k_gemm_sk<FMT, 1, 8, CBF16, 16, 2>), g2, dim3(1024), 0, s, w, sc_off, a16, lda, c, rs, M, N,
                           C, K);
      else
        return GQ_ERR_UNSUPPORTED;
      return gq_last_launch();
    }
    return GQ_ERR_UNSUPPORTED;
  }
  if (nck <= 1)
    hipLaunchKernelGGL((k_gemm_sk<FMT, CT, 1, CBF16>), grid, dim3(512), 0, s, w, sc_off, a16, lda, c, rs, M, N, C, K);
  else if (nck <= 2)
    hipLaunchKernelGGL((k_gemm_sk<FMT, CT, 2, CBF16>), grid, dim3(512), 0, s, w, sc_off, a16, lda, c, rs, M, N, C, K);
  else if constexpr (FMT != GQ_FMT_Q6_K)
    hipLaunchKernelGGL((k_gemm_sk<FMT, CT, 4, CBF16>), grid, dim3(512), 0, s, w, sc_off, a16, lda, c, rs, M, N, C, K);
  else
    return GQ_ERR_UNSUPPORTED;
  return gq_last_launch();
}
template <int FMT, bool CBF16>
int launch_sk_ct(const void *packed, const _Float16 *a16, int lda, void *c, const float *rs, int M, int N, int K, int ct,
                 int nck, hipStream_t s) {
  return ct == 2 ? launch_sk<FMT, 2, CBF16>(packed, a16, lda, c, rs, M, N, K, nck, s)
                 : launch_sk<FMT, 1, CBF16>(packed, a16, lda, c, rs, M, N, K, nck, s);
}
template <int FMT>
int launch_sk_fmt(const void *packed, const _Float16 *a16, int lda, void *c, const float *rs, int cbf16, int M, int N,
                  int K, int ct, int nck, hipStream_t s) {
  return cbf16 ? launch_sk_ct<FMT, true>(packed, a16, lda, c, rs, M, N, K, ct, nck, s)
               : launch_sk_ct<FMT, false>(packed, a16, lda, c, rs, M, N, K, ct, nck, s);
}
}  // namespace

int gq_launch_gemm_skinny(int fmt, const void *packed, const _Float16 *a16, int lda, void *c, const float *rs,
                          int cbf16, int M, int N, int K, hipStream_t s) {
  int ct = 1, nck = 1;
  GQ_TRY(gq_gemm_skinny_plan(fmt, (size_t)M, (size_t)N, (size_t)K, &ct, &nck));
  if (gq_fmt_is_q6k(fmt)) return launch_sk_fmt<GQ_FMT_Q6_K>(packed, a16, lda, c, rs, cbf16, M, N, K, ct, nck, s);
  switch (gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt) {
  case GQ_FMT_Q4_0: return launch_sk_fmt<GQ_FMT_Q4_0>(packed, a16, lda, c, rs, cbf16, M, N, K, ct, nck, s);
  case GQ_FMT_Q8_0: return launch_sk_fmt<GQ_FMT_Q8_0>(packed, a16, lda, c, rs, cbf16, M, N, K, ct, nck, s);
  default: return launch_sk_fmt<GQ_FMT_Q4_K>(packed, a16, lda, c, rs, cbf16, M, N, K, ct, nck, s);
  }
}
