// gq_gemv_i8.h -- device pieces of the int8-MFMA decode GEMV shared by the
// single-launch kernels (gq_gemv.hip) and the chained decode kernel
// (gq_chain.hip): the T16 chunk records of each format, their loads, the
// code-group extraction, and the two-limb activation split.
#pragma once
#include "gq_internal.h"

namespace {

template <int FMT>
struct Fmt;
template <>
struct Fmt<GQ_FMT_Q4_0> {
  static constexpr int CK = 128, QB = 1024, SB = 128, MAXC = 8, STEPS = 2;
};
template <>
struct Fmt<GQ_FMT_Q8_0> {
  static constexpr int CK = 128, QB = 2048, SB = 128, MAXC = 8, STEPS = 2;
};
template <>
struct Fmt<GQ_FMT_Q4_K> {
  static constexpr int CK = 256, QB = 2048, SB = 256, MAXC = 4, STEPS = 4;
};
template <>
struct Fmt<GQ_FMT_Q6_K> {
  static constexpr int CK = 256, QB = 3072, SB = 288, MAXC = 4, STEPS = 4;
};

// weight registers of one chunk (one row tile)
template <int FMT>
struct Chunk;
template <>
struct Chunk<GQ_FMT_Q4_0> {
  gq_u4 q;      // steps 0, 1: 8-byte code groups
  uint32_t d;   // (d of block h', d of block 2 + h') for this lane
};
template <>
struct Chunk<GQ_FMT_Q8_0> {
  gq_u4 q0, q1;  // steps 0, 1: 16 int8
  uint32_t d;
};
template <>
struct Chunk<GQ_FMT_Q4_K> {
  gq_u4 qa, qb;  // steps 0,1 and 2,3
  gq_u4 meta;    // d, dmin, W1, W2, W3 of this lane's row
};
template <>
struct Chunk<GQ_FMT_Q6_K> {
  gq_u4 qa, qb;  // low-nibble code groups, steps 0,1 and 2,3
  gq_u4 hi;      // high 2-bit fields, one word per step
  gq_u4 sc;      // the row's 16 int8 scales
  uint32_t d;    // the row's fp16 d (low half)
};

// qp / sp: wave-uniform chunk bases; qo / so: this lane's 32-bit offsets
template <int FMT>
GQ_DEV void load_chunk(const uint8_t *qp, const uint8_t *sp, uint32_t qo, uint32_t so, Chunk<FMT> &ch) {
  if constexpr (FMT == GQ_FMT_Q4_0) {
    ch.q = gq_ld16_nt(qp + qo);
    ch.d = gq_ld4_nt(sp + so);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    ch.q0 = gq_ld16_nt(qp + qo);
    ch.q1 = gq_ld16_nt(qp + 1024 + qo);
    ch.d = gq_ld4_nt(sp + so);
  } else {
    if constexpr (FMT == GQ_FMT_Q4_K) {
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
}

// The code words of a chunk only (Q4_0, Q8_0, Q4_K): the scales come from an
// LDS copy of the wave's scale-plane run (gq_gemv.hip)
template <int FMT>
GQ_DEV void load_chunk_codes(const uint8_t *qp, uint32_t qo, Chunk<FMT> &ch) {
  if constexpr (FMT == GQ_FMT_Q4_0) {
    ch.q = gq_ld16_nt(qp + qo);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    ch.q0 = gq_ld16_nt(qp + qo);
    ch.q1 = gq_ld16_nt(qp + 1024 + qo);
  } else {
    static_assert(FMT == GQ_FMT_Q4_K, "Q4_0, Q8_0, Q4_K");
    ch.qa = gq_ld16_nt(qp + qo);
    ch.qb = gq_ld16_nt(qp + 1024 + qo);
  }
}

// code group (2 words) -> 16 codes as bytes, slot order
GQ_DEV gq_i4 codes16(uint32_t w0, uint32_t w1) {
  gq_i4 v;
  v[0] = (int)(w0 & 0x0F0F0F0Fu);
  v[1] = (int)((w0 >> 4) & 0x0F0F0F0Fu);
  v[2] = (int)(w1 & 0x0F0F0F0Fu);
  v[3] = (int)((w1 >> 4) & 0x0F0F0F0Fu);
  return v;
}

GQ_DEV gq_i4 mfma_i8(const gq_i4 &a, const gq_i4 &b) {
  const gq_i4 z = {0, 0, 0, 0};
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, z, 0, 0, 0);
}

GQ_DEV float h16lo(uint32_t v) { return (float)__builtin_bit_cast(gq_half2, v)[0]; }
GQ_DEV float h16hi(uint32_t v) { return (float)__builtin_bit_cast(gq_half2, v)[1]; }

// low byte of each of four floats, packed into one word
GQ_DEV uint32_t pack_lo_bytes(float f0, float f1, float f2, float f3) {
  const uint32_t p01 = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x00000400u);
  const uint32_t p23 = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x00000400u);
  return __builtin_amdgcn_perm(p23, p01, 0x05040100u);
}

// ---------------------------------------------------------------------------
// Activation limbs.  Per batch row b and limb l (0: a, 1: b) an int8 array of
// the slice, a zero region of the slice length, and per (b, 32-block) the
// float4 (s, S, s / 254, 0): the (scale, sum) pair of limb a then of limb b.
// ---------------------------------------------------------------------------
struct XlLayout {
  int lk, zero_off, scl_off, wave_bytes;
};
__host__ __device__ inline XlLayout xl_layout(int lk, int nb) {
  XlLayout L;
  L.lk = lk;
  L.zero_off = 2 * nb * lk;
  L.scl_off = L.zero_off + lk;
  L.wave_bytes = (L.scl_off + nb * (lk / 32) * 16 + 15) & ~15;
  return L;
}

constexpr float kMagic = 12582912.0f;  // 1.5 * 2^23: adding it rounds to an integer in the low mantissa bits

// Splits 8 consecutive elements into the two limbs (4 int8 per word) and
// returns sum(a) * 254 + sum(b) as an exact integer, so the block sum of the
// represented values is s / 254 times it.  a = round(v * inv) comes out of the
// low mantissa bits of fma(v, inv, 1.5 * 2^23); the remainder v * inv - a is
// formed by a second fma (exact), scaled by 254 and rounded the same way.  The
// limb sums are integer dot products of the packed bytes with ones.
GQ_DEV int split8(const float (&v)[8], float inv, uint32_t (&la)[2], uint32_t (&lb)[2]) {
  float fa[8], fb[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    fa[e] = __builtin_fmaf(v[e], inv, kMagic);  // bits: integer a in the low byte
    const float ai = fa[e] - kMagic;
    fb[e] = __builtin_fmaf(__builtin_fmaf(v[e], inv, -ai), 254.0f, kMagic);
  }
  la[0] = pack_lo_bytes(fa[0], fa[1], fa[2], fa[3]);
  la[1] = pack_lo_bytes(fa[4], fa[5], fa[6], fa[7]);
  lb[0] = pack_lo_bytes(fb[0], fb[1], fb[2], fb[3]);
  lb[1] = pack_lo_bytes(fb[4], fb[5], fb[6], fb[7]);
  constexpr int kOnes = 0x01010101;
  const int sa = __builtin_amdgcn_sdot4((int)la[1], kOnes, __builtin_amdgcn_sdot4((int)la[0], kOnes, 0, false), false);
  const int sb = __builtin_amdgcn_sdot4((int)lb[1], kOnes, __builtin_amdgcn_sdot4((int)lb[0], kOnes, 0, false), false);
  return 254 * sa + sb;
}

// Largest |v| of 8 elements as a bit pattern: the sign cleared, the patterns
// compare as unsigned integers in the order of the magnitudes, and a NaN
// (exponent all ones, mantissa nonzero) ranks above Inf, so a NaN or Inf in
// the block comes out as the block's maximum instead of being skipped the way
// fmaxf skips a NaN.
GQ_DEV uint32_t abs_max_bits8(const float (&v)[8]) {
  uint32_t m = 0u;
#pragma unroll
  for (int e = 0; e < 8; ++e) m = max(m, __float_as_uint(v[e]) & 0x7FFFFFFFu);
  return m;
}
// Quad-wide (lanes 4j .. 4j+3) max of such patterns / integer sum through DPP
// quad permutes.  The quad max returns the float the pattern encodes.
GQ_DEV float quad_max(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));  // lane ^ 1
  return __uint_as_float(max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false)));  // lane ^ 2
}
GQ_DEV int quad_sum(int v) {
  v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
  return v + __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
}
// Sum over the whole wave, every lane receiving it: quads (DPP lane ^ 1,
// lane ^ 2), then the mirrored quad of each 8-lane half (row_half_mirror) and
// the mirrored half of each 16-lane row (row_mirror), then the 16-lane groups
// (sum_lane_groups).
GQ_DEV float sum_lane_groups(float p);
GQ_DEV float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));
  return sum_lane_groups(v);
}
// Sum over the four 16-lane groups (lane, lane ^ 16, lane ^ 32, lane ^ 48):
// each permlane swap returns the pair (own, partner) in some order.
GQ_DEV float sum_lane_groups(float p) {
  const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(p), __float_as_uint(p), false, false);
  p = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
  const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(p), false, false);
  return __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
}

}  // namespace
