// gq_device.h -- device helpers for CDNA4 (gfx950): fp16 decoding with the
// reference's semantics, nibble/byte -> fp16 operand construction and MFMA
// wrappers.  Wave64 throughout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gq_layout.h"

typedef _Float16 gq_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 gq_half2 __attribute__((ext_vector_type(2)));
typedef float gq_f4 __attribute__((ext_vector_type(4)));
typedef float gq_f16v __attribute__((ext_vector_type(16)));
typedef int gq_i4 __attribute__((ext_vector_type(4)));
typedef int gq_i16v __attribute__((ext_vector_type(16)));
typedef uint32_t gq_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t gq_u2 __attribute__((ext_vector_type(2)));

#define GQ_DEV static __device__ __forceinline__

// fp16 -> fp32 with the reference's semantics (weight_loader.cpp:91-110):
// finite values and infinities convert exactly (the hardware conversion keeps
// fp16 subnormals), every exponent-31 input becomes +-Inf (NaN payloads are
// dropped exactly as the reference does).
GQ_DEV float gq_h2f(uint32_t h16) {
  h16 &= 0xFFFFu;
  if ((h16 & 0x7C00u) == 0x7C00u)
    return __uint_as_float(((h16 & 0x8000u) << 16) | 0x7F800000u);
  _Float16 hv = __builtin_bit_cast(_Float16, (uint16_t)h16);
  return (float)hv;
}
// Same, for a scale that only feeds a GEMV/GEMM: the NaN->Inf rule is kept so
// results match the reference semantics on every input.
GQ_DEV float gq_scale_h2f(uint32_t h16) { return gq_h2f(h16); }

GQ_DEV uint32_t gq_h2_bits(gq_half2 v) { return __builtin_bit_cast(uint32_t, v); }
GQ_DEV gq_half2 gq_bits_h2(uint32_t v) { return __builtin_bit_cast(gq_half2, v); }

// Canonical Q4 word -> 4 fp16 pairs holding (q - bias) for elements (2s, 2s+1),
// s = 0..3.  (0x6400 | q) is the fp16 value 1024 + q; one packed subtract of
// (1024 + bias) leaves the small integer exactly.
template <int BIAS>
GQ_DEV void gq_q4word_to_h8(uint32_t w, gq_half8 &out) {
  const gq_half2 off = {(_Float16)(-(1024.0f + BIAS)), (_Float16)(-(1024.0f + BIAS))};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    uint32_t t = ((w >> (4 * s)) & 0x000F000Fu) | 0x64006400u;
    gq_half2 h = gq_bits_h2(t) + off;
    out[2 * s] = h[0];
    out[2 * s + 1] = h[1];
  }
}

// Canonical Q4 word -> fp16 pairs of sc * q (0 <= q <= 15, 0 <= sc <= 63), exact:
// fma((1024+q), sc, -1024*sc) is computed exactly and the result (<= 945) is an
// fp16 integer.  sc2 = (sc, sc), nsc2 = (-1024 sc, -1024 sc).
GQ_DEV void gq_q4word_scaled_h8(uint32_t w, gq_half2 sc2, gq_half2 nsc2, gq_half8 &out) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    uint32_t t = ((w >> (4 * s)) & 0x000F000Fu) | 0x64006400u;
    gq_half2 h = __builtin_elementwise_fma(gq_bits_h2(t), sc2, nsc2);
    out[2 * s] = h[0];
    out[2 * s + 1] = h[1];
  }
}

// 8 int8 (two little-endian words) -> 8 exact fp16 values.  (q ^ 0x80) is q+128
// in [0,255]; placing it under an 0x64 high byte gives 1024 + q + 128.
GQ_DEV void gq_i8x8_to_h8(uint32_t w0, uint32_t w1, gq_half8 &out) {
  const gq_half2 off = {(_Float16)(-1152.0f), (_Float16)(-1152.0f)};
  uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
  uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u);
  uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u);
  uint32_t p2 = __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u);
  uint32_t p3 = __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u);
  gq_half2 h0 = gq_bits_h2(p0) + off, h1 = gq_bits_h2(p1) + off;
  gq_half2 h2 = gq_bits_h2(p2) + off, h3 = gq_bits_h2(p3) + off;
  out[0] = h0[0]; out[1] = h0[1]; out[2] = h1[0]; out[3] = h1[1];
  out[4] = h2[0]; out[5] = h2[1]; out[6] = h3[0]; out[7] = h3[1];
}

GQ_DEV gq_f4 gq_mfma16(const gq_half8 &a, const gq_half8 &b, const gq_f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
GQ_DEV gq_f16v gq_mfma32(const gq_half8 &a, const gq_half8 &b, const gq_f16v &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Q4_K scale/min codes for sub-blocks 2g and 2g+1 from the repacked meta words.
GQ_DEV void gq_q4k_codes(uint32_t W1, uint32_t W2, uint32_t W3, int g, uint32_t &sc0,
                         uint32_t &m0, uint32_t &sc1, uint32_t &m1) {
  uint32_t b1 = (W1 >> (8 * g)) & 0xFFu, b2 = (W2 >> (8 * g)) & 0xFFu,
           b3 = (W3 >> (8 * g)) & 0xFFu;
  sc0 = b1 & 63u;
  sc1 = b2 & 63u;
  m0 = (b1 >> 6) | ((b3 & 15u) << 2);
  m1 = (b2 >> 6) | ((b3 >> 4) << 2);
}

GQ_DEV gq_u4 gq_ld16(const void *p) { return *reinterpret_cast<const gq_u4 *>(p); }
GQ_DEV gq_u2 gq_ld8(const void *p) { return *reinterpret_cast<const gq_u2 *>(p); }
