// gq_repack_impl.h -- one implementation of GGUF block <-> T16 canonical form,
// compiled for both host (load-time repack on the CPU) and device (repack
// kernel).  The layout itself is specified in gq_layout.h.
#pragma once
#include <stdint.h>

#include "gq_layout.h"

#if defined(__HIPCC__)
#define GQ_HD __host__ __device__ inline
#else
#define GQ_HD inline
#endif

GQ_HD uint32_t gq_rd16(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

// Build the canonical word for elements 8*w8 .. 8*w8+7 of a 32-element block
// whose element e has 4-bit value nib(e).
template <typename NibFn>
GQ_HD uint32_t gq_canon_word(int w8, NibFn nib) {
  uint32_t w = 0;
  for (int i = 0; i < 8; ++i)
    w |= (uint32_t)(nib(8 * w8 + i) & 15u) << (4 * gq_canon_pos(i));
  return w;
}

// ---- Q4_0 ----------------------------------------------------------------
// GGUF Q4_0: byte j holds element j (low nibble) and element j+16 (high).
GQ_HD void gq_q4_0_canon(const uint8_t *blk, uint32_t words[4], uint32_t *d16) {
  const uint8_t *qs = blk + 2;
  *d16 = gq_rd16(blk);
  for (int w8 = 0; w8 < 4; ++w8)
    words[w8] = gq_canon_word(w8, [&](int e) -> uint32_t {
      return e < 16 ? (qs[e] & 15u) : (qs[e - 16] >> 4);
    });
}
GQ_HD void gq_q4_0_uncanon(const uint32_t words[4], uint32_t d16, uint8_t *blk) {
  blk[0] = (uint8_t)(d16 & 0xFF);
  blk[1] = (uint8_t)(d16 >> 8);
  uint8_t q[32];
  for (int w8 = 0; w8 < 4; ++w8)
    for (int i = 0; i < 8; ++i) q[8 * w8 + i] = (words[w8] >> (4 * gq_canon_pos(i))) & 15u;
  for (int j = 0; j < 16; ++j) blk[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
}

// ---- Q4_K ----------------------------------------------------------------
// Reference (GRETA) layout, weight_loader.cpp:125-156.
GQ_HD void gq_q4k_ref_codes(const uint8_t *s, uint8_t sc[8], uint8_t m[8]) {
  for (int j = 0; j < 4; ++j) {
    sc[j] = s[j] & 63;
    m[j] = s[6 + j] & 63;
  }
  sc[4] = (uint8_t)((s[0] >> 6) | ((s[4] & 15) << 2));
  sc[5] = (uint8_t)((s[1] >> 6) | ((s[4] >> 4) << 2));
  sc[6] = (uint8_t)((s[2] >> 6) | ((s[5] & 15) << 2));
  sc[7] = (uint8_t)((s[3] >> 6) | ((s[5] >> 4) << 2));
  m[4] = (uint8_t)((s[6] >> 6) | ((s[10] & 15) << 2));
  m[5] = (uint8_t)((s[7] >> 6) | ((s[10] >> 4) << 2));
  m[6] = (uint8_t)((s[8] >> 6) | ((s[11] & 15) << 2));
  m[7] = (uint8_t)((s[9] >> 6) | ((s[11] >> 4) << 2));
}
GQ_HD void gq_q4k_ref_pack_codes(const uint8_t sc[8], const uint8_t m[8], uint8_t *s) {
  for (int j = 0; j < 4; ++j) {
    s[j] = (uint8_t)(sc[j] | ((sc[4 + j] & 3) << 6));
    s[6 + j] = (uint8_t)(m[j] | ((m[4 + j] & 3) << 6));
  }
  s[4] = (uint8_t)((sc[4] >> 2) | ((sc[5] >> 2) << 4));
  s[5] = (uint8_t)((sc[6] >> 2) | ((sc[7] >> 2) << 4));
  s[10] = (uint8_t)((m[4] >> 2) | ((m[5] >> 2) << 4));
  s[11] = (uint8_t)((m[6] >> 2) | ((m[7] >> 2) << 4));
}
// llama.cpp canonical layout (get_scale_min_k4 in ggml-quants.c).
GQ_HD void gq_q4k_ggml_codes(const uint8_t *q, uint8_t sc[8], uint8_t m[8]) {
  for (int j = 0; j < 8; ++j) {
    if (j < 4) {
      sc[j] = q[j] & 63;
      m[j] = q[j + 4] & 63;
    } else {
      sc[j] = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
      m[j] = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
  }
}
GQ_HD void gq_q4k_ggml_pack_codes(const uint8_t sc[8], const uint8_t m[8], uint8_t *q) {
  for (int j = 0; j < 4; ++j) {
    q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
    q[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
    q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
  }
}
// 4-bit value of element e (0..31) of sub-block j (0..7).
GQ_HD uint32_t gq_q4k_nib(int ggml, const uint8_t *qs, int j, int e) {
  if (!ggml) {  // reference: sub-block j = qs[16j..16j+15], byte l -> (2l lo, 2l+1 hi)
    uint8_t b = qs[16 * j + (e >> 1)];
    return (e & 1) ? (b >> 4) : (b & 15u);
  }
  // ggml: pair p = j/2 shares qs[32p..32p+31]; even j low nibbles, odd j high
  uint8_t b = qs[32 * (j >> 1) + e];
  return (j & 1) ? (b >> 4) : (b & 15u);
}
GQ_HD void gq_q4k_set_nib(int ggml, uint8_t *qs, int j, int e, uint32_t v) {
  if (!ggml) {
    uint8_t *b = &qs[16 * j + (e >> 1)];
    *b = (e & 1) ? (uint8_t)((*b & 0x0F) | (v << 4)) : (uint8_t)((*b & 0xF0) | v);
  } else {
    uint8_t *b = &qs[32 * (j >> 1) + e];
    *b = (j & 1) ? (uint8_t)((*b & 0x0F) | (v << 4)) : (uint8_t)((*b & 0xF0) | v);
  }
}
// GGUF Q4_K super-block -> canonical: words[8][4] (sub-block j, word w8) and
// the 16-byte meta record (d | dmin | W1 | W2 | W3).
GQ_HD void gq_q4k_canon(int ggml, const uint8_t *blk, uint32_t words[8][4], uint32_t meta[4]) {
  uint8_t sc[8], m[8];
  if (ggml) gq_q4k_ggml_codes(blk + 4, sc, m);
  else gq_q4k_ref_codes(blk + 4, sc, m);
  const uint8_t *qs = blk + 16;
  for (int j = 0; j < 8; ++j)
    for (int w8 = 0; w8 < 4; ++w8)
      words[j][w8] = gq_canon_word(w8, [&](int e) -> uint32_t { return gq_q4k_nib(ggml, qs, j, e); });
  meta[0] = gq_rd16(blk) | (gq_rd16(blk + 2) << 16);
  uint32_t W1 = 0, W2 = 0, W3 = 0;
  for (int g = 0; g < 4; ++g) {
    uint32_t s0 = sc[2 * g], s1 = sc[2 * g + 1], m0 = m[2 * g], m1 = m[2 * g + 1];
    W1 |= (s0 | ((m0 & 3u) << 6)) << (8 * g);
    W2 |= (s1 | ((m1 & 3u) << 6)) << (8 * g);
    W3 |= ((m0 >> 2) | ((m1 >> 2) << 4)) << (8 * g);
  }
  meta[1] = W1;
  meta[2] = W2;
  meta[3] = W3;
}
GQ_HD void gq_q4k_uncanon(int ggml, const uint32_t words[8][4], const uint32_t meta[4], uint8_t *blk) {
  uint8_t sc[8], m[8];
  for (int g = 0; g < 4; ++g) {
    uint32_t b1 = (meta[1] >> (8 * g)) & 0xFF, b2 = (meta[2] >> (8 * g)) & 0xFF,
             b3 = (meta[3] >> (8 * g)) & 0xFF;
    sc[2 * g] = (uint8_t)(b1 & 63);
    sc[2 * g + 1] = (uint8_t)(b2 & 63);
    m[2 * g] = (uint8_t)((b1 >> 6) | ((b3 & 15) << 2));
    m[2 * g + 1] = (uint8_t)((b2 >> 6) | ((b3 >> 4) << 2));
  }
  blk[0] = (uint8_t)(meta[0] & 0xFF);
  blk[1] = (uint8_t)((meta[0] >> 8) & 0xFF);
  blk[2] = (uint8_t)((meta[0] >> 16) & 0xFF);
  blk[3] = (uint8_t)(meta[0] >> 24);
  if (ggml) gq_q4k_ggml_pack_codes(sc, m, blk + 4);
  else gq_q4k_ref_pack_codes(sc, m, blk + 4);
  uint8_t *qs = blk + 16;
  for (int i = 0; i < 128; ++i) qs[i] = 0;
  for (int j = 0; j < 8; ++j)
    for (int w8 = 0; w8 < 4; ++w8)
      for (int i = 0; i < 8; ++i)
        gq_q4k_set_nib(ggml, qs, j, 8 * w8 + i, (words[j][w8] >> (4 * gq_canon_pos(i))) & 15u);
}

// ---- addressing in the T16 layout ---------------------------------------
// Byte offset, within the qs plane, of the 4-byte word holding canonical word
// `w8` of block `blk` (Q4_0: 32-block index; Q4_K: sub-block index) of row n.
GQ_HD size_t gq_q4_0_word_off(size_t n, size_t blk, int w8, size_t C) {
  size_t t = n >> 4, r = n & 15, c = blk >> 2, j = blk & 3;
  return ((t * C + c) << 10) + 16 * (16 * (size_t)w8 + r) + 4 * j;
}
GQ_HD size_t gq_q4_0_d_off(size_t n, size_t blk, size_t C) {
  size_t t = n >> 4, r = n & 15, c = blk >> 2, j = blk & 3;
  return (t * C + c) * 128 + (r * 4 + j) * 2;
}
// Q8_0: byte `b` (0..31) of 32-block `blk` of row n.
GQ_HD size_t gq_q8_0_byte_off(size_t n, size_t blk, int b, size_t C) {
  size_t t = n >> 4, r = n & 15, c = blk >> 2, j = blk & 3;
  size_t p = j >> 1, half = j & 1;
  size_t g = (size_t)b >> 3, within = (size_t)b & 7;
  return ((t * C + c) << 11) + (p << 10) + 16 * (16 * g + r) + 8 * half + within;
}
// Q4_K: canonical word w8 of sub-block j of super-block s of row n.
GQ_HD size_t gq_q4k_word_off(size_t n, size_t s, int j, int w8, size_t S) {
  size_t t = n >> 4, r = n & 15;
  size_t g = (size_t)j >> 1, h = (size_t)j & 1;
  return ((t * S + s) << 11) + (h << 10) + 16 * (16 * g + r) + 4 * (size_t)w8;
}
GQ_HD size_t gq_q4k_meta_off(size_t n, size_t s, size_t S) {
  size_t t = n >> 4, r = n & 15;
  return (t * S + s) * 256 + 16 * r;
}
