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

// A T16 "code group": the 16 codes of 16 consecutive elements of a block packed
// into 8 bytes.  Byte b holds slot 8*(b>>2) + (b&3) in its low nibble and
// slot 8*(b>>2) + (b&3) + 4 in its high nibble, so that with the two words w0,
// w1 of the group
//   w0 & 0x0F0F0F0F, (w0 >> 4) & 0x0F0F0F0F, w1 & 0x0F0F0F0F, (w1 >> 4) & 0x0F0F0F0F
// are the 16 codes as bytes in slot order (an int8 MFMA operand).
GQ_HD uint64_t gq_pack_codes16(const uint8_t codes[16]) {
  uint64_t v = 0;
  for (int b = 0; b < 8; ++b) {
    int s = 8 * (b >> 2) + (b & 3);
    v |= (uint64_t)((codes[s] & 15u) | ((codes[s + 4] & 15u) << 4)) << (8 * b);
  }
  return v;
}
GQ_HD void gq_unpack_codes16(uint64_t v, uint8_t codes[16]) {
  for (int b = 0; b < 8; ++b) {
    int s = 8 * (b >> 2) + (b & 3);
    uint32_t byte = (uint32_t)(v >> (8 * b)) & 0xFFu;
    codes[s] = (uint8_t)(byte & 15u);
    codes[s + 4] = (uint8_t)(byte >> 4);
  }
}

// ---- Q4_0 ----------------------------------------------------------------
// GGUF Q4_0: byte j holds element j (low nibble) and element j+16 (high).
GQ_HD uint32_t gq_q4_0_code(const uint8_t *blk, int e) {
  const uint8_t *qs = blk + 2;
  return e < 16 ? (qs[e] & 15u) : (qs[e - 16] >> 4);
}
// GGUF Q4_0 block -> the two code groups (elements 0..15, 16..31) and d.
GQ_HD void gq_q4_0_groups(const uint8_t *blk, uint64_t grp[2], uint32_t *d16) {
  *d16 = gq_rd16(blk);
  for (int eh = 0; eh < 2; ++eh) {
    uint8_t c[16];
    for (int s = 0; s < 16; ++s) c[s] = (uint8_t)gq_q4_0_code(blk, 16 * eh + s);
    grp[eh] = gq_pack_codes16(c);
  }
}
GQ_HD void gq_q4_0_from_groups(const uint64_t grp[2], uint32_t d16, uint8_t *blk) {
  blk[0] = (uint8_t)(d16 & 0xFF);
  blk[1] = (uint8_t)(d16 >> 8);
  uint8_t q[32];
  gq_unpack_codes16(grp[0], q);
  gq_unpack_codes16(grp[1], q + 16);
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
// GGUF Q4_K super-block -> 16 code groups (sub-block j, half eh -> grp[2j+eh])
// and the 16-byte meta record (d | dmin | W1 | W2 | W3):
//   byte i of W1 = sc[2i]   | (m[2i]   & 3) << 6
//   byte i of W2 = sc[2i+1] | (m[2i+1] & 3) << 6
//   byte i of W3 = (m[2i] >> 2) | (m[2i+1] >> 2) << 4
GQ_HD void gq_q4k_groups(int ggml, const uint8_t *blk, uint64_t grp[16], uint32_t meta[4]) {
  uint8_t sc[8], m[8];
  if (ggml) gq_q4k_ggml_codes(blk + 4, sc, m);
  else gq_q4k_ref_codes(blk + 4, sc, m);
  const uint8_t *qs = blk + 16;
  for (int j = 0; j < 8; ++j)
    for (int eh = 0; eh < 2; ++eh) {
      uint8_t c[16];
      for (int s2 = 0; s2 < 16; ++s2) c[s2] = (uint8_t)gq_q4k_nib(ggml, qs, j, 16 * eh + s2);
      grp[2 * j + eh] = gq_pack_codes16(c);
    }
  meta[0] = gq_rd16(blk) | (gq_rd16(blk + 2) << 16);
  uint32_t W1 = 0, W2 = 0, W3 = 0;
  for (int i = 0; i < 4; ++i) {
    uint32_t s0 = sc[2 * i], s1 = sc[2 * i + 1], m0 = m[2 * i], m1 = m[2 * i + 1];
    W1 |= (s0 | ((m0 & 3u) << 6)) << (8 * i);
    W2 |= (s1 | ((m1 & 3u) << 6)) << (8 * i);
    W3 |= ((m0 >> 2) | ((m1 >> 2) << 4)) << (8 * i);
  }
  meta[1] = W1;
  meta[2] = W2;
  meta[3] = W3;
}
// codes of sub-block j from the meta words
GQ_HD void gq_q4k_meta_codes(const uint32_t meta[4], int j, uint32_t *sc, uint32_t *mn) {
  int i = j >> 1;
  uint32_t b = ((j & 1) ? meta[2] : meta[1]) >> (8 * i) & 0xFFu;
  uint32_t b3 = (meta[3] >> (8 * i)) & 0xFFu;
  *sc = b & 63u;
  *mn = (b >> 6) | ((((j & 1) ? (b3 >> 4) : b3) & 15u) << 2);
}
GQ_HD void gq_q4k_from_groups(int ggml, const uint64_t grp[16], const uint32_t meta[4], uint8_t *blk) {
  uint8_t sc[8], m[8];
  for (int j = 0; j < 8; ++j) {
    uint32_t a, b;
    gq_q4k_meta_codes(meta, j, &a, &b);
    sc[j] = (uint8_t)a;
    m[j] = (uint8_t)b;
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
    for (int eh = 0; eh < 2; ++eh) {
      uint8_t c[16];
      gq_unpack_codes16(grp[2 * j + eh], c);
      for (int s2 = 0; s2 < 16; ++s2) gq_q4k_set_nib(ggml, qs, j, 16 * eh + s2, c[s2]);
    }
}

// ---- Q6_K ----------------------------------------------------------------
// Block: ql[128] | qh[64] | int8 scales[16] | fp16 d; code c = low 4 | high 2 << 4,
// value (d * (c - 32)) * scales[i / 16] (scales in element order in both layouts).
// Reference (GRETA) layout, weight_loader.cpp:158-177: element i takes its low
// bits from ql[i/2] (nibble i%2) and its high bits from qh[i/4] (pair i%4).
// llama.cpp layout (dequantize_row_q6_K): per 128-element half h, l in 0..31,
// elements 128h + 32k + l take ql[64h + l + 32 (k & 1)] (nibble k >> 1) and
// qh[32h + l] (pair k).
GQ_HD void gq_q6k_locate(int ggml, int i, int *li, int *ls, int *hi, int *hs) {
  if (!ggml) {
    *li = i >> 1;
    *ls = 4 * (i & 1);
    *hi = 128 + (i >> 2);
    *hs = 2 * (i & 3);
  } else {
    const int h = i >> 7, k = (i >> 5) & 3, l = i & 31;
    *li = 64 * h + l + 32 * (k & 1);
    *ls = 4 * (k >> 1);
    *hi = 128 + 32 * h + l;
    *hs = 2 * k;
  }
}
GQ_HD uint32_t gq_q6k_code(int ggml, const uint8_t *blk, int i) {
  int li, ls, hi, hs;
  gq_q6k_locate(ggml, i, &li, &ls, &hi, &hs);
  return ((blk[li] >> ls) & 15u) | (((blk[hi] >> hs) & 3u) << 4);
}
GQ_HD void gq_q6k_set_code(int ggml, uint8_t *blk, int i, uint32_t c) {
  int li, ls, hi, hs;
  gq_q6k_locate(ggml, i, &li, &ls, &hi, &hs);
  blk[li] = (uint8_t)((blk[li] & ~(15u << ls)) | ((c & 15u) << ls));
  blk[hi] = (uint8_t)((blk[hi] & ~(3u << hs)) | (((c >> 4) & 3u) << hs));
}
// The 16 high 2-bit fields of a lane's 16 slots as one word: byte b holds slot
// 4q + b at bits 2q .. 2q+1.
GQ_HD uint32_t gq_q6k_pack_hi(const uint8_t codes[16]) {
  uint32_t w = 0;
  for (int s = 0; s < 16; ++s) w |= (uint32_t)((codes[s] >> 4) & 3u) << (8 * (s & 3) + 2 * (s >> 2));
  return w;
}
GQ_HD uint32_t gq_q6k_hi_of(uint32_t w, int s) { return (w >> (8 * (s & 3) + 2 * (s >> 2))) & 3u; }

// ---- addressing in the T16 layout ---------------------------------------
// Within a chunk of a 16-row tile, lane l = 16*g + r (row r) holds, for the
// int8 MFMA pair m, the 16 elements 16*(g&1) .. +15 of (sub-)block 2m + (g>>1).
//
// Q4_0: byte offset (qs plane) of the code group (element half eh) of 32-block
// `blk` of row n; 8 bytes.
GQ_HD size_t gq_q4_0_grp_off(size_t n, size_t blk, int eh, size_t C) {
  size_t t = n >> 4, r = n & 15, c = blk >> 2, j = blk & 3;
  size_t m = j >> 1, g = 2 * (j & 1) + (size_t)eh;
  return ((t * C + c) << 10) + 16 * (16 * g + r) + 8 * m;
}
// d of 32-block blk of row n (Q4_0 and Q8_0).  Per row and chunk the four d
// are stored in the order (d0, d2, d1, d3): lane (g, r) reads the 4 bytes at
// 4*(g>>1), the d of its blocks (g>>1) and 2 + (g>>1).
GQ_HD size_t gq_q4_0_d_off(size_t n, size_t blk, size_t C) {
  size_t t = n >> 4, r = n & 15, c = blk >> 2, j = blk & 3;
  return (t * C + c) * 128 + r * 8 + 4 * (j & 1) + 2 * (j >> 1);
}
// Q8_0: byte offset of the 16 int8 elements 16*eh .. +15 of 32-block blk.
GQ_HD size_t gq_q8_0_half_off(size_t n, size_t blk, int eh, size_t C) {
  size_t t = n >> 4, r = n & 15, c = blk >> 2, j = blk & 3;
  size_t m = j >> 1, g = 2 * (j & 1) + (size_t)eh;
  return ((t * C + c) << 11) + (m << 10) + 16 * (16 * g + r);
}
// Q4_K: code group (sub-block j, half eh) of super-block s of row n; 8 bytes.
GQ_HD size_t gq_q4k_grp_off(size_t n, size_t s, int j, int eh, size_t S) {
  size_t t = n >> 4, r = n & 15;
  size_t m = (size_t)j >> 1, g = 2 * ((size_t)j & 1) + (size_t)eh;
  return ((t * S + s) << 11) + ((m >> 1) << 10) + 16 * (16 * g + r) + 8 * (m & 1);
}
GQ_HD size_t gq_q4k_meta_off(size_t n, size_t s, size_t S) {
  size_t t = n >> 4, r = n & 15;
  return (t * S + s) * 256 + 16 * r;
}
// Q6_K: code group of the low nibbles (sub-block j, half eh) of super-block s
// of row n (8 bytes), the high-bit word of the same 16 slots (4 bytes), and
// the row's scales (16 bytes) and d (2 bytes) in the scale plane.
GQ_HD size_t gq_q6k_grp_off(size_t n, size_t s, int j, int eh, size_t S) {
  size_t t = n >> 4, r = n & 15;
  size_t m = (size_t)j >> 1, g = 2 * ((size_t)j & 1) + (size_t)eh;
  return (t * S + s) * 3072 + ((m >> 1) << 10) + 16 * (16 * g + r) + 8 * (m & 1);
}
GQ_HD size_t gq_q6k_hi_off(size_t n, size_t s, int j, int eh, size_t S) {
  size_t t = n >> 4, r = n & 15;
  size_t m = (size_t)j >> 1, g = 2 * ((size_t)j & 1) + (size_t)eh;
  return (t * S + s) * 3072 + 2048 + 16 * (16 * g + r) + 4 * m;
}
GQ_HD size_t gq_q6k_sc_off(size_t n, size_t s, size_t S) {
  size_t t = n >> 4, r = n & 15;
  return (t * S + s) * 288 + 16 * r;
}
GQ_HD size_t gq_q6k_d_off(size_t n, size_t s, size_t S) {
  size_t t = n >> 4, r = n & 15;
  return (t * S + s) * 288 + 256 + 2 * r;
}
// GGUF Q6_K super-block of row n -> its T16 places (packed: the whole tensor,
// sc: its scale plane).  Writes every byte it owns, zeros for a null block.
GQ_HD void gq_q6k_put(int ggml, const uint8_t *blk, uint8_t *packed, uint8_t *sc, size_t n, size_t s, size_t S) {
  for (int j = 0; j < 8; ++j)
    for (int eh = 0; eh < 2; ++eh) {
      uint8_t c[16];
      for (int e = 0; e < 16; ++e) c[e] = blk ? (uint8_t)gq_q6k_code(ggml, blk, 32 * j + 16 * eh + e) : 0;
      const uint64_t g = gq_pack_codes16(c);
      uint8_t *gp = packed + gq_q6k_grp_off(n, s, j, eh, S);
      for (int b = 0; b < 8; ++b) gp[b] = (uint8_t)(g >> (8 * b));
      const uint32_t h = gq_q6k_pack_hi(c);
      uint8_t *hp = packed + gq_q6k_hi_off(n, s, j, eh, S);
      for (int b = 0; b < 4; ++b) hp[b] = (uint8_t)(h >> (8 * b));
    }
  uint8_t *sp = sc + gq_q6k_sc_off(n, s, S);
  for (int i = 0; i < 16; ++i) sp[i] = blk ? blk[192 + i] : 0;
  uint8_t *dp = sc + gq_q6k_d_off(n, s, S);
  dp[0] = blk ? blk[208] : 0;
  dp[1] = blk ? blk[209] : 0;
}
// T16 -> GGUF Q6_K super-block (inverse of gq_q6k_put)
GQ_HD void gq_q6k_get(int ggml, const uint8_t *packed, const uint8_t *sc, size_t n, size_t s, size_t S, uint8_t *blk) {
  for (int i = 0; i < 210; ++i) blk[i] = 0;
  for (int j = 0; j < 8; ++j)
    for (int eh = 0; eh < 2; ++eh) {
      const uint8_t *gp = packed + gq_q6k_grp_off(n, s, j, eh, S);
      uint64_t g = 0;
      for (int b = 0; b < 8; ++b) g |= (uint64_t)gp[b] << (8 * b);
      const uint8_t *hp = packed + gq_q6k_hi_off(n, s, j, eh, S);
      const uint32_t h = (uint32_t)hp[0] | ((uint32_t)hp[1] << 8) | ((uint32_t)hp[2] << 16) | ((uint32_t)hp[3] << 24);
      uint8_t c[16];
      gq_unpack_codes16(g, c);
      for (int e = 0; e < 16; ++e) gq_q6k_set_code(ggml, blk, 32 * j + 16 * eh + e, c[e] | (gq_q6k_hi_of(h, e) << 4));
    }
  const uint8_t *sp = sc + gq_q6k_sc_off(n, s, S);
  for (int i = 0; i < 16; ++i) blk[192 + i] = sp[i];
  const uint8_t *dp = sc + gq_q6k_d_off(n, s, S);
  blk[208] = dp[0];
  blk[209] = dp[1];
}
