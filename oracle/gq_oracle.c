/*
 * gq_oracle.c -- CPU restatement of the reference's quantized-weight path.
 *
 * TEST INFRASTRUCTURE ONLY (see gq_oracle.h).  Compiled with
 * -ffp-contract=off so that every product / difference is rounded on its own,
 * exactly as the reference's x86-64 host build (no -mfma) evaluates them.
 * Reference paths are relative to the leaatimberini/gretacore-v3 tree.
 */
#include "gq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* src/inference/src/weight_loader.cpp:91-110: subnormals are normalised by a
 * shift loop; exponent 31 maps to +-Inf for every mantissa (NaN payloads are
 * NOT preserved -- that is the reference's behaviour). */
float gqo_fp16_to_fp32(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u;
  uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x3FFu;
  if (e == 31) return bits_to_f32((sign << 31) | 0x7F800000u);
  if (e == 0) {
    if (m == 0) return bits_to_f32(sign << 31);
    /* value = m * 2^-24; normalise so that bit 10 is the implicit one */
    int shift = 0;
    while ((m & 0x400u) == 0) {
      m <<= 1;
      shift++;
    }
    m &= 0x3FFu;
    uint32_t fe = (uint32_t)(113 - shift); /* 127 - 14 - shift */
    return bits_to_f32((sign << 31) | (fe << 23) | (m << 13));
  }
  return bits_to_f32((sign << 31) | ((e + 112u) << 23) | (m << 13));
}

/* src/rt/ref/cpu/include/gcore/rt/ref/cpu_reference.hpp:19-38: round to
 * nearest even; subnormal results are truncated; overflow -> Inf. */
uint16_t gqo_float_to_half(float f) {
  uint32_t x = f32_to_bits(f);
  uint32_t sign = (x >> 31) & 1u;
  int e = (int)((x >> 23) & 0xFFu) - 127;
  uint32_t m = x & 0x7FFFFFu;
  if (e > 15) return (uint16_t)((sign << 15) | 0x7C00u);
  if (e < -14) {
    if (e < -24) return (uint16_t)(sign << 15);
    m |= 0x800000u;
    int sh = -e - 14;
    return (uint16_t)((sign << 15) | (m >> (sh + 13)));
  }
  uint32_t eh = (uint32_t)(e + 15);
  uint32_t mh = m >> 13;
  uint32_t r = m & 0x1FFFu;
  if (r > 0x1000u || (r == 0x1000u && (mh & 1u))) mh++;
  if (mh == 0x400u) {
    mh = 0;
    eh++;
    if (eh >= 31) return (uint16_t)((sign << 15) | 0x7C00u);
  }
  return (uint16_t)((sign << 15) | (eh << 10) | mh);
}

/* src/inference/src/weight_loader.cpp:112-123 (truncating fp32->fp16 used by
 * load_tensor_fp16). */
uint16_t gqo_fp32_to_fp16_trunc(float f) {
  uint32_t x = f32_to_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  int32_t e = (int32_t)((x >> 23) & 0xFFu) - 127 + 15;
  uint32_t m = x & 0x7FFFFFu;
  if (e <= 0) return (uint16_t)sign;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
}

void gqo_fp16_to_fp32_n(const uint16_t *h, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) out[i] = gqo_fp16_to_fp32(h[i]);
}
void gqo_fp32_to_fp16_trunc_n(const float *f, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; ++i) out[i] = gqo_fp32_to_fp16_trunc(f[i]);
}

/* Block geometry, weight_loader.cpp:38-82. */
size_t gqo_block_elems(int fmt) {
  switch (fmt) {
  case GQO_F32:
  case GQO_F16:
    return 1;
  case GQO_Q4_0:
  case GQO_Q8_0:
    return 32;
  case GQO_Q4_K:
  case GQO_Q4_K_GGML:
  case GQO_Q6_K:
  case GQO_Q6_K_GGML:
    return 256;
  default:
    return 0;
  }
}
size_t gqo_block_bytes(int fmt) {
  switch (fmt) {
  case GQO_F32:
    return 4;
  case GQO_F16:
    return 2;
  case GQO_Q4_0:
    return 18;
  case GQO_Q8_0:
    return 34;
  case GQO_Q4_K:
  case GQO_Q4_K_GGML:
    return 144;
  case GQO_Q6_K:
  case GQO_Q6_K_GGML:
    return 210;
  default:
    return 0;
  }
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Q8_0: 2-byte fp16 d then 32 int8.  Intended reference semantics
 * weight_loader.cpp:703-712 + gemm_kernels.hip:612-616: w = (float)q * d. */
static void deq_q8_0(const uint8_t *b, float *y) {
  float d = gqo_fp16_to_fp32(rd16(b));
  const int8_t *q = (const int8_t *)(b + 2);
  for (int i = 0; i < 32; ++i) y[i] = (float)q[i] * d;
}

/* Q4_0 (GGUF spec; the reference only recognises the type,
 * weight_loader.cpp:18,44-45,67-68): byte j holds element j in its low nibble
 * and element j+16 in its high nibble; w = (q - 8) * d. */
static void deq_q4_0(const uint8_t *b, float *y) {
  float d = gqo_fp16_to_fp32(rd16(b));
  const uint8_t *qs = b + 2;
  for (int j = 0; j < 16; ++j) {
    y[j] = (float)((int)(qs[j] & 0x0F) - 8) * d;
    y[j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
  }
}

/* Q4_K, reference layout: weight_loader.cpp:84-89 (struct), :125-156 (math).
 * 6-bit scale codes: sc[0..3] = s[0..3] & 63, sc[4..7] = s[0..3]>>6 | nibble of
 * s[4..5] << 2 (low nibble first); mins the same from s[6..11].  Sub-block j uses
 * qs[16j..16j+15]; byte l gives element 2l (low nibble) and 2l+1 (high).  Each
 * product and the difference are rounded separately (no FMA). */
static void q4k_ref_codes(const uint8_t *s, uint8_t *sc, uint8_t *mn) {
  for (int j = 0; j < 4; ++j) {
    sc[j] = s[j] & 0x3F;
    mn[j] = s[6 + j] & 0x3F;
  }
  sc[4] = (uint8_t)((s[0] >> 6) | ((s[4] & 0x0F) << 2));
  sc[5] = (uint8_t)((s[1] >> 6) | ((s[4] >> 4) << 2));
  sc[6] = (uint8_t)((s[2] >> 6) | ((s[5] & 0x0F) << 2));
  sc[7] = (uint8_t)((s[3] >> 6) | ((s[5] >> 4) << 2));
  mn[4] = (uint8_t)((s[6] >> 6) | ((s[10] & 0x0F) << 2));
  mn[5] = (uint8_t)((s[7] >> 6) | ((s[10] >> 4) << 2));
  mn[6] = (uint8_t)((s[8] >> 6) | ((s[11] & 0x0F) << 2));
  mn[7] = (uint8_t)((s[9] >> 6) | ((s[11] >> 4) << 2));
}
static void deq_q4_k(const uint8_t *b, float *y) {
  float d = gqo_fp16_to_fp32(rd16(b));
  float dmin = gqo_fp16_to_fp32(rd16(b + 2));
  uint8_t sc[8], mn[8];
  q4k_ref_codes(b + 4, sc, mn);
  const uint8_t *qs = b + 16;
  for (int j = 0; j < 8; ++j) {
    volatile float scale = d * (float)sc[j];
    volatile float minv = dmin * (float)mn[j];
    for (int l = 0; l < 16; ++l) {
      uint8_t q = qs[16 * j + l];
      volatile float p0 = scale * (float)(q & 0x0F);
      volatile float p1 = scale * (float)(q >> 4);
      y[32 * j + 2 * l] = p0 - minv;
      y[32 * j + 2 * l + 1] = p1 - minv;
    }
  }
}

/* Q4_K, llama.cpp canonical layout (ggml-quants.c dequantize_row_q4_K and
 * get_scale_min_k4, restated from the published format): 64-element groups
 * share 32 qs bytes, low nibbles then high nibbles; codes j<4: q[j]&63 /
 * q[j+4]&63, j>=4: (q[j+4]&15)|(q[j-4]>>6)<<4 / (q[j+4]>>4)|(q[j]>>6)<<4. */
static void q4k_ggml_code(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
  if (j < 4) {
    *d = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}
static void deq_q4_k_ggml(const uint8_t *b, float *y) {
  float d = gqo_fp16_to_fp32(rd16(b));
  float dmin = gqo_fp16_to_fp32(rd16(b + 2));
  const uint8_t *sc = b + 4;
  const uint8_t *q = b + 16;
  int is = 0;
  for (int j = 0; j < 256; j += 64) {
    uint8_t s1, m1, s2, m2;
    q4k_ggml_code(is, sc, &s1, &m1);
    q4k_ggml_code(is + 1, sc, &s2, &m2);
    volatile float d1 = d * (float)s1, mm1 = dmin * (float)m1;
    volatile float d2 = d * (float)s2, mm2 = dmin * (float)m2;
    for (int l = 0; l < 32; ++l) {
      volatile float p = d1 * (float)(q[l] & 0x0F);
      y[j + l] = p - mm1;
    }
    for (int l = 0; l < 32; ++l) {
      volatile float p = d2 * (float)(q[l] >> 4);
      y[j + 32 + l] = p - mm2;
    }
    q += 32;
    is += 2;
  }
}

/* Q6_K, reference layout weight_loader.cpp:158-177: ql[128] | qh[64] |
 * int8 scales[16] | fp16 d; element i: low 4 bits from ql[i/2] (nibble i%2),
 * high 2 bits from qh[i/4] (pair i%4); w = (d * (q-32)) * scales[i/16]. */
static void deq_q6_k(const uint8_t *b, float *y) {
  const uint8_t *ql = b, *qh = b + 128;
  const int8_t *sc = (const int8_t *)(b + 192);
  float d = gqo_fp16_to_fp32(rd16(b + 208));
  for (int i = 0; i < 256; ++i) {
    int lo = (ql[i / 2] >> ((i % 2) * 4)) & 0x0F;
    int hi = (qh[i / 4] >> ((i % 4) * 2)) & 0x03;
    int q = (lo | (hi << 4)) - 32;
    volatile float t = d * (float)q;
    y[i] = t * (float)sc[i / 16];
  }
}

/* Q6_K, llama.cpp layout (ggml dequantize_row_q6_K, not part of the
 * reference): per 128-element half h and l in 0..31, element 128h + 32k + l
 * takes its low 4 bits from ql[64h + l + 32(k & 1)] (high nibble when k >= 2)
 * and its high 2 bits from qh[32h + l] (bits 2k, 2k+1); scales in element
 * order.  Values are rounded as the reference rounds Q6_K: (d * (q-32)) * sc. */
static void deq_q6_k_ggml(const uint8_t *b, float *y) {
  const uint8_t *ql = b, *qh = b + 128;
  const int8_t *sc = (const int8_t *)(b + 192);
  float d = gqo_fp16_to_fp32(rd16(b + 208));
  for (int i = 0; i < 256; ++i) {
    int h = i >> 7, k = (i >> 5) & 3, l = i & 31;
    int lo = (ql[64 * h + l + 32 * (k & 1)] >> (4 * (k >> 1))) & 0x0F;
    int hi = (qh[32 * h + l] >> (2 * k)) & 0x03;
    int q = (lo | (hi << 4)) - 32;
    volatile float t = d * (float)q;
    y[i] = t * (float)sc[i / 16];
  }
}

int gqo_dequant(int fmt, const uint8_t *blocks, size_t n_blocks, float *out) {
  size_t be = gqo_block_elems(fmt), bb = gqo_block_bytes(fmt);
  if (!be) return 1;
  for (size_t i = 0; i < n_blocks; ++i) {
    const uint8_t *b = blocks + i * bb;
    float *y = out + i * be;
    switch (fmt) {
    case GQO_F32:
      memcpy(y, b, 4);
      break;
    case GQO_F16:
      y[0] = gqo_fp16_to_fp32(rd16(b));
      break;
    case GQO_Q4_0:
      deq_q4_0(b, y);
      break;
    case GQO_Q8_0:
      deq_q8_0(b, y);
      break;
    case GQO_Q4_K:
      deq_q4_k(b, y);
      break;
    case GQO_Q4_K_GGML:
      deq_q4_k_ggml(b, y);
      break;
    case GQO_Q6_K:
      deq_q6_k(b, y);
      break;
    case GQO_Q6_K_GGML:
      deq_q6_k_ggml(b, y);
      break;
    default:
      return 1;
    }
  }
  return 0;
}

static void set_threads(int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
  else omp_set_num_threads(omp_get_num_procs());
#else
  (void)threads;
#endif
}

/* y = W x in the style of CpuReference::gemm (cpu_reference.hpp:56-66):
 * double accumulation, one cast to float at the end.  W is dequantized one
 * row at a time (the reference dequantizes the whole tensor first; the values
 * are identical). */
int gqo_gemv(int fmt, const uint8_t *w, const float *x, float *y, int N, int K,
             int B, int threads) {
  size_t be = gqo_block_elems(fmt), bb = gqo_block_bytes(fmt);
  if (!be || K % (int)be) return 1;
  size_t row_bytes = (size_t)K / be * bb;
  set_threads(threads);
  int err = 0;
#pragma omp parallel
  {
    float *row = (float *)malloc(sizeof(float) * (size_t)K);
    if (!row) {
#pragma omp atomic write
      err = 1;
    } else {
#pragma omp for schedule(static)
      for (int n = 0; n < N; ++n) {
        gqo_dequant(fmt, w + (size_t)n * row_bytes, (size_t)K / be, row);
        for (int b = 0; b < B; ++b) {
          const float *xb = x + (size_t)b * K;
          double acc = 0.0;
          for (int k = 0; k < K; ++k) acc += (double)xb[k] * (double)row[k];
          y[(size_t)b * N + n] = (float)acc;
        }
      }
      free(row);
    }
  }
  return err;
}

int gqo_gemm(int fmt, const uint8_t *w, const float *A, float *C, int M, int N,
             int K, int threads) {
  return gqo_gemv(fmt, w, A, C, N, K, M, threads);
}

/* cpu_reference.hpp:56-66: B is [K][N]. */
void gqo_gemm_ref(const float *A, const float *B, float *C, int M, int N, int K) {
  for (int i = 0; i < M; ++i)
    for (int j = 0; j < N; ++j) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k)
        acc += (double)A[i * K + k] * (double)B[k * N + j];
      C[i * N + j] = (float)acc;
    }
}

/* weight_loader.cpp:780-802: per 32-group s = amax/127, inv = s>1e-9 ? 1/s : 0,
 * q = (int8)round(w*inv) (round half away from zero), no clamp. */
void gqo_requant_int8(const float *w, size_t n, int8_t *q, float *scales) {
  size_t nb = (n + 31) / 32;
  for (size_t b = 0; b < nb; ++b) {
    float mx = 0.0f;
    for (size_t i = 0; i < 32 && b * 32 + i < n; ++i) {
      float a = fabsf(w[b * 32 + i]);
      mx = a > mx ? a : mx;
    }
    float s = mx / 127.0f;
    scales[b] = s;
    float inv = s > 1e-9f ? 1.0f / s : 0.0f;
    for (size_t i = 0; i < 32 && b * 32 + i < n; ++i) {
      volatile float t = w[b * 32 + i] * inv;
      q[b * 32 + i] = (int8_t)roundf(t);
    }
  }
}

/* weight_loader.cpp:920-957: s = amax/7, q = clamp(round(w*inv), -8, 7),
 * byte = (q0 & 15) | (q1 & 15) << 4 (even index in the low nibble). */
void gqo_requant_int4(const float *w, size_t n, uint8_t *packed, float *scales) {
  size_t ng = (n + 31) / 32;
  for (size_t g = 0; g < ng; ++g) {
    float mx = 0.0f;
    for (size_t i = 0; i < 32 && g * 32 + i < n; ++i) {
      float a = fabsf(w[g * 32 + i]);
      mx = a > mx ? a : mx;
    }
    float s = mx / 7.0f;
    scales[g] = s;
    float inv = s > 1e-9f ? 1.0f / s : 0.0f;
    for (size_t i = 0; i < 32 && g * 32 + i < n; i += 2) {
      size_t i0 = g * 32 + i, i1 = i0 + 1;
      volatile float t0 = w[i0] * inv;
      int8_t v0 = (int8_t)roundf(t0);
      v0 = v0 < -8 ? -8 : (v0 > 7 ? 7 : v0);
      int8_t v1 = 0;
      if (i1 < n) {
        volatile float t1 = w[i1] * inv;
        v1 = (int8_t)roundf(t1);
        v1 = v1 < -8 ? -8 : (v1 > 7 ? 7 : v1);
      }
      packed[i0 / 2] = (uint8_t)((v0 & 0x0F) | ((v1 & 0x0F) << 4));
    }
  }
}

/* weight_loader.cpp:972-998: h[h] = max|w| over rows [h*Dh, (h+1)*Dh) of a
 * [*, D] matrix, 1.0 when that is <= 1e-9. */
void gqo_head_scales(const float *w, uint32_t num_heads, uint32_t head_dim,
                     uint32_t dim, float *h_scales) {
  for (uint32_t h = 0; h < num_heads; ++h) {
    float mx = 0.0f;
    size_t n = (size_t)head_dim * dim;
    for (size_t i = 0; i < n; ++i) {
      float a = fabsf(w[(size_t)h * n + i]);
      mx = a > mx ? a : mx;
    }
    h_scales[h] = mx > 1e-9f ? mx : 1.0f;
  }
}

/* weight_loader.cpp:893-905: out[r*D + c] = in[c*KV + r]. */
void gqo_gqa_transpose(const float *in, uint32_t model_dim, uint32_t kv_dim,
                       float *out) {
  for (uint32_t r = 0; r < kv_dim; ++r)
    for (uint32_t c = 0; c < model_dim; ++c)
      out[(size_t)r * model_dim + c] = in[(size_t)c * kv_dim + r];
}

/* Scale of weight (n, k) in the reference's INT8 / INT4 launchers.  The two
 * routes index the flat per-group scale array differently:
 *   GEMV kernels (M <= 32 or force_gemv), gemm_kernels.hip:610,615 and
 *   781,796-797: s_row = scales + (n*K)/gs, then s_row[k/gs];
 *   MFMA kernels (M > 32), gemm_kernels.hip:717 and 886: scales[(n*K + k)/gs].
 * They agree whenever K % gs == 0. */
static size_t scale_index(size_t n, size_t K, size_t k, size_t gs, int gemv_route) {
  return gemv_route ? (n * K) / gs + k / gs : (n * K + k) / gs;
}

/* gemm_kernels.hip:594-634 (GEMV route) / 640-740 (MFMA route): the math,
 * rows in the "row" layout. */
void gqo_gemm_int8_wt(const float *x, const int8_t *q, const float *s, float *y,
                      int M, int N, int K, int gs, int gemv_route) {
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k) {
        size_t idx = (size_t)n * K + k;
        volatile float wv = (float)q[idx] * s[scale_index(n, K, k, gs, gemv_route)];
        acc += (double)x[(size_t)m * K + k] * (double)wv;
      }
      y[(size_t)m * N + n] = (float)acc;
    }
}

/* gemm_kernels.hip:763-817 (GEMV route) / 820-908 (MFMA route): sign-extended
 * nibbles, row n at byte n*(K/2) (even k in the low nibble), x head scale.
 * K is even (the reference's loader packs the flat tensor, which matches the
 * kernels' row addressing only then). */
void gqo_gemm_int4_wt(const float *x, const uint8_t *packed, const float *s,
                      const float *head_scales, float *y, int M, int N, int K,
                      int gs, int head_dim, int gemv_route) {
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k) {
        uint8_t p = packed[(size_t)n * (K / 2) + k / 2];
        int v = (k % 2 == 0) ? (p & 0x0F) : (p >> 4);
        if (v & 8) v -= 16;
        volatile float wv = (float)v * s[scale_index(n, K, k, gs, gemv_route)];
        acc += (double)x[(size_t)m * K + k] * (double)wv;
      }
      float h = 1.0f;
      if (head_scales && head_dim > 0) h = head_scales[n / head_dim];
      y[(size_t)m * N + n] = (float)acc * h;
    }
}

void gqo_quantize_act_q8(const float *a, int M, int K, int8_t *q, float *d) {
  int nb = K / 32;
  for (int m = 0; m < M; ++m)
    gqo_requant_int8(a + (size_t)m * K, (size_t)K, q + (size_t)m * K,
                     d + (size_t)m * nb);
}

int gqo_gemm_q8_i8(const uint8_t *w, const int8_t *qa, const float *da,
                   float *C, int M, int N, int K, int threads) {
  if (K % 32) return 1;
  int nb = K / 32;
  set_threads(threads);
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint8_t *row = w + (size_t)n * nb * 34;
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + (size_t)b * 34;
        float dw = gqo_fp16_to_fp32(rd16(blk));
        const int8_t *qw = (const int8_t *)(blk + 2);
        const int8_t *qx = qa + (size_t)m * K + (size_t)b * 32;
        long s = 0;
        for (int i = 0; i < 32; ++i) s += (long)qw[i] * (long)qx[i];
        acc += (double)da[(size_t)m * nb + b] * (double)dw * (double)s;
      }
      C[(size_t)m * N + n] = (float)acc;
    }
  }
  return 0;
}

void gqo_rmsnorm(const float *x, const float *gamma, int rows, int K, float eps, double *out) {
  for (int b = 0; b < rows; ++b) {
    double ss = 0.0;
    for (int k = 0; k < K; ++k) ss += (double)x[(size_t)b * K + k] * (double)x[(size_t)b * K + k];
    const double inv = 1.0 / sqrt(ss / (double)K + (double)eps);
    for (int k = 0; k < K; ++k) out[(size_t)b * K + k] = (double)x[(size_t)b * K + k] * inv * (double)gamma[k];
  }
}

void gqo_swiglu(const double *g, const double *u, size_t n, double *out) {
  for (size_t i = 0; i < n; ++i) out[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
}
