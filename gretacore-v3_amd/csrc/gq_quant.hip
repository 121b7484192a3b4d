// gq_quant.hip -- bit-exact GGUF dequantization, the T16 repack kernel and the
// activation preparation kernels used by the GEMV/GEMM paths.
//
// Dequantized values follow the reference semantics exactly:
//   Q4_K  src/inference/src/weight_loader.cpp:125-156 (products and the final
//         difference rounded separately -> contraction is disabled below)
//   Q8_0  weight_loader.cpp:703-712 + gemm_kernels.hip:612-616: (float)q * d
//   Q4_0  GGUF spec (no reference implementation): (float)(q - 8) * d
//   Q6_K  weight_loader.cpp:158-177: (d * (c - 32)) * scale
//   fp16  weight_loader.cpp:91-110 (NaN -> Inf)
#include "gq_internal.h"

#pragma clang fp contract(off)

namespace {

// ---------------------------------------------------------------------------
// Dequantization of raw GGUF blocks: one thread per 32 output elements.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_dequant_q4_0(const uint8_t *__restrict__ src, float *__restrict__ out, size_t nblk) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nblk) return;
  const uint8_t *b = src + i * 18;
  float d = gq_h2f(gq_rd16(b));
  float y[32];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    uint32_t q = b[2 + j];
    y[j] = (float)((int)(q & 15u) - 8) * d;
    y[j + 16] = (float)((int)(q >> 4) - 8) * d;
  }
  float4 *o = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int v = 0; v < 8; ++v) o[v] = make_float4(y[4 * v], y[4 * v + 1], y[4 * v + 2], y[4 * v + 3]);
}

__global__ void __launch_bounds__(256)
k_dequant_q8_0(const uint8_t *__restrict__ src, float *__restrict__ out, size_t nblk) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nblk) return;
  const uint8_t *b = src + i * 34;
  float d = gq_h2f(gq_rd16(b));
  float4 *o = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int v = 0; v < 8; ++v) {
    float y0 = (float)(int8_t)b[2 + 4 * v] * d, y1 = (float)(int8_t)b[3 + 4 * v] * d;
    float y2 = (float)(int8_t)b[4 + 4 * v] * d, y3 = (float)(int8_t)b[5 + 4 * v] * d;
    o[v] = make_float4(y0, y1, y2, y3);
  }
}

// one thread per 32-element sub-block of a Q4_K super-block
__global__ void __launch_bounds__(256)
k_dequant_q4_k(const uint8_t *__restrict__ src, float *__restrict__ out, size_t nsub, int ggml) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nsub) return;
  size_t sb = i >> 3;
  int j = (int)(i & 7);
  const uint8_t *b = src + sb * 144;
  float d = gq_h2f(gq_rd16(b)), dmin = gq_h2f(gq_rd16(b + 2));
  uint8_t sc[8], m[8];
  if (ggml) gq_q4k_ggml_codes(b + 4, sc, m);
  else gq_q4k_ref_codes(b + 4, sc, m);
  float scale = d * (float)sc[j];
  float minv = dmin * (float)m[j];
  float y[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    float p = scale * (float)gq_q4k_nib(ggml, b + 16, j, e);
    y[e] = p - minv;
  }
  float4 *o = reinterpret_cast<float4 *>(out + i * 32);
#pragma unroll
  for (int v = 0; v < 8; ++v) o[v] = make_float4(y[4 * v], y[4 * v + 1], y[4 * v + 2], y[4 * v + 3]);
}

// ---------------------------------------------------------------------------
// Dequantization straight from the T16 layout (proves the repack is lossless
// and gives the GEMM paths' weight values).  One thread per (row, 32-block).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_dequant_t16(int fmt, const uint8_t *__restrict__ w, float *__restrict__ out, int N, int K) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  int nb = K / 32;
  if (i >= (size_t)N * nb) return;
  size_t n = i / nb, blk = i % nb;
  float y[32];
  const size_t C = gq_chunks(fmt, K);
  const uint8_t *scp = w + gq_sc_plane_offset(fmt, N, K);
  if (fmt == GQ_FMT_Q4_0) {
    float d = gq_h2f(gq_rd16(scp + gq_q4_0_d_off(n, blk, C)));
#pragma unroll
    for (int eh = 0; eh < 2; ++eh) {
      uint8_t c[16];
      gq_unpack_codes16(*reinterpret_cast<const uint64_t *>(w + gq_q4_0_grp_off(n, blk, eh, C)), c);
#pragma unroll
      for (int s = 0; s < 16; ++s) y[16 * eh + s] = (float)((int)c[s] - 8) * d;
    }
  } else if (fmt == GQ_FMT_Q8_0) {
    float d = gq_h2f(gq_rd16(scp + gq_q4_0_d_off(n, blk, C)));
#pragma unroll
    for (int eh = 0; eh < 2; ++eh) {
      const int8_t *q = reinterpret_cast<const int8_t *>(w + gq_q8_0_half_off(n, blk, eh, C));
#pragma unroll
      for (int s = 0; s < 16; ++s) y[16 * eh + s] = (float)q[s] * d;
    }
  } else if (fmt == GQ_FMT_Q6_K) {
    // (d * (c - 32)) * scale, as weight_loader.cpp:158-177 rounds it
    size_t s = blk >> 3;
    int j = (int)(blk & 7);
    const float d = gq_h2f(gq_rd16(scp + gq_q6k_d_off(n, s, C)));
    const int8_t *scl = reinterpret_cast<const int8_t *>(scp + gq_q6k_sc_off(n, s, C));
#pragma unroll
    for (int eh = 0; eh < 2; ++eh) {
      uint8_t c[16];
      gq_unpack_codes16(*reinterpret_cast<const uint64_t *>(w + gq_q6k_grp_off(n, s, j, eh, C)), c);
      const uint32_t hw = *reinterpret_cast<const uint32_t *>(w + gq_q6k_hi_off(n, s, j, eh, C));
      const float sc = (float)scl[2 * j + eh];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = d * (float)((int)(c[e] | (gq_q6k_hi_of(hw, e) << 4)) - 32);
        y[16 * eh + e] = p * sc;
      }
    }
  } else {
    size_t s = blk >> 3;
    int j = (int)(blk & 7);
    const uint32_t *meta = reinterpret_cast<const uint32_t *>(scp + gq_q4k_meta_off(n, s, C));
    uint32_t mv[4] = {meta[0], meta[1], meta[2], meta[3]};
    float d = gq_h2f(mv[0] & 0xFFFFu), dmin = gq_h2f(mv[0] >> 16);
    uint32_t scj, mj;
    gq_q4k_meta_codes(mv, j, &scj, &mj);
    float scale = d * (float)scj;
    float minv = dmin * (float)mj;
#pragma unroll
    for (int eh = 0; eh < 2; ++eh) {
      uint8_t c[16];
      gq_unpack_codes16(*reinterpret_cast<const uint64_t *>(w + gq_q4k_grp_off(n, s, j, eh, C)), c);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float p = scale * (float)c[e];
        y[16 * eh + e] = p - minv;
      }
    }
  }
  float4 *o = reinterpret_cast<float4 *>(out + n * (size_t)K + blk * 32);
#pragma unroll
  for (int v = 0; v < 8; ++v) o[v] = make_float4(y[4 * v], y[4 * v + 1], y[4 * v + 2], y[4 * v + 3]);
}

// ---------------------------------------------------------------------------
// Repack GGUF -> T16.  One thread per (padded row, padded block) of the rows
// [row0, row0 + rows) of an N-row tensor (row0 a multiple of 16; src points at
// row row0 of the GGUF data); positions outside the tensor are written as
// zeros, so no memset is needed.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_repack_q4_0(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int N, int K, int row0, int rows) {
  size_t C = gq_chunks(GQ_FMT_Q4_0, K), nbp = C * 4;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)rows * nbp) return;
  size_t r = i / nbp, blk = i % nbp, n = row0 + r;
  size_t nb = (size_t)K / 32;
  uint64_t grp[2] = {0, 0};
  uint32_t d16 = 0;
  if (n < (size_t)N && blk < nb) gq_q4_0_groups(src + (r * nb + blk) * 18, grp, &d16);
  for (int eh = 0; eh < 2; ++eh) *reinterpret_cast<uint64_t *>(dst + gq_q4_0_grp_off(n, blk, eh, C)) = grp[eh];
  *reinterpret_cast<uint16_t *>(dst + gq_sc_plane_offset(GQ_FMT_Q4_0, N, K) + gq_q4_0_d_off(n, blk, C)) =
      (uint16_t)d16;
}

__global__ void __launch_bounds__(256)
k_repack_q8_0(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int N, int K, int row0, int rows) {
  size_t C = gq_chunks(GQ_FMT_Q8_0, K), nbp = C * 4;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)rows * nbp) return;
  size_t r = i / nbp, blk = i % nbp, n = row0 + r;
  size_t nb = (size_t)K / 32;
  bool in = n < (size_t)N && blk < nb;
  const uint8_t *b = src + (r * nb + blk) * 34;
  for (int eh = 0; eh < 2; ++eh) {
    uint32_t wv[4] = {0, 0, 0, 0};
    if (in)
      for (int q = 0; q < 4; ++q)
        wv[q] = (uint32_t)b[2 + 16 * eh + 4 * q] | ((uint32_t)b[3 + 16 * eh + 4 * q] << 8) |
                ((uint32_t)b[4 + 16 * eh + 4 * q] << 16) | ((uint32_t)b[5 + 16 * eh + 4 * q] << 24);
    *reinterpret_cast<gq_u4 *>(dst + gq_q8_0_half_off(n, blk, eh, C)) = gq_u4{wv[0], wv[1], wv[2], wv[3]};
  }
  *reinterpret_cast<uint16_t *>(dst + gq_sc_plane_offset(GQ_FMT_Q8_0, N, K) + gq_q4_0_d_off(n, blk, C)) =
      (uint16_t)(in ? gq_rd16(b) : 0u);
}

__global__ void __launch_bounds__(256)
k_repack_q4_k(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int N, int K, int row0, int rows,
              int ggml) {
  size_t S = gq_chunks(GQ_FMT_Q4_K, K);
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)rows * S) return;
  size_t r = i / S, s = i % S, n = row0 + r;
  uint64_t grp[16];
  uint32_t meta[4] = {0, 0, 0, 0};
  if (n < (size_t)N) {
    gq_q4k_groups(ggml, src + (r * S + s) * 144, grp, meta);
  } else {
    for (int q = 0; q < 16; ++q) grp[q] = 0;
  }
  for (int j = 0; j < 8; ++j)
    for (int eh = 0; eh < 2; ++eh)
      *reinterpret_cast<uint64_t *>(dst + gq_q4k_grp_off(n, s, j, eh, S)) = grp[2 * j + eh];
  *reinterpret_cast<gq_u4 *>(dst + gq_sc_plane_offset(GQ_FMT_Q4_K, N, K) + gq_q4k_meta_off(n, s, S)) =
      gq_u4{meta[0], meta[1], meta[2], meta[3]};
}

// one thread per (padded row, super-block)
__global__ void __launch_bounds__(256)
k_repack_q6_k(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int N, int K, int row0, int rows,
              int ggml) {
  size_t S = gq_chunks(GQ_FMT_Q6_K, K);
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)rows * S) return;
  size_t r = i / S, s = i % S, n = row0 + r;
  gq_q6k_put(ggml, n < (size_t)N ? src + (r * S + s) * 210 : nullptr, dst,
             dst + gq_sc_plane_offset(GQ_FMT_Q6_K, N, K), n, s, S);
}

// ---------------------------------------------------------------------------
// Activation preparation for the GEMV with batch > 4.  x f32 [B][K] ->
//   limbs int8 [B][2][Kp]: x ~ s * (a + b / 254) per 32-block, s = amax / 127
//   zero  int8 [Kp]
//   scl   float4 [B][Kp/32]: (s, S, s / 254, 0), S = sum of the represented block
// Elements k >= K are zeros.  One thread per 32-block.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
k_prep_x(const float *__restrict__ x, int8_t *__restrict__ xl, float *__restrict__ scl, int B, int K, int Kp) {
  const int nblk = Kp / 32;
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= B * nblk) return;
  const int b = i / nblk, j = i % nblk;
  const float *xr = x + (size_t)b * K + 32 * j;
  float v[32];
  if (32 * j + 32 <= K) {
    const float4 *p = reinterpret_cast<const float4 *>(xr);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float4 t = p[q];
      v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) v[e] = 0.0f;
  }
  float amax = 0.f, s = 0.f;
#pragma unroll
  for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
  const float inv = amax > 0.f ? 127.0f / amax : 0.f;
  const float sx = amax * (1.0f / 127.0f);
  uint32_t la[8], lb[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    uint32_t wa = 0, wb = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t = v[4 * q + e] * inv;
      const float a = rintf(t);
      const float bb = rintf((t - a) * 254.0f);
      s += a * 254.0f + bb;  // exact integer
      wa |= ((uint32_t)(int)a & 0xFFu) << (8 * e);
      wb |= ((uint32_t)(int)bb & 0xFFu) << (8 * e);
    }
    la[q] = wa;
    lb[q] = wb;
  }
  gq_u4 *pa = reinterpret_cast<gq_u4 *>(xl + (size_t)(2 * b) * Kp + 32 * j);
  gq_u4 *pb = reinterpret_cast<gq_u4 *>(xl + (size_t)(2 * b + 1) * Kp + 32 * j);
  pa[0] = gq_u4{la[0], la[1], la[2], la[3]};
  pa[1] = gq_u4{la[4], la[5], la[6], la[7]};
  pb[0] = gq_u4{lb[0], lb[1], lb[2], lb[3]};
  pb[1] = gq_u4{lb[4], lb[5], lb[6], lb[7]};
  if (b == 0) {
    gq_u4 *pz = reinterpret_cast<gq_u4 *>(xl + (size_t)2 * B * Kp + 32 * j);
    pz[0] = gq_u4{0u, 0u, 0u, 0u};
    pz[1] = gq_u4{0u, 0u, 0u, 0u};
  }
  s *= sx * (1.0f / 254.0f);  // block sum of the represented values
  *reinterpret_cast<gq_f4 *>(scl + 4 * ((size_t)b * nblk + j)) = gq_f4{sx, s, sx * (1.0f / 254.0f), 0.f};
}

// Per-32 int8 activation quantization (Q8_0 int8-MFMA path): the reference's
// INT8 requant rule applied to activations (weight_loader.cpp:780-802):
// d = amax/127, inv = d > 1e-9 ? 1/d : 0, q = round(a * inv), half away.
__global__ void __launch_bounds__(256)
k_quantize_act_q8(const void *__restrict__ a, int a_dtype, int8_t *__restrict__ q,
                  float *__restrict__ dq, int M, int K) {
  int nb = K / 32;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * nb) return;
  size_t m = i / nb, blk = i % nb;
  float v[32];
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    size_t idx = m * K + blk * 32 + e;
    if (a_dtype == GQ_DT_BF16)
      v[e] = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t *>(a)[idx] << 16);
    else if (a_dtype == GQ_DT_F16)
      v[e] = (float)reinterpret_cast<const _Float16 *>(a)[idx];
    else
      v[e] = reinterpret_cast<const float *>(a)[idx];
  }
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) mx = fmaxf(mx, fabsf(v[e]));
  float d = mx / 127.0f;
  float inv = d > 1e-9f ? 1.0f / d : 0.0f;
  uint32_t words[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    uint32_t u = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float t = v[4 * w + e] * inv;
      int qi = (int)roundf(t);
      u |= ((uint32_t)qi & 0xFFu) << (8 * e);
    }
    words[w] = u;
  }
  gq_u4 *o = reinterpret_cast<gq_u4 *>(q + m * K + blk * 32);
  o[0] = gq_u4{words[0], words[1], words[2], words[3]};
  o[1] = gq_u4{words[4], words[5], words[6], words[7]};
  dq[m * nb + blk] = d;
}

}  // namespace

static unsigned blocks_for(size_t n) { return (unsigned)((n + 255) / 256); }

extern "C" int gq_dequant_gguf(int fmt, const void *blocks, size_t n_blocks, float *out, void *stream) {
  GQ_CHECK(gq_fmt_valid(fmt) || fmt == GQ_FMT_F16, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(blocks && out, GQ_ERR_INVALID_ARGS);
  if (n_blocks == 0) return GQ_OK;
  hipStream_t s = (hipStream_t)stream;
  if (fmt == GQ_FMT_F16) return gq_launch_f16_to_f32(blocks, n_blocks, out, s);
  if (gq_fmt_is_q6k(fmt)) return gq_launch_dequant_q6_k(blocks, n_blocks, out, fmt == GQ_FMT_Q6_K_GGML, s);
  const uint8_t *src = (const uint8_t *)blocks;
  if (fmt == GQ_FMT_Q4_0)
    hipLaunchKernelGGL(k_dequant_q4_0, dim3(blocks_for(n_blocks)), dim3(256), 0, s, src, out, n_blocks);
  else if (fmt == GQ_FMT_Q8_0)
    hipLaunchKernelGGL(k_dequant_q8_0, dim3(blocks_for(n_blocks)), dim3(256), 0, s, src, out, n_blocks);
  else
    hipLaunchKernelGGL(k_dequant_q4_k, dim3(blocks_for(n_blocks * 8)), dim3(256), 0, s, src, out,
                       n_blocks * 8, (int)(fmt == GQ_FMT_Q4_K_GGML));
  return gq_last_launch();
}

extern "C" int gq_dequant_packed(int fmt, const void *packed, size_t N, size_t K, float *out, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(packed && out, GQ_ERR_INVALID_ARGS);
  if (N == 0 || K == 0) return GQ_OK;
  int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt;
  hipLaunchKernelGGL(k_dequant_t16, dim3(blocks_for(N * (K / 32))), dim3(256), 0, (hipStream_t)stream, f,
                     (const uint8_t *)packed, out, (int)N, (int)K);
  return gq_last_launch();
}

extern "C" int gq_repack_rows(int fmt, const void *gguf_rows, size_t N, size_t K, size_t row0, size_t rows,
                              void *packed, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(gguf_rows && packed, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(row0 % 16 == 0 && row0 <= N && rows <= N - row0, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(row0 + rows == N || rows % 16 == 0, GQ_ERR_INVALID_ARGS);  // whole tiles, or the tensor's end
  if (rows == 0 || K == 0) return GQ_OK;
  hipStream_t s = (hipStream_t)stream;
  // rows padded to whole tiles: the padding rows of the last tile are zeroed
  const size_t rp = gq_tiles(row0 + rows) * 16 - row0, C = gq_chunks(fmt, K);
  const uint8_t *src = (const uint8_t *)gguf_rows;
  uint8_t *dst = (uint8_t *)packed;
  const int n = (int)N, k = (int)K, r0 = (int)row0, r = (int)rp;
  if (fmt == GQ_FMT_Q4_0)
    hipLaunchKernelGGL(k_repack_q4_0, dim3(blocks_for(rp * C * 4)), dim3(256), 0, s, src, dst, n, k, r0, r);
  else if (fmt == GQ_FMT_Q8_0)
    hipLaunchKernelGGL(k_repack_q8_0, dim3(blocks_for(rp * C * 4)), dim3(256), 0, s, src, dst, n, k, r0, r);
  else if (gq_fmt_is_q6k(fmt))
    hipLaunchKernelGGL(k_repack_q6_k, dim3(blocks_for(rp * C)), dim3(256), 0, s, src, dst, n, k, r0, r,
                       (int)(fmt == GQ_FMT_Q6_K_GGML));
  else
    hipLaunchKernelGGL(k_repack_q4_k, dim3(blocks_for(rp * C)), dim3(256), 0, s, src, dst, n, k, r0, r,
                       (int)(fmt == GQ_FMT_Q4_K_GGML));
  return gq_last_launch();
}

extern "C" int gq_repack(int fmt, const void *gguf, size_t N, size_t K, void *packed, void *stream) {
  return gq_repack_rows(fmt, gguf, N, K, 0, N, packed, stream);
}

int gq_launch_prep_x(int fmt, const float *x, void *ws, int B, int K, hipStream_t s) {
  const int Kp = (int)gq_kpad(fmt, K);
  int8_t *xl = (int8_t *)ws;
  float *scl = (float *)((uint8_t *)ws + gq_xl_bytes(fmt, K, B));
  const int n = B * (Kp / 32);
  hipLaunchKernelGGL(k_prep_x, dim3(blocks_for(n)), dim3(256), 0, s, x, xl, scl, B, K, Kp);
  return gq_last_launch();
}

namespace {
__global__ void __launch_bounds__(256) k_fill_zero(float *p, size_t n) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}
}  // namespace

int gq_fill_zero(float *p, size_t n, hipStream_t s) {
  if (n == 0) return GQ_OK;
  hipLaunchKernelGGL(k_fill_zero, dim3(blocks_for(n)), dim3(256), 0, s, p, n);
  return gq_last_launch();
}


extern "C" int gq_quantize_act_q8(const void *a, int a_dtype, size_t M, size_t K, int8_t *q, float *d,
                                  void *stream) {
  GQ_CHECK(a && q && d, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(a_dtype == GQ_DT_F32 || a_dtype == GQ_DT_F16 || a_dtype == GQ_DT_BF16, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(K % 32 == 0 && K <= GQ_MAX_DIM && M <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  if (M == 0 || K == 0) return GQ_OK;
  hipLaunchKernelGGL(k_quantize_act_q8, dim3(blocks_for(M * (K / 32))), dim3(256), 0, (hipStream_t)stream,
                     a, a_dtype, q, d, (int)M, (int)K);
  return gq_last_launch();
}
