// gq_loadconv.hip -- load-time conversions of the GGUF loader, on the GPU and
// bit-exact with the reference's CPU loops:
//   fp16 -> fp32 (NaN -> Inf)          weight_loader.cpp:91-110
//   fp32 -> fp16 (truncating, FTZ)     weight_loader.cpp:112-123
//   Q6_K dequant (reference layout)    weight_loader.cpp:158-177
//   GQA K/V transpose [D][KV]->[KV][D] weight_loader.cpp:634-658, 739-781, 877-918
//   INT8 requant, per 32               weight_loader.cpp:780-802
//   INT4 requant + nibble pack         weight_loader.cpp:920-957
//   per-head max |w|                   weight_loader.cpp:972-998
//   Q8_0 -> int8 + fp32 scale split    weight_loader.cpp:703-712
// All of these are memory-bound single passes; they run once per tensor.
#include "gq_internal.h"

#pragma clang fp contract(off)

namespace {

static unsigned grid_for(size_t n) { return (unsigned)((n + 255) / 256); }

// std::max(a, b) as the reference calls it: (a < b) ? b : a, so a NaN second
// operand is ignored.
__device__ __forceinline__ float ref_max(float a, float b) { return (a < b) ? b : a; }

__global__ void __launch_bounds__(256) k_f16_to_f32(const uint16_t *__restrict__ in, float *__restrict__ out,
                                                    size_t n) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = gq_h2f(in[i]);
}

// weight_loader.cpp:112-123: exponent rebias; results below the fp16 normal
// range become signed zero, above it signed infinity; mantissa truncated.
__global__ void __launch_bounds__(256) k_f32_to_f16_trunc(const float *__restrict__ in, uint16_t *__restrict__ out,
                                                          size_t n) {
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  uint32_t x = __float_as_uint(in[i]);
  uint32_t sign = (x >> 16) & 0x8000u;
  int e = (int)((x >> 23) & 0xFFu) - 127 + 15;
  uint32_t m = x & 0x7FFFFFu;
  uint16_t h;
  if (e <= 0) h = (uint16_t)sign;
  else if (e >= 31) h = (uint16_t)(sign | 0x7C00u);
  else h = (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
  out[i] = h;
}

// One thread per 16 outputs (one int8 scale) of a 210-byte Q6_K block:
// ql[128] | qh[64] | int8 scales[16] | fp16 d; element i takes 4 low bits from
// ql[i/2] (nibble i%2) and 2 high bits from qh[i/4] (pair i%4) in the
// reference layout (ggml: gq_q6k_locate); w = (d * (q - 32)) * scales[i/16],
// each product rounded.
__global__ void __launch_bounds__(256) k_dequant_q6_k(const uint8_t *__restrict__ src, float *__restrict__ out,
                                                      size_t ngrp, int ggml) {
  size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= ngrp) return;
  const uint8_t *b = src + (t >> 4) * 210;
  const int g = (int)(t & 15);
  const float d = gq_h2f(gq_rd16(b + 208));
  const float sc = (float)(int8_t)b[192 + g];
  float y[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int i = 16 * g + e;
    const float p = d * (float)((int)gq_q6k_code(ggml, b, i) - 32);
    y[e] = p * sc;
  }
  float4 *o = reinterpret_cast<float4 *>(out + t * 16);
#pragma unroll
  for (int v = 0; v < 4; ++v) o[v] = make_float4(y[4 * v], y[4 * v + 1], y[4 * v + 2], y[4 * v + 3]);
}

// out[r][c] = in[c][r] for in [D][KV] (KV contiguous), via a 32x32 LDS tile.
template <typename T>
__global__ void __launch_bounds__(256) k_transpose(const T *__restrict__ in, T *__restrict__ out, int D, int KV) {
  __shared__ T tile[32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const int r0 = blockIdx.x * 32, c0 = blockIdx.y * 32;       // r over KV, c over D
  for (int j = ty; j < 32; j += 8) {
    int c = c0 + j, r = r0 + tx;
    if (c < D && r < KV) tile[j][tx] = in[(size_t)c * KV + r];
  }
  __syncthreads();
  for (int j = ty; j < 32; j += 8) {
    int r = r0 + j, c = c0 + tx;
    if (r < KV && c < D) out[(size_t)r * D + c] = tile[tx][j];
  }
}

// One thread per 32-element group of the flat tensor (the last group may be
// partial): s = amax / 127, inv = s > 1e-9 ? 1 / s : 0, q = round(w * inv)
// (half away from zero), no clamp.
__global__ void __launch_bounds__(256) k_requant_int8(const float *__restrict__ w, size_t n, int8_t *__restrict__ q,
                                                      float *__restrict__ scales, size_t ngrp) {
  size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= ngrp) return;
  const size_t base = g * 32;
  const int cnt = (int)((n - base) < 32 ? (n - base) : 32);
  float amax = 0.0f;
  for (int i = 0; i < cnt; ++i) amax = ref_max(amax, fabsf(w[base + i]));
  const float s = amax / 127.0f;
  scales[g] = s;
  const float inv = s > 1e-9f ? 1.0f / s : 0.0f;
  for (int i = 0; i < cnt; ++i) q[base + i] = (int8_t)(int)roundf(w[base + i] * inv);
}

// INT4: s = amax / 7, q clamped to [-8, 7], byte = (q0 & 15) | (q1 & 15) << 4
// with the even element in the low nibble; a missing odd element packs as 0.
__global__ void __launch_bounds__(256) k_requant_int4(const float *__restrict__ w, size_t n,
                                                      uint8_t *__restrict__ packed, float *__restrict__ scales,
                                                      size_t ngrp) {
  size_t g = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= ngrp) return;
  const size_t base = g * 32;
  const int cnt = (int)((n - base) < 32 ? (n - base) : 32);
  float amax = 0.0f;
  for (int i = 0; i < cnt; ++i) amax = ref_max(amax, fabsf(w[base + i]));
  const float s = amax / 7.0f;
  scales[g] = s;
  const float inv = s > 1e-9f ? 1.0f / s : 0.0f;
  for (int i = 0; i < cnt; i += 2) {
    int v0 = (int8_t)(int)roundf(w[base + i] * inv);
    v0 = v0 < -8 ? -8 : (v0 > 7 ? 7 : v0);
    int v1 = 0;
    if (i + 1 < cnt) {
      v1 = (int8_t)(int)roundf(w[base + i + 1] * inv);
      v1 = v1 < -8 ? -8 : (v1 > 7 ? 7 : v1);
    }
    packed[(base + i) >> 1] = (uint8_t)((v0 & 0x0F) | ((v1 & 0x0F) << 4));
  }
}

// One workgroup per head: max |w| over w[h * head_dim * dim .. + head_dim * dim),
// 1.0 when that maximum is not above 1e-9.  max is exact, so the parallel
// order gives the reference's sequential result.
__global__ void __launch_bounds__(256) k_head_scales(const float *__restrict__ w, size_t per_head,
                                                     float *__restrict__ out) {
  __shared__ float red[256];
  const float *p = w + (size_t)blockIdx.x * per_head;
  float m = 0.0f;
  for (size_t i = threadIdx.x; i < per_head; i += 256) m = ref_max(m, fabsf(p[i]));
  red[threadIdx.x] = m;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] = ref_max(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = red[0] > 1e-9f ? red[0] : 1.0f;
}

// Q8_0 block b -> q[32 b .. 32 b + 31] and scales[b] = fp16_to_fp32(d).
__global__ void __launch_bounds__(256) k_split_q8_0(const uint8_t *__restrict__ src, int8_t *__restrict__ q,
                                                    float *__restrict__ scales, size_t nblk) {
  size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;  // one thread per 8 bytes
  if (t >= nblk * 4) return;
  const size_t b = t >> 2;
  const int part = (int)(t & 3);
  const uint8_t *blk = src + b * 34;
  uint8_t v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = blk[2 + 8 * part + i];
  uint2 o;
  o.x = (uint32_t)v[0] | ((uint32_t)v[1] << 8) | ((uint32_t)v[2] << 16) | ((uint32_t)v[3] << 24);
  o.y = (uint32_t)v[4] | ((uint32_t)v[5] << 8) | ((uint32_t)v[6] << 16) | ((uint32_t)v[7] << 24);
  *reinterpret_cast<uint2 *>(q + b * 32 + 8 * part) = o;
  if (part == 0) scales[b] = gq_h2f(gq_rd16(blk));
}

}  // namespace

int gq_launch_dequant_q6_k(const void *blocks, size_t n_blocks, float *out, int ggml, hipStream_t s) {
  hipLaunchKernelGGL(k_dequant_q6_k, dim3(grid_for(n_blocks * 16)), dim3(256), 0, s, (const uint8_t *)blocks, out,
                     n_blocks * 16, ggml);
  return gq_last_launch();
}

int gq_launch_f16_to_f32(const void *in, size_t n, float *out, hipStream_t s) {
  hipLaunchKernelGGL(k_f16_to_f32, dim3(grid_for(n)), dim3(256), 0, s, (const uint16_t *)in, out, n);
  return gq_last_launch();
}

extern "C" int gq_convert_f32_to_f16(const float *in, size_t n, uint16_t *out, void *stream) {
  GQ_CHECK(in && out, GQ_ERR_INVALID_ARGS);
  if (n == 0) return GQ_OK;
  hipLaunchKernelGGL(k_f32_to_f16_trunc, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, in, out, n);
  return gq_last_launch();
}

extern "C" int gq_transpose_kv(int elem_bytes, const void *in, size_t model_dim, size_t kv_dim, void *out,
                               void *stream) {
  GQ_CHECK(in && out && in != out, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(elem_bytes == 2 || elem_bytes == 4, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(model_dim <= GQ_MAX_DIM && kv_dim <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  if (model_dim == 0 || kv_dim == 0) return GQ_OK;
  dim3 grid((unsigned)((kv_dim + 31) / 32), (unsigned)((model_dim + 31) / 32));
  GQ_CHECK(grid.y <= 65535u, GQ_ERR_INVALID_ARGS);
  if (elem_bytes == 4)
    hipLaunchKernelGGL(k_transpose<uint32_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint32_t *)in,
                       (uint32_t *)out, (int)model_dim, (int)kv_dim);
  else
    hipLaunchKernelGGL(k_transpose<uint16_t>, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t *)in,
                       (uint16_t *)out, (int)model_dim, (int)kv_dim);
  return gq_last_launch();
}

extern "C" int gq_requant_int8(const float *w, size_t n, int8_t *q, float *scales, void *stream) {
  GQ_CHECK(w && q && scales, GQ_ERR_INVALID_ARGS);
  if (n == 0) return GQ_OK;
  size_t ng = (n + 31) / 32;
  hipLaunchKernelGGL(k_requant_int8, dim3(grid_for(ng)), dim3(256), 0, (hipStream_t)stream, w, n, q, scales, ng);
  return gq_last_launch();
}

extern "C" int gq_requant_int4(const float *w, size_t n, uint8_t *packed, float *scales, void *stream) {
  GQ_CHECK(w && packed && scales, GQ_ERR_INVALID_ARGS);
  if (n == 0) return GQ_OK;
  size_t ng = (n + 31) / 32;
  hipLaunchKernelGGL(k_requant_int4, dim3(grid_for(ng)), dim3(256), 0, (hipStream_t)stream, w, n, packed, scales,
                     ng);
  return gq_last_launch();
}

extern "C" int gq_head_scales(const float *w, size_t n, uint32_t num_heads, uint32_t head_dim, uint32_t dim,
                              float *out, void *stream) {
  GQ_CHECK(w && out, GQ_ERR_INVALID_ARGS);
  if (num_heads == 0) return GQ_OK;
  const size_t per_head = (size_t)head_dim * dim;
  // the reference reads num_heads * head_dim * dim values without a bound
  // check; here that range must lie inside the tensor
  GQ_CHECK(per_head > 0 && (size_t)num_heads * per_head <= n, GQ_ERR_INVALID_ARGS);
  hipLaunchKernelGGL(k_head_scales, dim3(num_heads), dim3(256), 0, (hipStream_t)stream, w, per_head, out);
  return gq_last_launch();
}

extern "C" int gq_split_q8_0(const void *blocks, size_t n_blocks, int8_t *q, float *scales, void *stream) {
  GQ_CHECK(blocks && q && scales, GQ_ERR_INVALID_ARGS);
  if (n_blocks == 0) return GQ_OK;
  hipLaunchKernelGGL(k_split_q8_0, dim3(grid_for(n_blocks * 4)), dim3(256), 0, (hipStream_t)stream,
                     (const uint8_t *)blocks, q, scales, n_blocks);
  return gq_last_launch();
}
