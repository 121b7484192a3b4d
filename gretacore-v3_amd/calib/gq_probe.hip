// gq_probe.hip -- calibration kernels for the benchmark's roofline figures
// (built into lib/libgqcalib.so, apart from the product library; bench.py
// loads it; no counterpart in the reference).
//
// k_probe_read streams a buffer the way the decode GEMV streams its weights
// (the same grid of workgroups and waves, each wave issuing all of its
// 16-byte-per-lane loads up front, non-temporal) and does nothing with the
// data but fold it into one word per wave: the fastest a kernel of that shape
// can move those bytes, i.e. the read ceiling the GEMV's time is compared
// with.  k_probe_empty is the same grid with no work: the fixed cost of a
// launch.
#include "gq_probe.h"

#include "../../include/gq.h"
#include "gq_device.h"

namespace {

// the launch's status (this library stands alone: no libgq symbols)
int last_launch() { return hipGetLastError() == hipSuccess ? GQ_OK : GQ_ERR_HIP; }

// NL loads of 1 KiB per wave (16 bytes per lane), all issued before any is
// used; a wave past the end of the buffer does nothing.  The data is folded
// into one word that is stored only if it equals a value the host chooses
// (never, in practice): no write traffic, yet the loads stay live.
template <int NL>
__global__ void __launch_bounds__(1024) k_probe_read(const uint8_t *__restrict__ src, size_t bytes,
                                                     uint32_t never, uint32_t *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const size_t wave = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const size_t w0 = wave * (size_t)NL * 1024;
  if (w0 >= bytes) return;
  gq_u4 v[NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    size_t off = w0 + (size_t)i * 1024 + 16u * (uint32_t)lane;
    off = off + 16 <= bytes ? off : bytes - 16;  // (a ragged last wave)
    v[i] = gq_ld16_nt(src + off);
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < NL; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  if (x == never) out[wave] = x;
}

__global__ void k_probe_empty() {}

template <int NL>
int launch_probe(const void *src, size_t bytes, int wgs, int waves, uint32_t *out, hipStream_t s) {
  if constexpr (NL > 16) {
    return GQ_ERR_INVALID_ARGS;
  } else {
    const size_t per = (size_t)wgs * (size_t)waves;
    if ((size_t)NL * 1024 * per < bytes) return launch_probe<NL + 1>(src, bytes, wgs, waves, out, s);
    hipLaunchKernelGGL(k_probe_read<NL>, dim3((unsigned)wgs), dim3(64 * waves), 0, s, (const uint8_t *)src, bytes,
                       0x9E3779B9u, out);
    return last_launch();
  }
}

}  // namespace

extern "C" int gq_probe_read(const void *src, size_t bytes, int wgs, int waves_per_wg, uint32_t *out,
                             void *stream) {
  if (!(src && out && bytes >= 16 && bytes % 16 == 0)) return GQ_ERR_INVALID_ARGS;
  if (!(wgs > 0 && waves_per_wg >= 1 && waves_per_wg <= 16)) return GQ_ERR_INVALID_ARGS;
  // the fewest 1 KiB loads per wave that cover the buffer (at most 16)
  return launch_probe<1>(src, bytes, wgs, waves_per_wg, out, (hipStream_t)stream);
}

extern "C" int gq_probe_empty(int wgs, int waves_per_wg, void *stream) {
  if (!(wgs > 0 && waves_per_wg >= 1 && waves_per_wg <= 16)) return GQ_ERR_INVALID_ARGS;
  hipLaunchKernelGGL(k_probe_empty, dim3((unsigned)wgs), dim3(64 * waves_per_wg), 0, (hipStream_t)stream);
  return last_launch();
}

// ---- effective shader clock under matrix-core load --------------------------
// Every SIMD runs chains of v_mfma_f32_32x32x16_f16 on operands that change
// every iteration (so the data toggles as a real GEMM's do); wave 0 of
// workgroup 0 reads the shader-clock counter (s_memtime) and the constant
// 100 MHz counter (s_memrealtime) before and after its loop.  The ratio of
// the two differences is the clock the box holds under MFMA load.
namespace {
__global__ void __launch_bounds__(256) k_probe_clock(unsigned long long *out, int iters, uint32_t never) {
  const int lane = threadIdx.x & 63;
  uint32_t h = 0x9E3779B9u * (uint32_t)(threadIdx.x + 1) ^ (uint32_t)blockIdx.x * 0x85EBCA6Bu;
  gq_u4 ua, ub;
  for (int e = 0; e < 4; ++e) {
    h = h * 1664525u + 1013904223u;
    ua[e] = (h & 0x3BFF3BFFu);  // fp16 values below 1 in magnitude, random mantissas
    h = h * 1664525u + 1013904223u;
    ub[e] = (h & 0x3BFF3BFFu);
  }
  gq_f16v acc0 = {}, acc1 = {}, acc2 = {}, acc3 = {};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < iters; ++i) {
    const gq_half8 a = __builtin_bit_cast(gq_half8, ua), b = __builtin_bit_cast(gq_half8, ub);
    acc0 = gq_mfma32(a, b, acc0);
    acc1 = gq_mfma32(b, a, acc1);
    acc2 = gq_mfma32(a, a, acc2);
    acc3 = gq_mfma32(b, b, acc3);
    ua ^= gq_u4{0x01230123u, 0x02460246u, 0x00FF00FFu, 0x01010101u};
    ub ^= gq_u4{0x00110011u, 0x03000300u, 0x000F000Fu, 0x02020202u};
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
  for (int v = 0; v < 16; ++v) s += acc0[v] + acc1[v] + acc2[v] + acc3[v];
  if (__float_as_uint(s) == never) out[4] = (unsigned long long)lane;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    out[0] = t0;
    out[1] = t1;
    out[2] = r0;
    out[3] = r1;
  }
}
}  // namespace

extern "C" int gq_probe_clock(unsigned long long *d_out, int wgs, int iters, void *stream) {
  if (!d_out || wgs <= 0 || iters <= 0) return GQ_ERR_INVALID_ARGS;
  hipLaunchKernelGGL(k_probe_clock, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream, d_out, iters,
                     0x7FC12345u);
  return last_launch();
}
