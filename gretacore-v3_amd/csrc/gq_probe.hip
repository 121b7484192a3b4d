// gq_probe.hip -- calibration kernels for the benchmark's roofline figures.
//
// k_probe_read streams a buffer the way the decode GEMV streams its weights
// (the same grid of workgroups and waves, each wave issuing all of its
// 16-byte-per-lane loads up front, non-temporal) and does nothing with the
// data but fold it into one word per wave: the fastest a kernel of that shape
// can move those bytes, i.e. the read ceiling the GEMV's time is compared
// with.  k_probe_empty is the same grid with no work: the fixed cost of a
// launch.
#include "gq_internal.h"

namespace {

constexpr int kProbeLoads = 16;  // 1 KiB per wave per load: at most 16 KiB per wave

__global__ void __launch_bounds__(1024) k_probe_read(const uint8_t *__restrict__ src, uint32_t per_wave,
                                                     size_t bytes, uint32_t *__restrict__ out) {
  const int lane = threadIdx.x & 63;
  const size_t wave = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const size_t w0 = wave * per_wave;
  const int n = (int)(per_wave >> 10);  // loads of this wave (wave-uniform)
  gq_u4 v[kProbeLoads];
#pragma unroll
  for (int i = 0; i < kProbeLoads; ++i) {
    const int ii = i < n ? i : n - 1;  // surplus loads repeat the last one (as the GEMV's)
    size_t off = w0 + (size_t)ii * 1024 + 16u * (uint32_t)lane;
    off = off + 16 <= bytes ? off : bytes - 16;
    v[i] = gq_ld16_nt(src + off);
  }
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < kProbeLoads; ++i) x ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  // one word per wave keeps the loads live
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x ^= (uint32_t)__shfl_xor((int)x, o, 64);
  if (lane == 0) out[wave] = x;
}

__global__ void k_probe_empty() {}

}  // namespace

extern "C" int gq_probe_read(const void *src, size_t bytes, int wgs, int waves_per_wg, uint32_t *out,
                             void *stream) {
  GQ_CHECK(src && out && bytes >= 16 && bytes % 16 == 0, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(wgs > 0 && waves_per_wg >= 1 && waves_per_wg <= 16, GQ_ERR_INVALID_ARGS);
  const size_t waves = (size_t)wgs * (size_t)waves_per_wg;
  const size_t per_wave = (bytes + waves - 1) / waves;
  const size_t pw = (per_wave + 1023) & ~(size_t)1023;
  GQ_CHECK(pw <= (size_t)kProbeLoads * 1024, GQ_ERR_INVALID_ARGS);
  hipLaunchKernelGGL(k_probe_read, dim3((unsigned)wgs), dim3(64 * waves_per_wg), 0, (hipStream_t)stream,
                     (const uint8_t *)src, (uint32_t)pw, bytes, out);
  return gq_last_launch();
}

extern "C" int gq_probe_empty(int wgs, int waves_per_wg, void *stream) {
  GQ_CHECK(wgs > 0 && waves_per_wg >= 1 && waves_per_wg <= 16, GQ_ERR_INVALID_ARGS);
  hipLaunchKernelGGL(k_probe_empty, dim3((unsigned)wgs), dim3(64 * waves_per_wg), 0, (hipStream_t)stream);
  return gq_last_launch();
}
