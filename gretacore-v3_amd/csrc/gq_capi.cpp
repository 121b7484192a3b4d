// gq_capi.cpp -- host side of the C ABI: status reporting, sizes, the host
// (CPU) repack used by the loader, the library-owned workspace and the
// GretaCompute::gemm-style routing entry.
#include <algorithm>
#include <mutex>
#include <thread>
#include <string.h>
#include <vector>

#include "gq_internal.h"

namespace {
thread_local char g_last_error[256] = {0};

struct DeviceWorkspace {
  void *ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mutex;
std::vector<DeviceWorkspace> g_ws;
std::vector<int> g_cus;
}  // namespace

int gq_hip_status(hipError_t e) {
  if (e == hipSuccess) return GQ_OK;
  strncpy(g_last_error, hipGetErrorString(e), sizeof(g_last_error) - 1);
  g_last_error[sizeof(g_last_error) - 1] = 0;
  return GQ_ERR_HIP;
}

int gq_last_launch(void) { return gq_hip_status(hipGetLastError()); }

int gq_default_workspace(size_t bytes, void **ptr) {
  int dev = 0;
  GQ_TRY(gq_hip_status(hipGetDevice(&dev)));
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  if ((size_t)dev >= g_ws.size()) g_ws.resize(dev + 1);
  DeviceWorkspace &w = g_ws[dev];
  if (w.bytes < bytes) {
    // the old buffer may still be in use by queued work on any stream
    GQ_TRY(gq_hip_status(hipDeviceSynchronize()));
    if (w.ptr) (void)hipFree(w.ptr);
    w.ptr = nullptr;
    w.bytes = 0;
    size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    GQ_TRY(gq_hip_status(hipMalloc(&w.ptr, want)));
    w.bytes = want;
  }
  *ptr = w.ptr;
  return GQ_OK;
}

int gq_device_cus(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  if ((size_t)dev >= g_cus.size()) g_cus.resize(dev + 1, -1);
  if (g_cus[dev] < 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

extern "C" {

int gq_abi_version(void) { return GQ_ABI_VERSION; }

const char *gq_status_string(int status) {
  switch (status) {
  case GQ_OK: return "ok";
  case GQ_ERR_INVALID_ARGS: return "invalid arguments";
  case GQ_ERR_UNSUPPORTED: return "unsupported format, dtype or batch";
  case GQ_ERR_HIP: return "HIP error";
  case GQ_ERR_WORKSPACE: return "workspace missing or too small";
  case GQ_ERR_NO_DEVICE: return "no usable GPU";
  default: return "unknown status";
  }
}

const char *gq_last_error(void) { return g_last_error; }

size_t gq_gguf_bytes(int fmt, size_t N, size_t K) {
  if (!gq_fmt_valid(fmt)) return 0;
  return gq_layout_gguf_bytes(fmt, N, K);
}

int gq_packed_size(int fmt, size_t N, size_t K, size_t *bytes) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(bytes, GQ_ERR_INVALID_ARGS);
  *bytes = (N == 0 || K == 0) ? 0 : gq_packed_bytes(fmt, N, K);
  return GQ_OK;
}

// Host repack: the same per-block functions the device kernel uses.
namespace {
// Repacks the GGUF rows [n0, n1) (whole tiles) into the T16 buffer.
void repack_host_rows(int fmt, const uint8_t *src, uint8_t *dst, size_t N, size_t K, size_t n0, size_t n1) {
  const size_t C = gq_chunks(fmt, K), sc = gq_sc_plane_offset(fmt, N, K);
  if (fmt == GQ_FMT_Q4_0) {
    const size_t nb = K / 32;
    for (size_t n = n0; n < n1; ++n)
      for (size_t b = 0; b < nb; ++b) {
        uint64_t grp[2];
        uint32_t d16;
        gq_q4_0_groups(src + (n * nb + b) * 18, grp, &d16);
        for (int eh = 0; eh < 2; ++eh) memcpy(dst + gq_q4_0_grp_off(n, b, eh, C), &grp[eh], 8);
        uint16_t d = (uint16_t)d16;
        memcpy(dst + sc + gq_q4_0_d_off(n, b, C), &d, 2);
      }
  } else if (fmt == GQ_FMT_Q8_0) {
    const size_t nb = K / 32;
    for (size_t n = n0; n < n1; ++n)
      for (size_t b = 0; b < nb; ++b) {
        const uint8_t *blk = src + (n * nb + b) * 34;
        for (int eh = 0; eh < 2; ++eh) memcpy(dst + gq_q8_0_half_off(n, b, eh, C), blk + 2 + 16 * eh, 16);
        memcpy(dst + sc + gq_q4_0_d_off(n, b, C), blk, 2);
      }
  } else if (gq_fmt_is_q6k(fmt)) {
    const int ggml = fmt == GQ_FMT_Q6_K_GGML;
    for (size_t n = n0; n < n1; ++n)
      for (size_t s = 0; s < C; ++s) gq_q6k_put(ggml, src + (n * C + s) * 210, dst, dst + sc, n, s, C);
  } else {
    const int ggml = fmt == GQ_FMT_Q4_K_GGML;
    for (size_t n = n0; n < n1; ++n)
      for (size_t s = 0; s < C; ++s) {
        uint64_t grp[16];
        uint32_t meta[4];
        gq_q4k_groups(ggml, src + (n * C + s) * 144, grp, meta);
        for (int j = 0; j < 8; ++j)
          for (int eh = 0; eh < 2; ++eh) memcpy(dst + gq_q4k_grp_off(n, s, j, eh, C), &grp[2 * j + eh], 8);
        memcpy(dst + sc + gq_q4k_meta_off(n, s, C), meta, 16);
      }
  }
}
}  // namespace

int gq_repack_host(int fmt, const void *gguf, size_t N, size_t K, void *packed) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(gguf && packed, GQ_ERR_INVALID_ARGS);
  if (N == 0 || K == 0) return GQ_OK;
  const uint8_t *src = (const uint8_t *)gguf;
  uint8_t *dst = (uint8_t *)packed;
  memset(dst, 0, gq_packed_bytes(fmt, N, K));  // padding rows and blocks
  // row tiles split over host threads (each tile's bytes are written by one)
  const size_t tiles = gq_tiles(N);
  const size_t bytes = gq_packed_bytes(fmt, N, K);
  size_t nt = std::min<size_t>(std::max(1u, std::thread::hardware_concurrency()), 16);
  nt = std::min(nt, std::max<size_t>(1, bytes >> 22));  // >= 4 MiB per thread
  nt = std::min(nt, tiles);
  if (nt <= 1) {
    repack_host_rows(fmt, src, dst, N, K, 0, N);
    return GQ_OK;
  }
  std::vector<std::thread> th;
  for (size_t t = 0; t < nt; ++t) {
    const size_t n0 = std::min(N, tiles * t / nt * 16), n1 = std::min(N, tiles * (t + 1) / nt * 16);
    if (n0 < n1) th.emplace_back(repack_host_rows, fmt, src, dst, N, K, n0, n1);
  }
  for (auto &x : th) x.join();
  return GQ_OK;
}

int gq_unpack_host(int fmt, const void *packed, size_t N, size_t K, void *gguf) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(gguf && packed, GQ_ERR_INVALID_ARGS);
  if (N == 0 || K == 0) return GQ_OK;
  const uint8_t *src = (const uint8_t *)packed;
  uint8_t *dst = (uint8_t *)gguf;
  const size_t C = gq_chunks(fmt, K), sc = gq_sc_plane_offset(fmt, N, K);
  if (fmt == GQ_FMT_Q4_0) {
    const size_t nb = K / 32;
    for (size_t n = 0; n < N; ++n)
      for (size_t b = 0; b < nb; ++b) {
        uint64_t grp[2];
        uint16_t d = 0;
        for (int eh = 0; eh < 2; ++eh) memcpy(&grp[eh], src + gq_q4_0_grp_off(n, b, eh, C), 8);
        memcpy(&d, src + sc + gq_q4_0_d_off(n, b, C), 2);
        gq_q4_0_from_groups(grp, d, dst + (n * nb + b) * 18);
      }
  } else if (fmt == GQ_FMT_Q8_0) {
    const size_t nb = K / 32;
    for (size_t n = 0; n < N; ++n)
      for (size_t b = 0; b < nb; ++b) {
        uint8_t *blk = dst + (n * nb + b) * 34;
        for (int eh = 0; eh < 2; ++eh) memcpy(blk + 2 + 16 * eh, src + gq_q8_0_half_off(n, b, eh, C), 16);
        memcpy(blk, src + sc + gq_q4_0_d_off(n, b, C), 2);
      }
  } else if (gq_fmt_is_q6k(fmt)) {
    const int ggml = fmt == GQ_FMT_Q6_K_GGML;
    for (size_t n = 0; n < N; ++n)
      for (size_t s = 0; s < C; ++s) gq_q6k_get(ggml, src, src + sc, n, s, C, dst + (n * C + s) * 210);
  } else {
    const int ggml = fmt == GQ_FMT_Q4_K_GGML;
    const size_t S = C;
    for (size_t n = 0; n < N; ++n)
      for (size_t s = 0; s < S; ++s) {
        uint64_t grp[16];
        uint32_t meta[4];
        for (int j = 0; j < 8; ++j)
          for (int eh = 0; eh < 2; ++eh) memcpy(&grp[2 * j + eh], src + gq_q4k_grp_off(n, s, j, eh, S), 8);
        memcpy(meta, src + sc + gq_q4k_meta_off(n, s, S), 16);
        gq_q4k_from_groups(ggml, grp, meta, dst + (n * S + s) * 144);
      }
  }
  return GQ_OK;
}

// GretaCompute::gemm routing for GGUF-native weights
// (src/compute/src/greta_compute_hip.cpp:148-374): small M goes to the GEMV
// kernels, larger M to the MFMA GEMM.  A and C are f32, as in the reference.
int gq_matmul(int fmt, const void *packed, const float *a, float *c, size_t M, size_t N, size_t K, void *stream) {
  if (M >= 1 && M <= GQ_MAX_BATCH)
    return gq_gemv(fmt, packed, a, c, N, K, (int)M, nullptr, 0, stream);
  int ct = 0, nck = 0;
  if (gq_fmt_is_q6k(fmt) && gq_gemm_skinny_plan(fmt, M, N, K, &ct, &nck) != GQ_OK) {
    // K too long for the skinny kernel: batches of 16 rows through the GEMV
    for (size_t m0 = 0; m0 < M; m0 += GQ_MAX_BATCH) {
      const size_t mb = M - m0 < GQ_MAX_BATCH ? M - m0 : GQ_MAX_BATCH;
      GQ_TRY(gq_gemv(fmt, packed, a + m0 * K, c + m0 * N, N, K, (int)mb, nullptr, 0, stream));
    }
    return GQ_OK;
  }
  return gq_gemm(fmt, packed, a, GQ_DT_F32, c, GQ_DT_F32, M, N, K, nullptr, 0, stream);
}

}  // extern "C"
