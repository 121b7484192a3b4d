// gq_gemm.hip -- prefill GEMM over T16-repacked GGUF weights on CDNA4 MFMA.
//
// Replaces gemm_mfma_int8_wt_kernel / gemm_mfma_int4_wt_kernel
// (src/rt/backend/hip/kernels/gemm_kernels.hip:640-740, 820-908) for
// GGUF-native weights.  Computes the mathematical C = A * W^T ("row" layout);
// the reference kernels' transposed 16x16 tile store is a bug, not a contract.
//
// Design:
//  * A (activations) is first converted to fp16 [M][Kp] (bf16 values are exact
//    in fp16 inside fp16's range) so the main loop stages it with plain copies.
//  * Workgroup tile BM x BN = 128 x 128, K step 128 (one T16 chunk; for Q4_K one
//    half super-block).  The weight tile is dequantized in registers with the
//    per-block scale folded in (one fp16 rounding per weight, as the reference's
//    __float2half(w * s) does) and written to LDS; A and W tiles are read back
//    as v_mfma_f32_32x32x16_f16 operands.  Global loads of step k+1 are issued
//    before the MFMAs of step k.
//  * 4 waves in a 2 x 2 arrangement, each owning a 64 x 64 block of C (2 x 2
//    MFMA tiles, fp32 accumulators).
#include "gq_internal.h"

namespace {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LDS_STRIDE = BK + 8;  // halves; pads rows apart in the LDS banks

// Global-load staging registers for one K step.
template <int FMT>
struct BRegs;
template <>
struct BRegs<GQ_FMT_Q4_0> {
  gq_u4 q[2];
  gq_u2 d[2];
};
template <>
struct BRegs<GQ_FMT_Q8_0> {
  gq_u4 q[4];
  gq_u2 d[4];
};
template <>
struct BRegs<GQ_FMT_Q4_K> {
  gq_u4 q[2];
  gq_u4 meta[2];
};

struct Tile {
  const uint8_t *w;
  size_t sc_off;
  int C;        // T16 chunks per row
  int tile0;    // first 16-row tile of this workgroup
  int ntiles;   // tiles in the tensor
};

// ---- weight tile: global -> registers --------------------------------------
template <int FMT>
GQ_DEV void load_b(const Tile &tl, int step, int tid, BRegs<FMT> &br) {
  if constexpr (FMT == GQ_FMT_Q4_0) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int slot = tid + 256 * i, rt = slot >> 6, lane = slot & 63;
      int tile = tl.tile0 + rt;
      if (tile >= tl.ntiles) tile = tl.ntiles - 1;  // clamped; results discarded
      size_t ch = (size_t)tile * tl.C + step;
      br.q[i] = gq_ld16(tl.w + (ch << 10) + 16 * lane);
      br.d[i] = gq_ld8(tl.w + tl.sc_off + ch * 128 + 8 * (lane & 15));
    }
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int slot = tid + 256 * i, rt = slot >> 7, part = (slot >> 6) & 1, lane = slot & 63;
      int tile = tl.tile0 + rt;
      if (tile >= tl.ntiles) tile = tl.ntiles - 1;
      size_t ch = (size_t)tile * tl.C + step;
      br.q[i] = gq_ld16(tl.w + (ch << 11) + (part << 10) + 16 * lane);
      br.d[i] = gq_ld8(tl.w + tl.sc_off + ch * 128 + 8 * (lane & 15));
    }
  } else {
    const int s = step >> 1, h = step & 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int slot = tid + 256 * i, rt = slot >> 6, lane = slot & 63;
      int tile = tl.tile0 + rt;
      if (tile >= tl.ntiles) tile = tl.ntiles - 1;
      size_t ch = (size_t)tile * tl.C + s;
      br.q[i] = gq_ld16(tl.w + (ch << 11) + (h << 10) + 16 * lane);
      br.meta[i] = gq_ld16(tl.w + tl.sc_off + ch * 256 + 16 * (lane & 15));
    }
  }
}

GQ_DEV gq_half2 h2_of_bits16(uint32_t b16) {
  uint32_t v = (b16 & 0xFFFFu) * 0x10001u;
  return gq_bits_h2(v);
}

// 4 byte values u (0..255) -> 2 fp16 pairs holding (1024 + u)
GQ_DEV void bytes_to_magic(uint32_t u, gq_half2 &lo, gq_half2 &hi) {
  lo = gq_bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u));
  hi = gq_bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u));
}

// T16 code group (8 bytes) -> 16 fp16 values (c - bias) * scale, slot order,
// computed as one rounding of the exact product.
GQ_DEV void group_to_h16(uint32_t w0, uint32_t w1, gq_half2 off, gq_half2 scale, gq_half8 &o0, gq_half8 &o1) {
  const uint32_t regs[4] = {w0 & 0x0F0F0F0Fu, (w0 >> 4) & 0x0F0F0F0Fu, w1 & 0x0F0F0F0Fu, (w1 >> 4) & 0x0F0F0F0Fu};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    gq_half2 lo, hi;
    bytes_to_magic(regs[q], lo, hi);
    lo = (lo + off) * scale;
    hi = (hi + off) * scale;
    gq_half8 &o = (q < 2) ? o0 : o1;
    const int b = 4 * (q & 1);
    o[b] = lo[0];
    o[b + 1] = lo[1];
    o[b + 2] = hi[0];
    o[b + 3] = hi[1];
  }
}

// ---- weight tile: registers -> dequantized fp16 in LDS ---------------------
// Thread slot (rt, lane = 16g + r): row 16rt + r, and for MFMA step m the
// elements 16(g&1)..+15 of block 2m + (g>>1) of the 128-k step.
template <int FMT>
GQ_DEV void store_b(const BRegs<FMT> &br, int step, int tid, _Float16 *Bs) {
  (void)step;
  if constexpr (FMT == GQ_FMT_Q4_0) {
    const gq_half2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int slot = tid + 256 * i, rt = slot >> 6, lane = slot & 63, g = lane >> 4, r = lane & 15;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int j = 2 * m + (g >> 1);
        uint32_t dbits = (j >> 1) ? (br.d[i][j & 1] >> 16) : br.d[i][j & 1];
        gq_half8 o0, o1;
        group_to_h16(br.q[i][2 * m], br.q[i][2 * m + 1], off, h2_of_bits16(dbits), o0, o1);
        _Float16 *dst = Bs + (16 * rt + r) * LDS_STRIDE + 32 * j + 16 * (g & 1);
        *reinterpret_cast<gq_half8 *>(dst) = o0;
        *reinterpret_cast<gq_half8 *>(dst + 8) = o1;
      }
    }
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    const gq_half2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int slot = tid + 256 * i, rt = slot >> 7, m = (slot >> 6) & 1, lane = slot & 63;
      int g = lane >> 4, r = lane & 15;
      const int j = 2 * m + (g >> 1);
      uint32_t dbits = (j >> 1) ? (br.d[i][j & 1] >> 16) : br.d[i][j & 1];
      const gq_half2 d2 = h2_of_bits16(dbits);
      _Float16 *dst = Bs + (16 * rt + r) * LDS_STRIDE + 32 * j + 16 * (g & 1);
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        gq_half8 o;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          gq_half2 lo, hi;
          bytes_to_magic(br.q[i][2 * q2 + q] ^ 0x80808080u, lo, hi);
          lo = (lo + off) * d2;
          hi = (hi + off) * d2;
          o[4 * q] = lo[0];
          o[4 * q + 1] = lo[1];
          o[4 * q + 2] = hi[0];
          o[4 * q + 3] = hi[1];
        }
        *reinterpret_cast<gq_half8 *>(dst + 8 * q2) = o;
      }
    }
  } else {
    const int hh = step & 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      int slot = tid + 256 * i, rt = slot >> 6, lane = slot & 63, g = lane >> 4, r = lane & 15;
      const gq_u4 &mt = br.meta[i];
      const uint32_t mv[4] = {mt[0], mt[1], mt[2], mt[3]};
      const float d = gq_h2f(mv[0] & 0xFFFFu), dmin = gq_h2f(mv[0] >> 16);
      const _Float16 hd = (_Float16)d;  // exact: d came from fp16 (NaN aside)
#pragma unroll
      for (int m2 = 0; m2 < 2; ++m2) {
        const int m = 2 * hh + m2, j = 2 * m + (g >> 1);
        uint32_t sc, mn;
        gq_q4k_meta_codes(mv, j, &sc, &mn);
        const _Float16 hsc = (_Float16)(float)sc, hnsc = (_Float16)(-1024.0f * (float)sc);
        const _Float16 hmin = (_Float16)(-(dmin * (float)mn));
        const gq_half2 sc2 = {hsc, hsc}, nsc2 = {hnsc, hnsc}, d2 = {hd, hd}, mn2 = {hmin, hmin};
        const uint32_t w0 = br.q[i][2 * m2], w1 = br.q[i][2 * m2 + 1];
        const uint32_t regs[4] = {w0 & 0x0F0F0F0Fu, (w0 >> 4) & 0x0F0F0F0Fu, w1 & 0x0F0F0F0Fu,
                                  (w1 >> 4) & 0x0F0F0F0Fu};
        gq_half8 o[2];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          gq_half2 lo, hi;
          bytes_to_magic(regs[q], lo, hi);
          lo = __builtin_elementwise_fma(__builtin_elementwise_fma(lo, sc2, nsc2), d2, mn2);
          hi = __builtin_elementwise_fma(__builtin_elementwise_fma(hi, sc2, nsc2), d2, mn2);
          const int b = 4 * (q & 1);
          o[q >> 1][b] = lo[0];
          o[q >> 1][b + 1] = lo[1];
          o[q >> 1][b + 2] = hi[0];
          o[q >> 1][b + 3] = hi[1];
        }
        // local k of sub-block j within this 128-k step: 32 * (j - 4hh)
        _Float16 *dst = Bs + (16 * rt + r) * LDS_STRIDE + 32 * (j - 4 * hh) + 16 * (g & 1);
        *reinterpret_cast<gq_half8 *>(dst) = o[0];
        *reinterpret_cast<gq_half8 *>(dst + 8) = o[1];
      }
    }
  }
}

// ---- activation tile -------------------------------------------------------
// LDS column kk of step `step` holds activation column step * BK + kk (a Q4_K
// super-block is two consecutive 128-k steps).
template <int FMT>
GQ_DEV int a_col(int step, int kk) {
  return step * BK + kk;
}

template <int FMT>
GQ_DEV void load_a(const _Float16 *__restrict__ a, int M, int Kp, int m0, int step, int tid, gq_u4 (&ar)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int idx = tid + 256 * i, row = idx >> 4, c8 = (idx & 15) * 8;
    int m = m0 + row;
    if (m >= M) m = M - 1;  // clamped; rows >= M are never stored
    ar[i] = gq_ld16(a + (size_t)m * Kp + a_col<FMT>(step, c8));
  }
}

GQ_DEV void store_a(const gq_u4 (&ar)[8], int tid, _Float16 *As) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int idx = tid + 256 * i, row = idx >> 4, c8 = (idx & 15) * 8;
    *reinterpret_cast<gq_u4 *>(As + row * LDS_STRIDE + c8) = ar[i];
  }
}

GQ_DEV uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int FMT, int CBF16>
__global__ void __launch_bounds__(256)
k_gemm_t16(const uint8_t *__restrict__ w, size_t sc_off, const _Float16 *__restrict__ a, void *__restrict__ c,
           int M, int N, int C, int Kp) {
  __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDS_STRIDE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  Tile tl{w, sc_off, C, n0 / 16, (int)gq_tiles(N)};
  const int nsteps = (FMT == GQ_FMT_Q4_K) ? 2 * C : C;

  gq_f16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  gq_u4 ar[8];
  BRegs<FMT> br;
  load_a<FMT>(a, M, Kp, m0, 0, tid, ar);
  load_b<FMT>(tl, 0, tid, br);

  for (int step = 0; step < nsteps; ++step) {
    __syncthreads();  // previous step's MFMAs are done with the LDS tiles
    store_a(ar, tid, As);
    store_b<FMT>(br, step, tid, Bs);
    __syncthreads();
    if (step + 1 < nsteps) {
      load_a<FMT>(a, M, Kp, m0, step + 1, tid, ar);
      load_b<FMT>(tl, step + 1, tid, br);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int kk = ks * 16 + 8 * (lane >> 5);
      gq_half8 af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        af[i] = *reinterpret_cast<const gq_half8 *>(As + (64 * wm + 32 * i + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const gq_half8 *>(Bs + (64 * wn + 32 * j + (lane & 31)) * LDS_STRIDE + kk);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = gq_mfma32(af[i], bf[j], acc[i][j]);
    }
  }

  // D layout (32x32): lane l holds column l%32, rows 8*(v/4) + 4*(l/32) + v%4.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + 64 * wn + 32 * j + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + 64 * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (m < M) {
          if constexpr (CBF16)
            reinterpret_cast<uint16_t *>(c)[(size_t)m * N + n] = f32_to_bf16_rne(acc[i][j][v]);
          else
            reinterpret_cast<float *>(c)[(size_t)m * N + n] = acc[i][j][v];
        }
      }
    }
}

template <int FMT>
int launch_gemm(const void *packed, const _Float16 *a16, void *c, int c_dtype, int M, int N, int K, hipStream_t s) {
  const int C = (int)gq_chunks(FMT, K), Kp = (int)gq_kpad(FMT, K);
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  if (c_dtype == GQ_DT_BF16)
    hipLaunchKernelGGL((k_gemm_t16<FMT, 1>), grid, dim3(256), 0, s, (const uint8_t *)packed, sc_off, a16, c, M, N,
                       C, Kp);
  else
    hipLaunchKernelGGL((k_gemm_t16<FMT, 0>), grid, dim3(256), 0, s, (const uint8_t *)packed, sc_off, a16, c, M, N,
                       C, Kp);
  return gq_last_launch();
}

}  // namespace

extern "C" size_t gq_gemm_workspace_bytes(int fmt, size_t M, size_t K) {
  if (!gq_fmt_valid(fmt) || M > GQ_MAX_DIM || K > GQ_MAX_DIM) return 0;
  return gq_align256(M * gq_kpad(fmt, K) * 2);
}

extern "C" int gq_gemm(int fmt, const void *packed, const void *a, int a_dtype, void *c, int c_dtype, size_t M,
                       size_t N, size_t K, void *ws, size_t ws_bytes, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(M <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(a_dtype == GQ_DT_F32 || a_dtype == GQ_DT_F16 || a_dtype == GQ_DT_BF16, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(c_dtype == GQ_DT_F32 || c_dtype == GQ_DT_BF16, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(packed && a && c, GQ_ERR_INVALID_ARGS);
  if (M == 0 || N == 0) return GQ_OK;
  GQ_CHECK(K > 0, GQ_ERR_INVALID_ARGS);
  size_t need = gq_gemm_workspace_bytes(fmt, M, K);
  if (!ws) {
    GQ_TRY(gq_default_workspace(need, &ws));
    ws_bytes = need;
  }
  GQ_CHECK(ws_bytes >= need, GQ_ERR_WORKSPACE);
  hipStream_t s = (hipStream_t)stream;
  const int Kp = (int)gq_kpad(fmt, K);
  _Float16 *a16 = (_Float16 *)ws;
  GQ_TRY(gq_launch_prep_a(a, a_dtype, a16, (int)M, (int)K, Kp, s));
  switch (fmt) {
  case GQ_FMT_Q4_0: return launch_gemm<GQ_FMT_Q4_0>(packed, a16, c, c_dtype, (int)M, (int)N, (int)K, s);
  case GQ_FMT_Q8_0: return launch_gemm<GQ_FMT_Q8_0>(packed, a16, c, c_dtype, (int)M, (int)N, (int)K, s);
  default: return launch_gemm<GQ_FMT_Q4_K>(packed, a16, c, c_dtype, (int)M, (int)N, (int)K, s);
  }
}
