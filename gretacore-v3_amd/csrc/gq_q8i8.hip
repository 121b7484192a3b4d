// gq_q8i8.hip -- Q8_0 weights x per-32 int8-quantized activations on the int8
// MFMA (v_mfma_i32_32x32x32_i8).  One 32-element block is one MFMA: the exact
// int32 block dot product is scaled by d_a[m][blk] * d_w[n][blk] in fp32 and
// accumulated.  Parity oracle: exact integer block sums with fp64 scale
// products (oracle gqo_gemm_q8_i8).
//
// Both operands carry a scale per 32-block, so every block of every output
// costs a conversion, a scale product and an fma after its MFMA (48 VALU
// instructions per 32 x 32 x 32 MFMA): the route is VALU-bound, not
// MFMA-bound.  The kernel keeps everything else off the VALU: operands come
// straight from the T16 tiles and the row-major int8 activations as 16-byte
// loads issued one block ahead, and the activation scales of a chunk (4
// blocks) are staged once per workgroup in LDS, four rows per LDS read.
#include "gq_internal.h"

namespace {

constexpr int kBM = 128, kBN = 128;  // workgroup tile; 4 waves of 64 x 64
constexpr int kThr = 256;

// workgroup id -> (M tile, N tile): each XCD (ids congruent mod 8) takes a
// contiguous run of tiles in column-major order, so the M tiles that share a
// weight column tile run on one XCD and read it from that XCD's L2
GQ_DEV void q8i8_tile(int id, int G, int tiles_m, int &mt, int &nt) {
  int g = id;
  if ((G & 7) == 0) g = (id & 7) * (G >> 3) + (id >> 3);
  mt = g % tiles_m;
  nt = g / tiles_m;
}

// buffer-resource loads: a 32-bit per-lane offset and a scalar offset
GQ_DEV __amdgpu_buffer_rsrc_t q8i8_rsrc(const void *p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, -1, 0x00020000);
}
GQ_DEV gq_i4 ld16(const void *base, uint32_t vo, uint32_t so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(q8i8_rsrc(base), vo, so, 0);
  return gq_i4{(int)v[0], (int)v[1], (int)v[2], (int)v[3]};
}
GQ_DEV gq_u2 ld8(const void *base, uint32_t vo, uint32_t so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(q8i8_rsrc(base), vo, so, 0);
  return gq_u2{v[0], v[1]};
}
// fp16 scale -> fp32 with the reference's rule (exponent 31 -> +-Inf) as a
// select instead of a branch
GQ_DEV float q8i8_scale(uint32_t h16) {
  const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)(h16 & 0xFFFFu));
  return __builtin_isnan(f) ? __builtin_copysignf(__builtin_inff(), f) : f;
}

__global__ void __launch_bounds__(kThr, 2)
k_gemm_q8_i8(const uint8_t *__restrict__ w, uint32_t sc_off, const int8_t *__restrict__ qa,
             const float *__restrict__ da, float *__restrict__ c, int M, int N, int K, int C, int tiles_m) {
  __shared__ __attribute__((aligned(16))) float ds[2][4][kBM];  // [buffer][block of chunk][row]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  int mt, nt;
  q8i8_tile(blockIdx.x, gridDim.x, tiles_m, mt, nt);
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int nb = K / 32;
  const int hl = lane >> 5;  // which 16-byte half of a block this lane holds
  const int ntiles = (N + 15) >> 4;

  // per MFMA tile: byte offsets of this lane's A row and B column at block 0
  // (clamped into the matrix; clamped rows and columns are never stored)
  uint32_t ao[2], bo[2], so[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int m = m0 + 64 * wm + 32 * i + (lane & 31);
    if (m >= M) m = M - 1;
    ao[i] = (uint32_t)m * (uint32_t)K + 16u * (uint32_t)hl;
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int n = n0 + 64 * wn + 32 * j + (lane & 31);
    if (n >= N) n = N - 1;
    int t = n >> 4;
    if (t >= ntiles) t = ntiles - 1;
    const uint32_t r = (uint32_t)(n & 15), tc = (uint32_t)t * (uint32_t)C;
    bo[j] = (tc << 11) + 16u * (16u * (uint32_t)hl + r);  // block 0 of chunk 0, half hl
    so[j] = sc_off + tc * 128u + 8u * r;                  // the row's 4 block scales of chunk 0
  }
  // byte offset of block blk relative to block 0 (the same for every lane):
  // blocks 2 h + e of a chunk sit in its h-th 1 KiB half, slot group 2 e + hl
  auto b_off = [](int blk) -> uint32_t {
    const uint32_t cc = (uint32_t)blk >> 2, jj = (uint32_t)blk & 3u;
    return (cc << 11) + ((jj >> 1) << 10) + 512u * (jj & 1u);
  };

  gq_f16v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // the activation scales of chunk cc (128 rows x 4 blocks): two entries per
  // thread, loaded unconditionally from clamped addresses (a load under a
  // branch would make the compiler wait for every load in flight), zero for
  // rows >= M and blocks >= nb -- the padding blocks of the last chunk then
  // add nothing
  auto load_scales = [&](int cc, float (&v)[2]) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int idx = tid + kThr * e;
      const int row = idx >> 2, jb = idx & 3;
      const int m = m0 + row, blk = 4 * cc + jb;
      float x = da[(size_t)(m < M ? m : M - 1) * nb + (blk < nb ? blk : nb - 1)];
      asm volatile("" : "+v"(x));  // keeps the load out of the select below
      v[e] = (m < M && blk < nb) ? x : 0.f;
    }
  };
  auto store_scales = [&](int buf, const float (&v)[2]) {
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int idx = tid + kThr * e;
      ds[buf][idx & 3][idx >> 2] = v[e];
    }
  };

  gq_i4 af[2][2], bf[2][2];  // [register stage][tile]
  auto load_ops = [&](int blk, int st) {
    if (blk >= nb) blk = nb - 1;  // (the padding blocks of the last chunk)
    const uint32_t sa = 32u * (uint32_t)blk, sb = b_off(blk);
#pragma unroll
    for (int i = 0; i < 2; ++i) af[st][i] = ld16(qa, ao[i], sa);
#pragma unroll
    for (int j = 0; j < 2; ++j) bf[st][j] = ld16(w, bo[j], sb);
  };

  const int nch = (nb + 3) >> 2;
  const gq_i16v zero = {};
  {
    float v0[2];
    load_scales(0, v0);
    store_scales(0, v0);
  }
  load_ops(0, 0);
  for (int cc = 0; cc < nch; ++cc) {
    const int buf = cc & 1;
    __syncthreads();  // ds[buf] staged; ds[buf ^ 1] no longer read
    float vn[2];
    load_scales(cc + 1 < nch ? cc + 1 : cc, vn);
    // the 4 block scales of this chunk for each column (block order 0, 2, 1, 3)
    gq_u2 dwp[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) dwp[j] = ld8(w, so[j], 128u * (uint32_t)cc);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int st = jb & 1;
      load_ops(4 * cc + jb + 1, st ^ 1);
      float dw[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t wd = dwp[j][jb & 1];
        dw[j] = q8i8_scale((jb >> 1) ? (wd >> 16) : wd);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        // rows 8 q + 4 hl + e (e = 0..3) of MFMA tile i: four runs of four
        const float *dr = &ds[buf][jb][64 * wm + 32 * i + 4 * hl];
        float dav[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const gq_f4 t = *reinterpret_cast<const gq_f4 *>(dr + 8 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) dav[4 * q + e] = t[e];
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const gq_i16v D = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[st][i], bf[st][j], zero, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[i][j][v] = fmaf(dav[v] * dw[j], (float)D[v], acc[i][j][v]);
        }
      }
    }
    store_scales(buf ^ 1, vn);
  }

#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + 64 * wn + 32 * j + (lane & 31);
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + 64 * wm + 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
        if (m < M) c[(size_t)m * N + n] = acc[i][j][v];
      }
  }
}

}  // namespace

extern "C" int gq_gemm_q8_i8(const void *packed, const int8_t *qa, const float *da, float *c, size_t M, size_t N,
                             size_t K, void *stream) {
  GQ_TRY(gq_check_shape(GQ_FMT_Q8_0, N, K));
  GQ_CHECK(M <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(packed && qa && da && c, GQ_ERR_INVALID_ARGS);
  if (M == 0 || N == 0) return GQ_OK;
  GQ_CHECK(K > 0, GQ_ERR_INVALID_ARGS);
  // 16-byte operand loads: activation rows start on 16-byte boundaries
  GQ_CHECK(((uintptr_t)qa & 15u) == 0, GQ_ERR_INVALID_ARGS);
  // 32-bit operand offsets
  GQ_CHECK(M * K < ((size_t)1 << 32) && gq_packed_bytes(GQ_FMT_Q8_0, N, K) < ((size_t)1 << 32), GQ_ERR_INVALID_ARGS);
  const int C = (int)gq_chunks(GQ_FMT_Q8_0, K);
  const int tiles_m = (int)((M + kBM - 1) / kBM), tiles_n = (int)((N + kBN - 1) / kBN);
  hipLaunchKernelGGL(k_gemm_q8_i8, dim3((unsigned)(tiles_m * tiles_n)), dim3(kThr), 0, (hipStream_t)stream,
                     (const uint8_t *)packed, (uint32_t)gq_sc_plane_offset(GQ_FMT_Q8_0, N, K), qa, da, c, (int)M, (int)N,
                     (int)K, C, tiles_m);
  return gq_last_launch();
}
