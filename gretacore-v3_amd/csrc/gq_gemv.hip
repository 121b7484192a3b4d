// gq_gemv.hip -- decode GEMV (batch 1..16) over T16-repacked GGUF weights.
//
// Replaces gemv_int8_wt_kernel / gemv_int4_wt_kernel
// (src/rt/backend/hip/kernels/gemm_kernels.hip:594-634, 763-817) for
// GGUF-native weights: y[b][n] = sum_k x[b][k] * W[n][k].
//
// Design (CDNA4, wave64), built so that the VALU work per weight stays far
// below what HBM delivers:
//  * Workgroup = R row tiles (16 rows each) x KSPLIT waves; each wave owns one K
//    slice and first issues the loads of ALL its chunks (one dwordx4 per lane
//    per chunk: 1 KiB per wave, fully coalesced), so the weight stream is in
//    flight at once; the chunks are then consumed in arrival order.
//  * Dot products run on the int8 matrix cores (v_mfma_i32_16x16x64_i8).  The
//    B operand is the weights themselves: Q4 codes come out of the T16 code
//    groups with one AND (plus one shift) per four weights, Q8_0 bytes are used
//    as they are.  Integer accumulation is exact.
//  * The activation is split per 32-block into two int8 limbs,
//    x ~ s * (a + b / 254) with s = amax / 127 (error <= s / 508), staged by
//    each wave for its K slice in LDS.  A rows are (block-of-pair h, limb l,
//    batch b) so each MFMA yields, per weight row, the exact integer dot
//    products of two blocks and both limbs at once; lane group g of the D
//    fragment holds combination (h, l) = (g >> 1, g & 1).
//  * Scales are applied in fp32 once per (row, block): acc += d * s' * D with
//    s' = s or s / 254.  The GGUF offsets are applied through block sums S of
//    the represented activation: Q4_0 y -= 8 d S, Q4_K y -= dmin m_j S_j;
//    Q8_0 is signed.
//  * Batch <= 4 stages the activations in-kernel (no workspace, one launch);
//    batch 5..16 uses a prep kernel that writes the same limbs to a workspace.
//  * Q6_K (batch 1..2): a lane's 16 k of an MFMA step are one 16-element scale
//    group, so the A rows are (scale group, limb) x two batch rows and each
//    lane applies its own group's d * sc; the -32 offset goes through
//    16-element sums of the represented activation.
#include <stdlib.h>

#include "gq_internal.h"

#include "gq_gemv_i8.h"

namespace {

constexpr size_t kLdsWg = 160 * 1024;  // LDS per workgroup on gfx950

// Static LDS of a kernel (its __shared__ arrays), looked up once per kernel:
// the launches check static + dynamic against the workgroup's LDS, so a plan
// that would not fit fails with an error instead of running past its LDS.
// Without a device (host-only plan queries) the attributes are unavailable:
// `otherwise` is returned (kLdsWg: nothing fits; a plan passes its estimate).
size_t kernel_static_lds(const void *kern, size_t otherwise = kLdsWg) {
  hipFuncAttributes a{};
  if (hipFuncGetAttributes(&a, kern) == hipSuccess) return a.sharedSizeBytes;
  (void)hipGetLastError();
  return otherwise;
}

// One weight matrix of a launch: T16 data, its scale-plane offset, output
// y [batch][N], and the end (exclusive) of its workgroup range.
struct GemvSeg {
  const uint8_t *w;
  size_t sc_off;
  float *y;
  int N;
  int wg_end;
};
// FUSE = 0: one matrix.  1: up to 4 matrices sharing x (e.g. q, k, v), each
// with its own workgroup range.  2: gate and up matrices of one FFN: the
// workgroup's row tile 0 is read from seg[0], tile 1 from seg[1] (same rows),
// and y = silu(gate) * up goes to seg[0].y.  With FUSE > 0 and gamma set, x is
// first RMS-normalised per batch row: x * (1 / sqrt(mean(x^2) + eps)) * gamma.
struct GemvFuse {
  GemvSeg seg[4];
  int nseg;
  const float *gamma;
  float eps;
};

template <int FMT, int NBC, int MT, int R, int NCKT, int KSPLIT, bool PREP, int FUSE>
__global__ void __launch_bounds__(64 * KSPLIT)
k_gemv_q(const GemvFuse fz, const float *__restrict__ x, const int8_t *__restrict__ xl_g,
         const float *__restrict__ scl_g, int K, int C, int Kp, int nb) {
  static_assert(FUSE != 2 || R == 2, "gate/up pairs need two row tiles");
  // this workgroup's matrix (wave-uniform selects; no dynamic indexing)
  int si = 0;
  if constexpr (FUSE == 1) {
#pragma unroll
    for (int q = 0; q < 3; ++q) si += (q + 1 < fz.nseg && (int)blockIdx.x >= fz.seg[q].wg_end) ? 1 : 0;
  }
  const GemvSeg s0 = fz.seg[0], s1 = fz.seg[1], s2 = fz.seg[2], s3 = fz.seg[3];
  const uint8_t *const w = si == 0 ? s0.w : si == 1 ? s1.w : si == 2 ? s2.w : s3.w;
  const size_t sc_off = si == 0 ? s0.sc_off : si == 1 ? s1.sc_off : si == 2 ? s2.sc_off : s3.sc_off;
  float *const y = si == 0 ? s0.y : si == 1 ? s1.y : si == 2 ? s2.y : s3.y;
  const int N = si == 0 ? s0.N : si == 1 ? s1.N : si == 2 ? s2.N : s3.N;
  const int wg0 = si == 0 ? 0 : si == 1 ? s0.wg_end : si == 2 ? s1.wg_end : s2.wg_end;
  using F = Fmt<FMT>;
  constexpr int NCK = NCKT;                  // chunks per wave (upper bound, <= MAXC / R)
  static_assert(NCK * R <= F::MAXC, "register budget");
  constexpr int LKMAX = F::CK * NCK;         // slice elements per wave
  constexpr int TPR = LKMAX / 8 / 64;        // 8-element staging tasks per batch row per lane
  constexpr int BPC = F::CK / 32;            // 32-blocks per chunk
  extern __shared__ __attribute__((aligned(16))) unsigned char gq_dyn_lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int g = lane >> 4, r = lane & 15;
  const size_t tile0 = FUSE == 2 ? (size_t)blockIdx.x : (size_t)((int)blockIdx.x - wg0) * R;
  const int ntiles = (int)gq_tiles(N);
  const int c0 = (C * wave) / KSPLIT, c1 = (C * (wave + 1)) / KSPLIT;
  const int nck = c1 - c0;  // <= NCK (host-checked)
  const int k0 = c0 * F::CK, LK = nck * F::CK;
  const bool norm = FUSE > 0 && fz.gamma != nullptr;
  float ssw[NBC];                               // this wave's sum of squares per batch row (norm)
  __shared__ float ssred[FUSE > 0 ? KSPLIT : 1][NBC];  // the waves' sums of squares (norm)
#pragma unroll
  for (int b = 0; b < NBC; ++b) ssw[b] = 0.f;

  // ---- 1. activation loads (fused path), issued before the weights ----------
  float4 xv[PREP ? 1 : NBC * TPR][2];
  bool xin[PREP ? 1 : NBC * TPR];
  if constexpr (!PREP) {
#pragma unroll
    for (int i = 0; i < NBC * TPR; ++i) {
      const int b = i / TPR, e8 = lane + 64 * (i % TPR), k = k0 + 8 * e8;
      xin[i] = b < nb && 8 * e8 < LK && k < K;
      const float4 *p = reinterpret_cast<const float4 *>(x + (xin[i] ? (size_t)b * K + k : 0));
      xv[i][0] = p[0];
      xv[i][1] = p[1];
    }
  }
  float4 gv[FUSE > 0 && !PREP ? TPR : 1][2];
  if constexpr (FUSE > 0 && !PREP) {
    if (norm) {
#pragma unroll
      for (int i = 0; i < TPR; ++i) {
        const int e8 = lane + 64 * i, k = k0 + 8 * e8;
        const bool in = 8 * e8 < LK && k < K;
        const float4 *p = reinterpret_cast<const float4 *>(fz.gamma + (in ? k : 0));
        gv[i][0] = p[0];
        gv[i][1] = p[1];
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. weight loads for every chunk of this wave (clamped, unconditional) -
  // Wave-uniform base addresses, so each load is a scalar base + the lane's
  // fixed offset.
  Chunk<FMT> ch[R][NCK];
  const uint32_t qlane = 16u * (uint32_t)lane;
  const uint32_t slane = (FMT == GQ_FMT_Q4_K || FMT == GQ_FMT_Q6_K) ? 16u * (uint32_t)r
                                                                    : 8u * (uint32_t)r + 4u * (uint32_t)(g >> 1);
  const uint8_t *qbase[R], *sbase[R];
#pragma unroll
  for (int rt = 0; rt < R; ++rt) {
    if constexpr (FUSE == 2) {
      const size_t t = tile0 < (size_t)ntiles ? tile0 : (size_t)ntiles - 1;
      const uint8_t *wr = rt == 0 ? s0.w : s1.w;
      const size_t so = rt == 0 ? s0.sc_off : s1.sc_off;
      qbase[rt] = wr + (t * (size_t)C + c0) * F::QB;
      sbase[rt] = wr + so + (t * (size_t)C + c0) * F::SB;
    } else {
      const size_t t = (tile0 + rt < (size_t)ntiles) ? tile0 + rt : (size_t)ntiles - 1;
      qbase[rt] = w + (t * (size_t)C + c0) * F::QB;
      sbase[rt] = w + sc_off + (t * (size_t)C + c0) * F::SB;
    }
  }
  // Scales (Q8_0; Q4_0 / Q4_K with 16 waves): a wave's chunks of one row tile
  // have one contiguous run of the scale plane (nck x SB bytes, at most
  // 1 KiB), read by one 16-byte load per lane and tile instead of one 4- or
  // 16-byte load per chunk, then passed between lanes through LDS: fewer
  // vector-memory instructions per CU (a timing-only build without the
  // per-chunk scale loads ran 0.6 us faster on Q4_0 14336 x 4096, compute
  // removed).  Measured with the compute in place: Q8_0 4096 x 4096 4.89 ->
  // 4.67 us, Q4_0 4096 x 14336 (16 waves) 7.97 -> 7.78 us; Q4_0 / Q4_K with 8
  // waves unchanged or up to 1 % slower, so they keep the per-chunk loads.
  // Lanes past the run re-read its last 16 bytes.  The loads go out before the
  // weight loads, so waiting for them waits for no weight.
  constexpr bool SDMA = FMT == GQ_FMT_Q8_0 || (KSPLIT == 16 && (FMT == GQ_FMT_Q4_0 || FMT == GQ_FMT_Q4_K));
  static_assert(!SDMA || NCK * F::SB <= 1024, "one 16-byte load per lane and row tile");
  __shared__ __attribute__((aligned(16))) unsigned char sdm[SDMA ? KSPLIT : 1][SDMA ? R : 1][SDMA ? 1024 : 16];
  gq_u4 sreg[SDMA ? R : 1];
  if constexpr (SDMA) {
    const int span = (nck > 0 ? nck : 1) * F::SB;
    const uint32_t soff = 16u * (uint32_t)lane < (uint32_t)span ? 16u * (uint32_t)lane : (uint32_t)span - 16u;
#pragma unroll
    for (int rt = 0; rt < R; ++rt) sreg[rt] = gq_ld16_nt(sbase[rt] + soff);
  }
  // Surplus loads re-read the wave's last chunk (its first one when the wave
  // has no chunk: c0 < C always holds), never outside the tensor.  All loads
  // are issued up front, tile by tile (each tile's chunks are one contiguous
  // run of memory; measured faster than interleaving the tiles chunk by chunk).
#pragma unroll
  for (int rt = 0; rt < R; ++rt)
#pragma unroll
    for (int i = 0; i < NCK; ++i) {
      const int ii = i < nck ? i : (nck > 0 ? nck - 1 : 0);
      if constexpr (SDMA)
        load_chunk_codes<FMT>(qbase[rt] + (size_t)ii * F::QB, qlane, ch[rt][i]);
      else
        load_chunk<FMT>(qbase[rt] + (size_t)ii * F::QB, sbase[rt] + (size_t)ii * F::SB, qlane, slane, ch[rt][i]);
    }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. activation limbs --------------------------------------------------
  const int8_t *limbs;
  const float *scl;
  const int8_t *zero;
  int lds_ld, scl_ld, kbase;  // limb row stride, scale row stride (blocks), slice origin
  if constexpr (!PREP) {
    // limb rows for the nb batch rows present only (rows nb..NBC-1 of the A
    // operand never carry data): batch 3 takes three quarters of batch 4's LDS
    const XlLayout L = xl_layout(F::CK * ((C + KSPLIT - 1) / KSPLIT), nb < NBC ? nb : NBC);
    unsigned char *base = gq_dyn_lds + (size_t)wave * L.wave_bytes;
    int8_t *lm = reinterpret_cast<int8_t *>(base);
    float *sc = reinterpret_cast<float *>(base + L.scl_off);
    const int nblk = L.lk / 32;
    for (int o = 16 * lane; o < L.lk; o += 1024)
      *reinterpret_cast<gq_u4 *>(base + L.zero_off + o) = gq_u4{0u, 0u, 0u, 0u};
    // RMS normalisation (fused entry points): y = inv_rms * (W (x * gamma)),
    // inv_rms = 1 / sqrt(mean(x^2) + eps) a scalar per batch row, so the
    // staging multiplies by gamma only (the limb split is per-block scaled,
    // hence indifferent to the factor) and each wave only records the sum of
    // squares of its slice; the factor is applied to the finished dot
    // products, after the reduction barrier the K split needs anyway
    if constexpr (FUSE > 0) {
      if (norm) {
        float ss[NBC];
#pragma unroll
        for (int b = 0; b < NBC; ++b) ss[b] = 0.f;
#pragma unroll
        for (int i = 0; i < NBC * TPR; ++i) {
          const float vv[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w,
                               xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) ss[i / TPR] += xin[i] ? vv[e] * vv[e] : 0.f;
        }
#pragma unroll
        for (int b = 0; b < NBC; ++b) {
          ssw[b] = wave_sum(ss[b]);
          if (lane == 0) ssred[wave][b] = ssw[b];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NBC * TPR; ++i) {
      const int b = i / TPR, e8 = lane + 64 * (i % TPR);
      float v[8] = {xv[i][0].x, xv[i][0].y, xv[i][0].z, xv[i][0].w, xv[i][1].x, xv[i][1].y, xv[i][1].z, xv[i][1].w};
      if constexpr (FUSE > 0) {
        if (norm) {
          const int ti = i % TPR;
          const float gg[8] = {gv[ti][0].x, gv[ti][0].y, gv[ti][0].z, gv[ti][0].w,
                               gv[ti][1].x, gv[ti][1].y, gv[ti][1].z, gv[ti][1].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = v[e] * gg[e];
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = xin[i] ? v[e] : 0.f;
      const float amax = quad_max(abs_max_bits8(v));
      // 127 / amax to one ulp: a (represented) limb split needs no correctly
      // rounded quotient, the scale sx below is what the products use.  A
      // block holding a NaN or Inf gets inv = 0 (zero limbs) and sx = NaN or
      // Inf, so every output that reads the block comes out NaN.
      const float inv = amax > 0.f ? 127.0f * __builtin_amdgcn_rcpf(amax) : 0.f;
      const float sx = amax * (1.0f / 127.0f);
      uint32_t la[2], lb[2];
      // block sum of the represented values: offsets and mins then act on
      // exactly the activation the integer products see
      // Q6_K (a scale per 16 elements): the two 16-element sums of the block,
      // in the float4's second and fourth slots
      const int t8 = split8(v, inv, la, lb);
      float s, s_hi = 0.f;
      if constexpr (FMT == GQ_FMT_Q6_K) {
        const int p16 = t8 + __builtin_amdgcn_mov_dpp(t8, 0xB1, 0xF, 0xF, false);  // lanes 4j + {0,1} | {2,3}
        s = (float)p16 * (sx * (1.0f / 254.0f));
        s_hi = (float)__builtin_amdgcn_mov_dpp(p16, 0x4E, 0xF, 0xF, false) * (sx * (1.0f / 254.0f));
      } else {
        s = (float)quad_sum(t8) * (sx * (1.0f / 254.0f));
      }
      if (b < nb && 8 * e8 < L.lk) {
        *reinterpret_cast<gq_u2 *>(lm + (2 * b) * L.lk + 8 * e8) = gq_u2{la[0], la[1]};
        *reinterpret_cast<gq_u2 *>(lm + (2 * b + 1) * L.lk + 8 * e8) = gq_u2{lb[0], lb[1]};
        if ((lane & 3) == 0)
          *reinterpret_cast<gq_f4 *>(sc + 4 * (b * nblk + (e8 >> 2))) = gq_f4{sx, s, sx * (1.0f / 254.0f), s_hi};
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    limbs = lm;
    scl = sc;
    zero = reinterpret_cast<const int8_t *>(base + L.zero_off);
    lds_ld = L.lk;
    scl_ld = nblk;
    kbase = k0;
  } else {
    limbs = xl_g;
    scl = scl_g;
    zero = xl_g + (size_t)2 * nb * Kp;
    lds_ld = Kp;
    scl_ld = Kp / 32;
    kbase = 0;
  }

  // A operand: lane (row r, group g) is combination c = r >> 2 = (h, l) of
  // batch row 4 * mt + (r & 3); it carries data only where its lane group
  // covers block h of the MFMA pair ((g >> 1) == h), zeros otherwise.
  // Q6_K (scales per 16 elements): row r is combination c = r >> 1 = (scale
  // group q = r >> 2, limb l = (r >> 1) & 1) of batch row r & 1 (two batch
  // rows per MFMA), with data where the lane group is that scale group
  // (g == q); D lane (g, r') then holds group g's dots: value v is limb v >> 1
  // of batch row v & 1.
  const int8_t *abase[MT];
  if constexpr (FMT == GQ_FMT_Q6_K) {
    static_assert(MT == 1 && NBC <= 2, "Q6_K: batch 1..2");
    const int q = r >> 2, l = (r >> 1) & 1, b = r & 1;
    const bool act = g == q && b < nb && b < NBC;
    abase[0] = act ? limbs + (size_t)(2 * b + l) * lds_ld + (k0 - kbase) + 16 * g : zero + (k0 - kbase);
  } else {
    const int c = r >> 2, h = c >> 1, l = c & 1;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int b = 4 * mt + (r & 3);
      const bool act = ((g >> 1) == h) && b < nb && (r & 3) < NBC;
      abase[mt] = act ? limbs + (size_t)(2 * b + l) * lds_ld + (k0 - kbase) + 32 * h + 16 * (g & 1)
                      : zero + (k0 - kbase);
    }
  }
  // D side: this lane's combination (h', l') = (g >> 1, g & 1)
  const int hp = g >> 1, lp = g & 1;

  float acc[R][MT][NBC], cor[R][MT][NBC];
#pragma unroll
  for (int rt = 0; rt < R; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < NBC; ++v) acc[rt][mt][v] = cor[rt][mt][v] = 0.f;

  if constexpr (SDMA) {  // the scale runs -> this wave's LDS slots (read back per chunk)
#pragma unroll
    for (int rt = 0; rt < R; ++rt) *reinterpret_cast<gq_u4 *>(&sdm[wave][rt][16 * lane]) = sreg[rt];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }

  // ---- 4. consume the chunks -------------------------------------------------
  // Chunk i of this wave; with a full chunk list (the common case) the loop
  // is straight-line code, so the waits on the weight loads stay in order.
  auto consume = [&](int i) {
    if constexpr (SDMA) {  // this chunk's scales from the LDS copy
#pragma unroll
      for (int rt = 0; rt < R; ++rt) {
        const unsigned char *sp = &sdm[wave][rt][i * F::SB + slane];
        if constexpr (FMT == GQ_FMT_Q4_K)
          ch[rt][i].meta = *reinterpret_cast<const gq_u4 *>(sp);
        else
          ch[rt][i].d = *reinterpret_cast<const uint32_t *>(sp);
      }
    }
#pragma unroll
    for (int m = 0; m < F::STEPS; ++m) {
      const int koff = i * F::CK + 64 * m;
      const int blk = (k0 - kbase) / 32 + i * BPC + 2 * m + hp;  // this lane's block, in scale rows
      if constexpr (FMT == GQ_FMT_Q6_K) {
        // lane (g, r): scale group 4 m + g of row r; D value v = (limb v >> 1,
        // batch row v & 1); the 16-element sums give the -32 offset
        const gq_i4 a0 = *reinterpret_cast<const gq_i4 *>(abase[0] + koff);
        float sxl[NBC], szl[NBC], s16[NBC];
#pragma unroll
        for (int v = 0; v < NBC; ++v) {
          const gq_f4 f = *reinterpret_cast<const gq_f4 *>(scl + 4 * ((size_t)(v < nb ? v : 0) * scl_ld + blk));
          sxl[v] = f[0];
          szl[v] = f[2];
          s16[v] = (g & 1) ? f[3] : f[1];
        }
#pragma unroll
        for (int rt = 0; rt < R; ++rt) {
          const Chunk<FMT> &cc = ch[rt][i];
          const gq_u4 &qq = (m < 2) ? cc.qa : cc.qb;
          gq_i4 bop = codes16(qq[2 * (m & 1)], qq[2 * (m & 1) + 1]);
          const uint32_t hw = cc.hi[m];
#pragma unroll
          for (int e = 0; e < 4; ++e) bop[e] |= (int)(((hw >> (2 * e)) & 0x03030303u) << 4);  // codes 0..63
          const float ws = h16lo(cc.d) * (float)(int8_t)((cc.sc[m] >> (8 * g)) & 0xFFu);
          const gq_i4 D = mfma_i8(a0, bop);
#pragma unroll
          for (int v = 0; v < NBC; ++v) {
            acc[rt][0][v] += (ws * sxl[v]) * (float)D[v] + (ws * szl[v]) * (float)D[2 + v];
            cor[rt][0][v] += ws * s16[v];
          }
        }
      } else {
        gq_i4 a[MT];
        float2 sv[MT][NBC];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          a[mt] = *reinterpret_cast<const gq_i4 *>(abase[mt] + koff);
#pragma unroll
          for (int v = 0; v < NBC; ++v) {
            const int b = 4 * mt + v;
            sv[mt][v] =
                *reinterpret_cast<const float2 *>(scl + 4 * ((size_t)(b < nb ? b : 0) * scl_ld + blk) + 2 * lp);
          }
        }
#pragma unroll
        for (int rt = 0; rt < R; ++rt) {
          const Chunk<FMT> &cc = ch[rt][i];
          gq_i4 bop;
          float ws, wm = 0.f;  // weight scale and offset/min factor of block (2m + h')
          if constexpr (FMT == GQ_FMT_Q4_0) {
            bop = codes16(cc.q[2 * m], cc.q[2 * m + 1]);
            ws = m ? h16hi(cc.d) : h16lo(cc.d);
            wm = ws;
          } else if constexpr (FMT == GQ_FMT_Q8_0) {
            const gq_u4 &qq = m ? cc.q1 : cc.q0;
            bop = gq_i4{(int)qq[0], (int)qq[1], (int)qq[2], (int)qq[3]};
            ws = m ? h16hi(cc.d) : h16lo(cc.d);
          } else {
            const uint32_t w0 = (m < 2) ? cc.qa[2 * (m & 1)] : cc.qb[2 * (m & 1)];
            const uint32_t w1 = (m < 2) ? cc.qa[2 * (m & 1) + 1] : cc.qb[2 * (m & 1) + 1];
            bop = codes16(w0, w1);
            const uint32_t wsc = hp ? cc.meta[2] : cc.meta[1];
            const uint32_t byte = (wsc >> (8 * m)) & 0xFFu;
            const uint32_t b3 = (cc.meta[3] >> (8 * m + 4 * hp)) & 15u;
            ws = h16lo(cc.meta[0]) * (float)(byte & 63u);
            wm = h16hi(cc.meta[0]) * (float)((byte >> 6) | (b3 << 2));
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const gq_i4 D = mfma_i8(a[mt], bop);
#pragma unroll
            for (int v = 0; v < NBC; ++v) {
              acc[rt][mt][v] += (ws * sv[mt][v].x) * (float)D[v];
              if constexpr (FMT != GQ_FMT_Q8_0) cor[rt][mt][v] += wm * sv[mt][v].y;
            }
          }
        }
      }
    }
  };
  if (nck == NCK) {
#pragma unroll
    for (int i = 0; i < NCK; ++i) consume(i);
  } else {
#pragma unroll
    for (int i = 0; i < NCK; ++i)
      if (i < nck) consume(i);
  }

  // ---- 5. reduce: lane groups (4 combinations), then the KSPLIT waves --------
  constexpr float OFF = (FMT == GQ_FMT_Q4_0) ? 8.f : (FMT == GQ_FMT_Q4_K) ? 1.f : (FMT == GQ_FMT_Q6_K) ? 32.f : 0.f;
  float part[R][MT][NBC];
#pragma unroll
  for (int rt = 0; rt < R; ++rt)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < NBC; ++v) {
        part[rt][mt][v] = sum_lane_groups(acc[rt][mt][v] - OFF * cor[rt][mt][v]);
      }
  if constexpr (KSPLIT > 1) {
    __shared__ float red[KSPLIT][R * MT * NBC][16];
    if (g == 0) {
#pragma unroll
      for (int rt = 0; rt < R; ++rt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int v = 0; v < NBC; ++v) red[wave][(rt * MT + mt) * NBC + v][r] = part[rt][mt][v];
    }
    __syncthreads();
    if (wave != 0 || g != 0) return;
#pragma unroll
    for (int rt = 0; rt < R; ++rt)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < NBC; ++v) {
          float s = 0.f;
#pragma unroll
          for (int q = 0; q < KSPLIT; ++q) s += red[q][(rt * MT + mt) * NBC + v][r];
          part[rt][mt][v] = s;
        }
  } else if (g != 0) {
    return;
  }
  if constexpr (FUSE > 0) {
    if (norm) {
#pragma unroll
      for (int v = 0; v < NBC; ++v) {
        float t = ssw[v];
        if constexpr (KSPLIT > 1) {  // (ordered by the reduction barrier)
          t = 0.f;
#pragma unroll
          for (int q = 0; q < KSPLIT; ++q) t += ssred[q][v];
        }
        const float inv = 1.0f / sqrtf(t / (float)K + fz.eps);
#pragma unroll
        for (int rt = 0; rt < R; ++rt)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) part[rt][mt][v] *= inv;
      }
    }
  }
  if constexpr (FUSE == 2) {
    const size_t row = tile0 * 16 + r;
    if (row < (size_t)N) {
#pragma unroll
      for (int v = 0; v < NBC; ++v) {
        if (v < nb) {
          const float gt = part[0][0][v], up = part[1][0][v];
          y[(size_t)v * N + row] = gt / (1.0f + expf(-gt)) * up;  // silu(gate) * up
        }
      }
    }
    return;
  }
#pragma unroll
  for (int rt = 0; rt < R; ++rt) {
    const size_t row = (tile0 + rt) * 16 + r;
    if (row >= (size_t)N) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < NBC; ++v) {
        const int b = 4 * mt + v;
        if (b < nb) y[(size_t)b * N + row] = part[rt][mt][v];
      }
  }
}

// GQ_GEMV_KSPLIT=2|4|8|16 and GQ_GEMV_R=1|2 override the launch heuristic
// (for tuning).
int env_int(const char *name) {
  const char *e = getenv(name);
  return e ? atoi(e) : 0;
}

template <int FMT, int NBC, int MT, int R, bool PREP, bool HALF>
int launch_r(const void *packed, const float *x, const void *ws, float *y, int N, int K, int nb, int ks,
             hipStream_t s) {
  using F = Fmt<FMT>;
  constexpr int NCKT = F::MAXC / R / (HALF ? 2 : 1);
  const int C = (int)gq_chunks(FMT, K);
  const int Kp = (int)gq_kpad(FMT, K);
  const size_t tiles = gq_tiles(N);
  const size_t wgs = (tiles + R - 1) / R;
  const size_t sc_off = gq_sc_plane_offset(FMT, N, K);
  const int8_t *xl = PREP ? (const int8_t *)ws : nullptr;
  const float *scl = PREP ? (const float *)((const uint8_t *)ws + gq_xl_bytes(FMT, K, nb)) : nullptr;
  const size_t lds = PREP ? 0 : (size_t)ks * xl_layout(F::CK * ((C + ks - 1) / ks), nb < NBC ? nb : NBC).wave_bytes;
  GemvFuse fz{};
  fz.seg[0] = GemvSeg{(const uint8_t *)packed, sc_off, y, N, (int)wgs};
  fz.nseg = 1;
#define GQ_LAUNCH_KS(KS)                                                                                         \
  {                                                                                                              \
    const void *kern = (const void *)k_gemv_q<FMT, NBC, MT, R, NCKT, KS, PREP, 0>;                              \
    static const size_t st = kernel_static_lds(kern);                                                           \
    if (lds + st > kLdsWg) return GQ_ERR_UNSUPPORTED;                                                            \
    hipLaunchKernelGGL((k_gemv_q<FMT, NBC, MT, R, NCKT, KS, PREP, 0>), dim3((unsigned)wgs), dim3(64 * KS), lds, \
                       s, fz, x, xl, scl, K, C, Kp, nb);                                                         \
  }
  switch (ks) {
  case 2: GQ_LAUNCH_KS(2); break;
  case 4: GQ_LAUNCH_KS(4); break;
  case 8: GQ_LAUNCH_KS(8); break;
  default: GQ_LAUNCH_KS(16); break;
  }
#undef GQ_LAUNCH_KS
  return gq_last_launch();
}

}  // namespace

// Launch plan: R row tiles per workgroup (2 when there are many tiles: halves
// the activation staging per weight) and KSPLIT waves, so that every wave holds
// at most MAXC / R chunks and the grid has enough waves to keep HBM busy.
// Every wave's chunk range [C*w/KSPLIT, C*(w+1)/KSPLIT) lies inside [0, C).
// LDS bytes of the in-kernel activation staging (batch <= 4) for a plan: one
// limb region per wave of KSPLIT.
static size_t q_staging_lds(int fmt, size_t K, int batch, int ks) {
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt;
  const int ck = (f == GQ_FMT_Q4_K || f == GQ_FMT_Q6_K) ? 256 : 128;
  const int C = (int)gq_chunks(f, K);
  return (size_t)ks * (size_t)xl_layout(ck * ((C + ks - 1) / ks), batch).wave_bytes;
}
// The int8 kernel's static LDS beside the staging (k_gemv_q's arrays): the
// scale-run copies (sdm, where the kernel loads scales by run), the K-split
// reduction tiles (red) and the norm sums (ssred); batch <= 4 (NBC 1, 2 or 4,
// MT 1).
static size_t q_static_lds(int fmt, int batch, int R, int ks, bool fuse) {
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt;
  const size_t nbc = batch == 1 ? 1 : batch == 2 ? 2 : 4;
  const bool sdma = f == GQ_FMT_Q8_0 || (ks == 16 && (f == GQ_FMT_Q4_0 || f == GQ_FMT_Q4_K));
  const size_t sdm = sdma ? (size_t)ks * R * 1024 : 16;
  const size_t red = (size_t)ks * R * nbc * 16 * 4;
  const size_t ssred = (fuse ? (size_t)ks : 1) * nbc * 4;
  return sdm + red + ssred;
}
constexpr size_t kLdsMax = 160 * 1024;  // LDS per workgroup on gfx950

static int q_plan(int fmt, size_t N, size_t K, int batch, int *R_out, int *ksplit_out, int *chunks_per_wave_out) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt;
  const int maxc = f == GQ_FMT_Q4_K   ? Fmt<GQ_FMT_Q4_K>::MAXC
                   : f == GQ_FMT_Q6_K ? Fmt<GQ_FMT_Q6_K>::MAXC
                   : f == GQ_FMT_Q8_0 ? Fmt<GQ_FMT_Q8_0>::MAXC
                                      : Fmt<GQ_FMT_Q4_0>::MAXC;
  const int C = (int)gq_chunks(f, K);
  const size_t tiles = gq_tiles(N);
  const int mt = batch <= 4 ? 1 : (batch + 3) / 4;
  int R = (tiles >= 512 && C >= 4) ? 2 : 1;
  if (R == 2) {
    // one-tile workgroups run best where every CU holds the same number of
    // tiles or at most three (measured, Q4_0 / Q4_K / Q8_0 at K = 4096:
    // 10240 rows 6.1 vs 6.9 us, 16384 rows 7.7 vs 8.1 us); two-tile ones
    // where the tiles per CU fall in between (14336 rows: 7.4 vs 7.8 us)
    const int cus0 = gq_device_cus();
    const size_t cus = cus0 > 0 ? (size_t)cus0 : 256;
    const size_t rounds = (tiles + cus - 1) / cus;
    if (rounds <= 3 || (tiles % cus == 0 && rounds <= 8)) R = 1;
  }
  const int er = env_int("GQ_GEMV_R");
  if (er == 1 || er == 2) R = er;
  if ((C + 15) / 16 > maxc / 2) R = 1;  // very long K: keep every register for chunks
  // 1024-thread workgroups cap a wave at 128 VGPRs: keep wide batches at <= 8 waves
  const int cap = mt >= 2 ? 8 : 16;
  if (R == 2 && (C + cap - 1) / cap > maxc / 2) R = 1;
  // fewest waves per workgroup that fit the register budget (measured best:
  // long per-wave chunk lists, every workgroup resident in the first round),
  // more only when the grid would otherwise have too few waves
  // a single-tile workgroup aims at maxc / 2 chunks per wave (half the
  // activation staging and registers per wave), when 16 waves can cover K so
  int target = maxc / R;
  if (R == 1 && (C + 15) / 16 <= maxc / 2) target = maxc / 2;
  int ks = 2;
  while (ks < 16 && (C + ks - 1) / ks > target) ks *= 2;
  // (grown to 512 waves and 8 per workgroup at most: small grids ran faster
  // so than at 1024 waves / 16 per workgroup -- batch 1 at K = 4096, 4 to 64
  // workgroups: Q4_0 2.7-2.9 us at 8 waves against 3.2-3.7 at 16, Q4_K 2.9-3.1
  // against 3.4-3.6, Q8_0 512 rows 3.26 against 4.36; 2048 x 2048 Q4_0 2.65 us
  // at 4 against 2.85 at 8; the register target above may still ask for 16)
  while (ks < cap && ks < 8 && ((tiles + R - 1) / R) * ks < 512 && 2 * ks <= C) ks *= 2;
  // batch <= 4 stages the activation limbs in LDS, about (2 batch + 1) bytes
  // per k of the padded K: a smaller split pads less (Q4_K 4096 x 14336 at
  // batch 4: 180 KiB at 16 waves, 154 KiB at 8), where the registers allow
  while (batch <= 4 && ks > 2 && q_staging_lds(fmt, K, batch, ks) + q_static_lds(fmt, batch, R, ks, false) > kLdsMax &&
         (C + ks / 2 - 1) / (ks / 2) <= maxc / R)
    ks /= 2;
  const int e = env_int("GQ_GEMV_KSPLIT");
  if ((e == 2 || e == 4 || e == 8 || e == 16) && (C + e - 1) / e <= maxc / R) ks = e;
  if (R_out) *R_out = R;
  if (ksplit_out) *ksplit_out = ks;
  if (chunks_per_wave_out) *chunks_per_wave_out = (C + ks - 1) / ks;
  return GQ_OK;
}

// The plan of the kernel gq_gemv launches for (fmt, N, K, batch): the int8
// kernel above, or from batch gq_gemv_h_min() on the fp16 batch kernel.
static bool gq_gemv_on_h(int fmt, size_t N, size_t K, int batch);

extern "C" int gq_gemv_plan(int fmt, size_t N, size_t K, int batch, int *R_out, int *ksplit_out,
                            int *chunks_per_wave_out) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  if (!gq_gemv_on_h(fmt, N, K, batch)) return q_plan(fmt, N, K, batch, R_out, ksplit_out, chunks_per_wave_out);
  int R = 1, ks = 1, cpw = 0;
  if (gq_gemv_h1_plan(fmt, N, K, batch, &R, &ks, &cpw) != GQ_OK) GQ_TRY(gq_gemv_h_plan(fmt, N, K, batch, &R, &ks, &cpw));
  if (R_out) *R_out = R;
  if (ksplit_out) *ksplit_out = ks;
  if (chunks_per_wave_out) *chunks_per_wave_out = cpw;
  return GQ_OK;
}

namespace {

template <int FMT, int NBC, int MT, bool PREP>
int launch_shape(const void *packed, const float *x, const void *ws, float *y, int N, int K, int nb, hipStream_t s) {
  int R = 1, ks = 2, cpw = 0;
  GQ_TRY(q_plan(FMT, N, K, nb, &R, &ks, &cpw));
  if (cpw > Fmt<FMT>::MAXC / R) return GQ_ERR_INVALID_ARGS;  // the kernel's register budget
  if (R == 2) return launch_r<FMT, NBC, MT, 2, PREP, false>(packed, x, ws, y, N, K, nb, ks, s);
  if (!PREP && cpw <= Fmt<FMT>::MAXC / 2)
    return launch_r<FMT, NBC, MT, 1, PREP, true>(packed, x, ws, y, N, K, nb, ks, s);
  return launch_r<FMT, NBC, MT, 1, PREP, false>(packed, x, ws, y, N, K, nb, ks, s);
}

template <int FMT>
int launch_gemv(const void *packed, const float *x, const void *ws, float *y, int N, int K, int nb, hipStream_t s) {
  if (x) {  // fused staging, batch <= 4
    if (nb == 1) return launch_shape<FMT, 1, 1, false>(packed, x, nullptr, y, N, K, nb, s);
    if (nb == 2) return launch_shape<FMT, 2, 1, false>(packed, x, nullptr, y, N, K, nb, s);
    return launch_shape<FMT, 4, 1, false>(packed, x, nullptr, y, N, K, nb, s);
  }
  if (nb <= 4) return launch_shape<FMT, 4, 1, true>(packed, nullptr, ws, y, N, K, nb, s);
  if (nb <= 8) return launch_shape<FMT, 4, 2, true>(packed, nullptr, ws, y, N, K, nb, s);
  if (nb <= 12) return launch_shape<FMT, 4, 3, true>(packed, nullptr, ws, y, N, K, nb, s);
  return launch_shape<FMT, 4, 4, true>(packed, nullptr, ws, y, N, K, nb, s);
}

int dispatch(int fmt, const void *packed, const float *x, const void *ws, float *y, int N, int K, int nb,
             hipStream_t s) {
  if (fmt == GQ_FMT_Q6_K) {  // fused staging, batch 1..2 only
    if (!x || nb > 2) return GQ_ERR_UNSUPPORTED;
    return nb == 1 ? launch_shape<GQ_FMT_Q6_K, 1, 1, false>(packed, x, nullptr, y, N, K, nb, s)
                   : launch_shape<GQ_FMT_Q6_K, 2, 1, false>(packed, x, nullptr, y, N, K, nb, s);
  }
  switch (fmt) {
  case GQ_FMT_Q4_0: return launch_gemv<GQ_FMT_Q4_0>(packed, x, ws, y, N, K, nb, s);
  case GQ_FMT_Q8_0: return launch_gemv<GQ_FMT_Q8_0>(packed, x, ws, y, N, K, nb, s);
  default: return launch_gemv<GQ_FMT_Q4_K>(packed, x, ws, y, N, K, nb, s);
  }
}

}  // namespace

// batch sizes whose activations are staged in-kernel (no workspace)
static inline bool gq_gemv_fused(int batch) { return batch <= 4; }

// smallest batch that gq_gemv runs on the fp16 batch kernel (GQ_GEMV_H_MIN
// overrides it, for tuning)
int gq_gemv_h_min(void) {
  const char *e = getenv("GQ_GEMV_H_MIN");
  const int v = e ? atoi(e) : 0;
  return (v >= 1 && v <= GQ_MAX_BATCH + 1) ? v : 5;
}


// Which kernel gq_gemv uses: the fp16 batch kernel from gq_gemv_h_min() on,
// for Q6_K beyond batch 2 (its int8 MFMA rows hold two batch rows), where K
// is too long for the int8 kernel's registers (more than 16 waves x MAXC
// chunks: K > 16384), and where its activation staging would not fit the LDS
// (batch 3..4 with K near 16384: Q4_K 4096 x 14336 at batch 4 needs 176 KiB);
// the int8 kernel otherwise.
static bool gq_gemv_on_h(int fmt, size_t N, size_t K, int batch) {
  if (batch >= gq_gemv_h_min() || (gq_fmt_is_q6k(fmt) && batch > 2)) return true;
  int R = 1, ks = 2, cpw = 0;
  if (q_plan(fmt, N, K, batch, &R, &ks, &cpw) != GQ_OK) return true;
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt;
  const int maxc = (f == GQ_FMT_Q4_K || f == GQ_FMT_Q6_K) ? 4 : 8;
  if (cpw > maxc / R) return true;
  // Q8_0 chunks (8 registers a lane) at batch 3..4 with 16 waves (128
  // registers a wave) spill: 4096 x 14336 batch 3 24.7 us against 17.4 on the
  // fp16 kernel
  if (f == GQ_FMT_Q8_0 && batch >= 3 && batch <= 4 && ks == 16 && cpw > maxc / 2) return true;
  return batch <= 4 && q_staging_lds(fmt, K, batch, ks) + q_static_lds(fmt, batch, R, ks, false) > kLdsMax;
}

extern "C" size_t gq_gemv_workspace_bytes(int fmt, size_t K, int batch) {
  if (!gq_fmt_valid(fmt) || gq_fmt_is_q6k(fmt) || batch < 1 || batch > GQ_MAX_BATCH || K > GQ_MAX_DIM) return 0;
  return gq_xl_bytes(fmt, K, batch) + gq_scl_bytes(fmt, K, batch);
}

extern "C" int gq_gemv_prep(int fmt, const float *x, size_t K, int batch, void *ws, size_t ws_bytes,
                            void *stream) {
  GQ_TRY(gq_check_shape(fmt, 0, K));
  GQ_CHECK(!gq_fmt_is_q6k(fmt), GQ_ERR_UNSUPPORTED);
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(x && ws, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(ws_bytes >= gq_gemv_workspace_bytes(fmt, K, batch), GQ_ERR_WORKSPACE);
  if (K == 0) return GQ_OK;
  return gq_launch_prep_x(fmt, x, ws, batch, (int)K, (hipStream_t)stream);
}

extern "C" int gq_gemv_prepped(int fmt, const void *packed, const void *ws, float *y, size_t N, size_t K,
                               int batch, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(!gq_fmt_is_q6k(fmt), GQ_ERR_UNSUPPORTED);
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(packed && ws && y, GQ_ERR_INVALID_ARGS);
  if (N == 0) return GQ_OK;
  if (K == 0) return gq_fill_zero(y, N * batch, (hipStream_t)stream);
  return dispatch(gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt, packed, nullptr, ws, y, (int)N, (int)K, batch,
                  (hipStream_t)stream);
}

extern "C" int gq_gemv(int fmt, const void *packed, const float *x, float *y, size_t N, size_t K, int batch,
                       void *ws, size_t ws_bytes, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(batch >= 1 && batch <= GQ_MAX_BATCH, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(packed && x && y, GQ_ERR_INVALID_ARGS);
  if (N == 0) return GQ_OK;
  if (K == 0) return gq_fill_zero(y, N * batch, (hipStream_t)stream);
  // wide batches, and Q6_K beyond batch 2, run on the fp16 matrix-core kernel
  if (gq_gemv_on_h(fmt, N, K, batch))
    return gq_launch_gemv_h(fmt, packed, x, y, (int)N, (int)K, batch, (hipStream_t)stream);
  if (gq_gemv_fused(batch))
    return dispatch(gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : gq_fmt_is_q6k(fmt) ? GQ_FMT_Q6_K : fmt, packed, x, nullptr,
                    y, (int)N, (int)K, batch, (hipStream_t)stream);
  size_t need = gq_gemv_workspace_bytes(fmt, K, batch);
  if (!ws) {
    GQ_TRY(gq_default_workspace(need, &ws));
    ws_bytes = need;
  }
  GQ_TRY(gq_gemv_prep(fmt, x, K, batch, ws, ws_bytes, stream));
  return gq_gemv_prepped(fmt, packed, ws, y, N, K, batch, stream);
}

// ---- fused entry points: several matrices sharing x, gate/up with SwiGLU ----
namespace {

// waves per workgroup for a forced R (the q_plan rules for a given R)
int ks_for(int fmt, size_t wgs, int C, int R) {
  const int f = gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt;
  const int maxc = f == GQ_FMT_Q4_K ? Fmt<GQ_FMT_Q4_K>::MAXC : Fmt<GQ_FMT_Q4_0>::MAXC;
  int ks = 2;
  while (ks < 16 && (C + ks - 1) / ks > maxc / R) ks *= 2;
  if ((C + ks - 1) / ks > maxc / R) return 0;  // K too long for one wave's registers
  while (ks < 8 && wgs * ks < 1024 && 2 * ks <= C) ks *= 2;
  return ks;
}

// HALF: register room for MAXC / R / 2 chunks per wave where the plan needs no
// more (fewer surplus loads, fewer registers)
// dry: only the checks (the staging fits the LDS), no launch
template <int FMT, int NBC, int R, int FUSE, bool HALF>
int launch_fused_nbc(const GemvFuse &fz, size_t wgs, int ks, const float *x, int K, int nb, hipStream_t s,
                     bool dry) {
  using F = Fmt<FMT>;
  constexpr int NCKT = F::MAXC / R / (HALF ? 2 : 1);
  const int C = (int)gq_chunks(FMT, K);
  const int Kp = (int)gq_kpad(FMT, K);
  if ((C + ks - 1) / ks > NCKT) return GQ_ERR_INVALID_ARGS;
  const size_t lds = (size_t)ks * xl_layout(F::CK * ((C + ks - 1) / ks), nb < NBC ? nb : NBC).wave_bytes;
  if (lds > kLdsMax) return GQ_ERR_UNSUPPORTED;  // (long K at batch 3..4)
#define GQ_LAUNCH_F(KS)                                                                                        \
  {                                                                                                            \
    const void *kern = (const void *)k_gemv_q<FMT, NBC, 1, R, NCKT, KS, false, FUSE>;                         \
    static const size_t st = kernel_static_lds(kern, q_static_lds(FMT, nb, R, KS, FUSE > 0));                  \
    if (lds + st > kLdsWg) return GQ_ERR_UNSUPPORTED;                                                          \
    if (dry) return GQ_OK;                                                                                     \
    hipLaunchKernelGGL((k_gemv_q<FMT, NBC, 1, R, NCKT, KS, false, FUSE>), dim3((unsigned)wgs), dim3(64 * KS), \
                       lds, s, fz, x, nullptr, nullptr, K, C, Kp, nb);                                         \
  }
  switch (ks) {
  case 2: GQ_LAUNCH_F(2); break;
  case 4: GQ_LAUNCH_F(4); break;
  case 8: GQ_LAUNCH_F(8); break;
  default: GQ_LAUNCH_F(16); break;
  }
#undef GQ_LAUNCH_F
  return gq_last_launch();
}

template <int FMT, int R, int FUSE, bool HALF>
int launch_fused_h(const GemvFuse &fz, size_t wgs, int ks, const float *x, int K, int nb, hipStream_t s, bool dry) {
  if (nb == 1) return launch_fused_nbc<FMT, 1, R, FUSE, HALF>(fz, wgs, ks, x, K, nb, s, dry);
  if (nb == 2) return launch_fused_nbc<FMT, 2, R, FUSE, HALF>(fz, wgs, ks, x, K, nb, s, dry);
  return launch_fused_nbc<FMT, 4, R, FUSE, HALF>(fz, wgs, ks, x, K, nb, s, dry);
}

template <int FMT, int R, int FUSE>
int launch_fused(const GemvFuse &fz, size_t wgs, int ks, const float *x, int K, int nb, hipStream_t s, bool dry) {
  const int C = (int)gq_chunks(FMT, K);
  if constexpr (R == 1) {  // (one-tile workgroups: a half list still stages whole 512-k slices)
    if ((C + ks - 1) / ks <= Fmt<FMT>::MAXC / 2)
      return launch_fused_h<FMT, 1, FUSE, true>(fz, wgs, ks, x, K, nb, s, dry);
  }
  return launch_fused_h<FMT, R, FUSE, false>(fz, wgs, ks, x, K, nb, s, dry);
}

template <int R, int FUSE>
int launch_fused_fmt(int fmt, const GemvFuse &fz, size_t wgs, int ks, const float *x, int K, int nb,
                     hipStream_t s, bool dry = false) {
  switch (gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt) {
  case GQ_FMT_Q4_0: return launch_fused<GQ_FMT_Q4_0, R, FUSE>(fz, wgs, ks, x, K, nb, s, dry);
  case GQ_FMT_Q8_0: return launch_fused<GQ_FMT_Q8_0, R, FUSE>(fz, wgs, ks, x, K, nb, s, dry);
  default: return launch_fused<GQ_FMT_Q4_K, R, FUSE>(fz, wgs, ks, x, K, nb, s, dry);
  }
}

// ---- the fused forms' fallback ------------------------------------------------
// Batch 3..4 with long K (about 15000 and more for Q4_0 / Q4_K) cannot stage
// the activation limbs of a fused launch in LDS.  Those shapes run as: x
// RMS-normalised into a workspace row (when gamma is given), one gq_gemv per
// matrix (which takes them to the fp16 batch kernel), and for SwiGLU an
// elementwise silu(gate) * up.  Same results within the GEMV's bound; the
// normalisation is applied to x before the products instead of to the dot
// products after them.
__global__ void __launch_bounds__(256) k_rmsnorm_rows(const float *__restrict__ x, const float *__restrict__ gamma,
                                                      float *__restrict__ xn, int K, float eps) {
  const size_t b = blockIdx.x;
  const float *xr = x + b * (size_t)K;
  float *o = xn + b * (size_t)K;
  float ss = 0.f;
  for (int k = (int)threadIdx.x; k < K; k += 256) ss += xr[k] * xr[k];
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)K + eps);
  for (int k = (int)threadIdx.x; k < K; k += 256) o[k] = xr[k] * inv * gamma[k];
}

__global__ void __launch_bounds__(256) k_silu_mul(const float *__restrict__ g, const float *__restrict__ u,
                                                  float *__restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) {
    const float gt = g[i];
    y[i] = gt / (1.0f + expf(-gt)) * u[i];
  }
}

// mats: n_mats matrices (SwiGLU: gate, up; y[0] the output)
int fused_fallback(int fmt, int n_mats, const void *const *packed, const size_t *N, size_t K, const float *x,
                   float *const *y, int batch, const float *gamma, float eps, bool swiglu, hipStream_t s) {
  const size_t xb = gamma ? gq_align256((size_t)batch * K * 4) : 0;
  const size_t tb = swiglu ? gq_align256((size_t)batch * N[0] * 4) : 0;
  void *ws = nullptr;
  if (xb + 2 * tb) GQ_TRY(gq_default_workspace(xb + 2 * tb, &ws));
  const float *xin = x;
  if (gamma) {
    hipLaunchKernelGGL(k_rmsnorm_rows, dim3((unsigned)batch), dim3(256), 0, s, x, gamma, (float *)ws, (int)K, eps);
    GQ_TRY(gq_last_launch());
    xin = (const float *)ws;
  }
  if (!swiglu) {
    for (int i = 0; i < n_mats; ++i) GQ_TRY(gq_gemv(fmt, packed[i], xin, y[i], N[i], K, batch, nullptr, 0, s));
    return GQ_OK;
  }
  float *tg = (float *)((uint8_t *)ws + xb), *tu = (float *)((uint8_t *)ws + xb + tb);
  GQ_TRY(gq_gemv(fmt, packed[0], xin, tg, N[0], K, batch, nullptr, 0, s));
  GQ_TRY(gq_gemv(fmt, packed[1], xin, tu, N[0], K, batch, nullptr, 0, s));
  const size_t n = (size_t)batch * N[0];
  hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, tg, tu, y[0], n);
  return gq_last_launch();
}

}  // namespace

extern "C" int gq_gemv_multi_plan(int fmt, int n_mats, const size_t *N, size_t K, int batch, int *R_out,
                                  int *ksplit_out, int *chunks_per_wave_out) {
  GQ_CHECK(n_mats >= 1 && n_mats <= 4 && N, GQ_ERR_INVALID_ARGS);
  GQ_CHECK(batch >= 1 && batch <= 4, GQ_ERR_UNSUPPORTED);
  size_t tiles = 0;
  for (int i = 0; i < n_mats; ++i) {
    GQ_TRY(gq_check_shape(fmt, N[i], K));
    tiles += gq_tiles(N[i]);
  }
  if (gq_fmt_is_q6k(fmt)) {  // no fused Q6_K kernel: the fallback
    if (R_out) *R_out = 0;
    if (ksplit_out) *ksplit_out = 0;
    if (chunks_per_wave_out) *chunks_per_wave_out = 0;
    return GQ_OK;
  }
  int R = 1, ks = 2, cpw = 0;
  GQ_TRY(q_plan(fmt, tiles * 16, K, batch, &R, &ks, &cpw));
  // (0, 0, 0): the staging does not fit, the call runs the fallback
  const int st = K == 0 ? GQ_OK
                        : R == 2 ? launch_fused_fmt<2, 1>(fmt, GemvFuse{}, 1, ks, nullptr, (int)K, batch, nullptr, true)
                                 : launch_fused_fmt<1, 1>(fmt, GemvFuse{}, 1, ks, nullptr, (int)K, batch, nullptr, true);
  // (the fused kernel's chunk list or its LDS staging does not fit)
  if (st == GQ_ERR_UNSUPPORTED || st == GQ_ERR_INVALID_ARGS) R = ks = cpw = 0;
  if (R_out) *R_out = R;
  if (ksplit_out) *ksplit_out = ks;
  if (chunks_per_wave_out) *chunks_per_wave_out = cpw;
  return GQ_OK;
}

extern "C" int gq_gemv_multi(int fmt, int n_mats, const void *const *packed, const size_t *N, size_t K,
                             const float *x, float *const *y, int batch, const float *gamma, float eps,
                             void *stream) {
  GQ_CHECK(packed && y && x && N, GQ_ERR_INVALID_ARGS);
  int R = 1, ks = 2, cpw = 0;
  GQ_TRY(gq_gemv_multi_plan(fmt, n_mats, N, K, batch, &R, &ks, &cpw));
  if (R == 0) {
    for (int i = 0; i < n_mats; ++i) GQ_CHECK(packed[i] && y[i], GQ_ERR_INVALID_ARGS);
    return fused_fallback(fmt, n_mats, packed, N, K, x, y, batch, gamma, eps, false, (hipStream_t)stream);
  }
  GemvFuse fz{};
  size_t wgs = 0;
  for (int i = 0; i < n_mats; ++i) {
    GQ_CHECK(packed[i] && y[i], GQ_ERR_INVALID_ARGS);
    wgs += (gq_tiles(N[i]) + R - 1) / R;
    fz.seg[i] = GemvSeg{(const uint8_t *)packed[i], gq_sc_plane_offset(fmt, N[i], K), y[i], (int)N[i], (int)wgs};
  }
  for (int i = n_mats; i < 4; ++i) fz.seg[i] = fz.seg[n_mats - 1];
  fz.nseg = n_mats;
  fz.gamma = gamma;
  fz.eps = eps;
  if (K == 0 || wgs == 0) return GQ_ERR_INVALID_ARGS;
  hipStream_t s = (hipStream_t)stream;
  return R == 2 ? launch_fused_fmt<2, 1>(fmt, fz, wgs, ks, x, (int)K, batch, s)
                : launch_fused_fmt<1, 1>(fmt, fz, wgs, ks, x, (int)K, batch, s);
}

extern "C" int gq_gemv_swiglu_plan(int fmt, size_t N, size_t K, int batch, int *ksplit_out,
                                   int *chunks_per_wave_out) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(batch >= 1 && batch <= 4, GQ_ERR_UNSUPPORTED);
  if (gq_fmt_is_q6k(fmt)) {  // no fused Q6_K kernel: the fallback
    if (ksplit_out) *ksplit_out = 0;
    if (chunks_per_wave_out) *chunks_per_wave_out = 0;
    return GQ_OK;
  }
  const int C = (int)gq_chunks(fmt, K);
  int ks = ks_for(fmt, gq_tiles(N), C, 2);
  int cpw = ks > 0 ? (C + ks - 1) / ks : 0;
  // (0, 0): K too long for a wave's chunk list, or the staging does not fit
  // the LDS: the call runs the fallback
  const int st = (K == 0 || ks <= 0) ? GQ_OK
                                      : launch_fused_fmt<2, 2>(fmt, GemvFuse{}, 1, ks, nullptr, (int)K, batch, nullptr,
                                                               true);
  if (ks <= 0 || st == GQ_ERR_UNSUPPORTED || st == GQ_ERR_INVALID_ARGS) ks = cpw = 0;
  if (ksplit_out) *ksplit_out = ks;
  if (chunks_per_wave_out) *chunks_per_wave_out = cpw;
  return GQ_OK;
}

extern "C" int gq_gemv_swiglu(int fmt, const void *gate, const void *up, size_t N, size_t K, const float *x,
                              float *y, int batch, const float *gamma, float eps, void *stream) {
  GQ_CHECK(gate && up && x && y, GQ_ERR_INVALID_ARGS);
  int ks = 2, cpw = 0;
  GQ_TRY(gq_gemv_swiglu_plan(fmt, N, K, batch, &ks, &cpw));
  if (N == 0) return GQ_OK;
  GQ_CHECK(K > 0, GQ_ERR_INVALID_ARGS);
  if (ks == 0) {
    const void *pk[2] = {gate, up};
    const size_t nn[2] = {N, N};
    float *yy[1] = {y};
    return fused_fallback(fmt, 2, pk, nn, K, x, yy, batch, gamma, eps, true, (hipStream_t)stream);
  }
  GemvFuse fz{};
  const size_t sc = gq_sc_plane_offset(fmt, N, K);
  const size_t wgs = gq_tiles(N);
  fz.seg[0] = GemvSeg{(const uint8_t *)gate, sc, y, (int)N, (int)wgs};
  fz.seg[1] = GemvSeg{(const uint8_t *)up, sc, y, (int)N, (int)wgs};
  fz.seg[2] = fz.seg[3] = fz.seg[1];
  fz.nseg = 2;
  fz.gamma = gamma;
  fz.eps = eps;
  return launch_fused_fmt<2, 2>(fmt, fz, wgs, ks, x, (int)K, batch, (hipStream_t)stream);
}
