// gq_gemm.hip -- prefill GEMM over T16-repacked GGUF weights on CDNA4 MFMA.
//
// Replaces gemm_mfma_int8_wt_kernel / gemm_mfma_int4_wt_kernel
// (src/rt/backend/hip/kernels/gemm_kernels.hip:640-740, 820-908) for
// GGUF-native weights.  Computes the mathematical C = A * W^T ("row" layout);
// the reference kernels' transposed 16x16 tile store is a bug, not a contract.
//
// Design:
//  * Workgroup tile BM x BN (256 x 256, 256 x 128 or 128 x 128), K step 64,
//    8 waves (two per SIMD, so one wave's dequantization overlaps the other's
//    MFMAs) in a 2 x 4 arrangement; each wave owns a (BM/2) x (BN/4) block of
//    C as v_mfma_f32_32x32x16_f16 tiles with fp32 accumulators.
//  * Activations are fp16 [M][lda] in HBM (bf16 / fp32 callers get one
//    conversion pass first; bf16 -> fp16 is exact inside fp16's range, and
//    the reference rounds A to fp16 before its MFMAs too).  They go straight
//    from global memory into LDS (global_load_lds_dwordx4, no registers, no
//    VALU) with the 16-byte chunks of each row XOR-swizzled by the row index,
//    so the MFMA fragment reads are free of bank conflicts.
//  * Weights are loaded two K steps ahead into registers (wave-uniform base +
//    32-bit lane offset addressing), dequantized with the per-block scale
//    folded in (one fp16 rounding of the exact product, as the reference's
//    __float2half(w * s) does) and stored to LDS one step ahead.  Both LDS
//    operand tiles are double-buffered: one barrier per K step.
//  * Tiles are assigned so that the 8 XCDs (workgroup id mod 8) each work on a
//    contiguous range of weight column tiles, all M tiles of one column tile
//    in a row: a weight tile is fetched from HBM once per XCD and then served
//    from that XCD's L2.
#include <stdlib.h>

#include <mutex>
#include <type_traits>

#include "gq_internal.h"

namespace {

constexpr int BK = 64;
constexpr int BSTRIDE = BK + 8;  // weight tile row stride (halves): padding keeps ds_read_b128 conflict-free
constexpr int NTHR = 512;

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


// ---- weight records ---------------------------------------------------------
// A record is (row tile tl of the workgroup, lane = 16 g + r): row 16 tl + r
// and, for K step s (64 k), the 16 elements 16 (g & 1) .. + 15 of the step's
// 32-block (g >> 1).
template <int FMT>
struct WRec;
template <>
struct WRec<GQ_FMT_Q4_0> {
  gq_u2 q;     // 16 codes
  uint32_t d;  // d of the record's block for step m = 0 (low half) and m = 1 (high half)
};
template <>
struct WRec<GQ_FMT_Q8_0> {
  gq_u4 q;     // 16 int8
  uint32_t d;
};
template <>
struct WRec<GQ_FMT_Q4_K> {
  gq_u2 q;
  gq_u4 meta;  // d, dmin, W1, W2, W3 of the row's super-block
};

// Per-record byte offsets that do not change with the K step (32-bit: the
// host checks that the packed tensor is smaller than 4 GiB).
struct WOff {
  uint32_t q, s;
};

template <int FMT>
GQ_DEV WOff rec_offsets(int tile, int lane, int C, uint32_t sc_off) {
  const int g = lane >> 4, r = lane & 15;
  const uint32_t tc = (uint32_t)tile * (uint32_t)C;
  WOff o;
  if constexpr (FMT == GQ_FMT_Q4_0) {
    o.q = (tc << 10) + 16u * lane;
    o.s = sc_off + tc * 128u + 8u * r + 4u * (g >> 1);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    o.q = (tc << 11) + 16u * lane;
    o.s = sc_off + tc * 128u + 8u * r + 4u * (g >> 1);
  } else {
    o.q = (tc << 11) + 16u * lane;
    o.s = sc_off + tc * 256u + 16u * r;
  }
  return o;
}

// K step `step` of a record: 16 codes (8 bytes, Q8_0 16 bytes) and the scales.
template <int FMT>
GQ_DEV void load_w(const uint8_t *w, const WOff &o, int step, WRec<FMT> &rec) {
  if constexpr (FMT == GQ_FMT_Q4_0) {
    const uint8_t *wq = w + (((size_t)(step >> 1)) << 10) + 8 * (step & 1);
    const uint8_t *ws = w + ((size_t)(step >> 1)) * 128;
    rec.q = gq_ld8(wq + o.q);
    rec.d = *reinterpret_cast<const uint32_t *>(ws + o.s);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    const uint8_t *wq = w + (((size_t)(step >> 1)) << 11) + ((step & 1) << 10);
    const uint8_t *ws = w + ((size_t)(step >> 1)) * 128;
    rec.q = gq_ld16(wq + o.q);
    rec.d = *reinterpret_cast<const uint32_t *>(ws + o.s);
  } else {
    const int m = step & 3;
    const uint8_t *wq = w + (((size_t)(step >> 2)) << 11) + ((m >> 1) << 10) + 8 * (m & 1);
    const uint8_t *ws = w + ((size_t)(step >> 2)) * 256;
    rec.q = gq_ld8(wq + o.q);
    rec.meta = gq_ld16(ws + o.s);
  }
}

// dequantized fp16 values of a record -> its 16 LDS slots
template <int FMT>
GQ_DEV void store_w(const WRec<FMT> &rec, int tl, int lane, int step, _Float16 *Bs) {
  const int g = lane >> 4, r = lane & 15;
  _Float16 *dst = Bs + (16 * tl + r) * BSTRIDE + 32 * (g >> 1) + 16 * (g & 1);
  gq_half8 o0, o1;
  if constexpr (FMT == GQ_FMT_Q4_0) {
    const gq_half2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const uint32_t dbits = (step & 1) ? (rec.d >> 16) : rec.d;
    group_to_h16(rec.q[0], rec.q[1], off, h2_of_bits16(dbits), o0, o1);
  } else if constexpr (FMT == GQ_FMT_Q8_0) {
    const gq_half2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t dbits = (step & 1) ? (rec.d >> 16) : rec.d;
    const gq_half2 d2 = h2_of_bits16(dbits);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gq_half2 lo, hi;
      bytes_to_magic(rec.q[q] ^ 0x80808080u, lo, hi);
      lo = (lo + off) * d2;
      hi = (hi + off) * d2;
      gq_half8 &o = (q < 2) ? o0 : o1;
      const int b = 4 * (q & 1);
      o[b] = lo[0];
      o[b + 1] = lo[1];
      o[b + 2] = hi[0];
      o[b + 3] = hi[1];
    }
  } else {
    const uint32_t mv[4] = {rec.meta[0], rec.meta[1], rec.meta[2], rec.meta[3]};
    // the fp16 bits as they are (the reference's NaN-to-Inf conversion would
    // compile to branches here)
    const _Float16 hd = __builtin_bit_cast(_Float16, (uint16_t)(mv[0] & 0xFFFFu));
    const float dmin = (float)__builtin_bit_cast(_Float16, (uint16_t)(mv[0] >> 16));
    const int j = 2 * (step & 3) + (g >> 1);
    uint32_t sc, mn;
    gq_q4k_meta_codes(mv, j, &sc, &mn);
    const _Float16 hsc = (_Float16)(float)sc, hnsc = (_Float16)(-1024.0f * (float)sc);
    const _Float16 hmin = (_Float16)(-(dmin * (float)mn));
    const gq_half2 sc2 = {hsc, hsc}, nsc2 = {hnsc, hnsc}, d2 = {hd, hd}, mn2 = {hmin, hmin};
    const uint32_t w0 = rec.q[0], w1 = rec.q[1];
    const uint32_t regs[4] = {w0 & 0x0F0F0F0Fu, (w0 >> 4) & 0x0F0F0F0Fu, w1 & 0x0F0F0F0Fu, (w1 >> 4) & 0x0F0F0F0Fu};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gq_half2 lo, hi;
      bytes_to_magic(regs[q], lo, hi);
      lo = __builtin_elementwise_fma(__builtin_elementwise_fma(lo, sc2, nsc2), d2, mn2);
      hi = __builtin_elementwise_fma(__builtin_elementwise_fma(hi, sc2, nsc2), d2, mn2);
      gq_half8 &o = (q < 2) ? o0 : o1;
      const int b = 4 * (q & 1);
      o[b] = lo[0];
      o[b + 1] = lo[1];
      o[b + 2] = hi[0];
      o[b + 3] = hi[1];
    }
  }
  *reinterpret_cast<gq_half8 *>(dst) = o0;
  *reinterpret_cast<gq_half8 *>(dst + 8) = o1;
}

// ---- activation tile: global fp16 -> LDS directly ----------------------------
// A K step of the tile is BM rows x 8 chunks of 16 B.  One wave instruction
// fills 8 consecutive rows (1 KiB of LDS, lane l at byte 16 l).  Logical chunk
// c of row j sits in physical chunk c ^ swz(j), swz(j) = (j ^ (j >> 3)) & 7 on
// the row index mod 32: any 8 (or 16) consecutive rows then read the same
// logical chunk from 8 (16) different bank groups, for 32 or 64 LDS banks.
GQ_DEV int a_swz(int row) { return (row ^ ((row >> 3) & 3)) & 7; }

template <int BM, int NW = 8>
GQ_DEV void load_a_lds(const _Float16 *a16, int lda, int M, int m0, int step, int wave, int lane, _Float16 *As) {
  constexpr int PER_WAVE = BM / (8 * NW);  // instructions per wave per K step (NW waves)
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int row0 = 8 * (wave * PER_WAVE + i);
    const int c = (lane & 7) ^ a_swz(row0 + (lane >> 3));
    int m = m0 + row0 + (lane >> 3);
    if (m >= M) m = M - 1;  // clamped; rows >= M are never stored
    const _Float16 *src = a16 + (size_t)m * lda + step * BK + 8 * c;
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                     (__attribute__((address_space(3))) void *)(As + row0 * BK), 16, 0, 0);
  }
}

GQ_DEV uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}


// Workgroup tile -> (m tile, n tile): ids are spread over the 8 XCDs
// round-robin, so id -> (id mod 8) * (G / 8) + id / 8 gives each XCD a
// contiguous range of tile indices; consecutive indices walk the M tiles of one
// weight column tile.
GQ_DEV void tile_of(int id, int G, int tiles_m, int &mt, int &nt) {
  const int t = (G % 8 == 0) ? (id % 8) * (G / 8) + id / 8 : id;
  nt = t / tiles_m;
  mt = t % tiles_m;
}
// The same with the tile index walked in groups of gm M tiles: within a group,
// consecutive indices walk its M tiles, then the next weight column tile, so
// the workgroups resident on one XCD at a time share fewer activation rows
// (gm <= 0: tile_of).
GQ_DEV void tile_of_g(int id, int G, int tiles_m, int tiles_n, int gm, int &mt, int &nt) {
  if (gm <= 0 || gm >= tiles_m) {
    tile_of(id, G, tiles_m, mt, nt);
    return;
  }
  const int t = (G % 8 == 0) ? (id % 8) * (G / 8) + id / 8 : id;
  const int per = gm * tiles_n, grp = t / per, first = grp * gm;
  const int rows = tiles_m - first < gm ? tiles_m - first : gm;
  const int u = t - grp * per;
  mt = first + u % rows;
  nt = u / rows;
}

// Row scales rs[m0 .. m0 + BM) of a tile, four per thread for the first BM / 4
// threads (1.0 where rs is NULL).  The load is unconditional, from a valid
// address either way (the scale buffer is padded past M; `any` is any
// readable 16 bytes), so no branch sits around it.
template <int BM>
GQ_DEV gq_f4 ld_row_scales(const float *rs, int m0, int tid, const void *any) {
  const int t = tid % (BM / 4);
  const gq_f4 *p = rs ? reinterpret_cast<const gq_f4 *>(rs + m0 + 4 * t) : reinterpret_cast<const gq_f4 *>(any);
  const gq_f4 v = *p;
  return rs ? v : gq_f4{1.f, 1.f, 1.f, 1.f};
}

template <int FMT, int CBF16, int BM, int BN>
__global__ void __launch_bounds__(NTHR) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_gemm_t16(const uint8_t *__restrict__ w, uint32_t sc_off, const _Float16 *__restrict__ a16, int lda,
           void *__restrict__ c, const float *__restrict__ rs, int M, int N, int C, int nsteps, int tiles_m) {
  constexpr int TM = BM / 64, TN = BN / 128;  // 32 x 32 MFMA tiles per wave along M and N
  static_assert(TN >= 1, "BN >= 128");
  static_assert(2 * (BN * 4 / NTHR) <= 15, "vmcnt immediate");
  constexpr int WR = BN * 4 / NTHR;          // weight records per thread per step
  constexpr int KS = BK / 16;                // MFMA k-steps per K step
  // separate arrays, so the compiler can tell the A tile's LDS DMA from the
  // weight tile's LDS stores
  // (one array per buffer: the buffer index is a compile-time constant
  // everywhere, so no wait for an in-flight DMA into the other buffer is needed)
  __shared__ __attribute__((aligned(16))) _Float16 As_0[BM * BK];  // [BM][BK], swizzled
  __shared__ __attribute__((aligned(16))) _Float16 As_1[BM * BK];
  __shared__ __attribute__((aligned(16))) _Float16 Bs_0[BN * BSTRIDE];  // [BN][BSTRIDE]
  __shared__ __attribute__((aligned(16))) _Float16 Bs_1[BN * BSTRIDE];
  auto As_of = [&](auto b) -> _Float16 * { return decltype(b)::value ? As_1 : As_0; };
  auto Bs_of = [&](auto b) -> _Float16 * { return decltype(b)::value ? Bs_1 : Bs_0; };
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  int mt, nt;
  tile_of(blockIdx.x, gridDim.x, tiles_m, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int ntiles = (int)gq_tiles(N);

  WOff wo[WR];
#pragma unroll
  for (int i = 0; i < WR; ++i) {
    const int rec = tid + NTHR * i;
    int tile = n0 / 16 + (rec >> 6);
    if (tile >= ntiles) tile = ntiles - 1;  // clamped; those columns are never stored
    wo[i] = rec_offsets<FMT>(tile, rec & 63, C, sc_off);
  }

  gq_f16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // two register stages of raw weight records: stage s & 1 holds step s
  WRec<FMT> wr[2][WR];
  auto load_w_step = [&](int step, int st) {
#pragma unroll
    for (int i = 0; i < WR; ++i) load_w<FMT>(w, wo[i], step, wr[st][i]);
  };
  auto store_w_part = [&](int q, int step, int st, auto buf_c) {
    _Float16 *Bs = Bs_of(buf_c);
#pragma unroll
    for (int i = 0; i < WR; ++i)
      if (i % KS == q) {
        const int rec = tid + NTHR * i;
        store_w<FMT>(wr[st][i], rec >> 6, rec & 63, step, Bs);
      }
  };

  // fragment addressing: A rows (BM/2) wm + 32 i + (lane & 31), swizzled chunk;
  // B rows (BN/4) wn + 32 j + (lane & 31), padded rows
  const int arow = (BM / 2) * wm + (lane & 31);
  const int brow = (BN / 4) * wn + (lane & 31);
  const int sw = a_swz(lane & 31);  // == a_swz(arow + 32 i): row bases are multiples of 32

  // One K step on LDS buffer BUF: the A tile of step + 1 is requested (LDS
  // DMA into A buffer BUF ^ 1); then, for each of the KS MFMA k-steps, its
  // MFMAs are issued and a quarter of the weight records of step + 1
  // (register stage BUF ^ 1, loaded a step ago) is dequantized into weight
  // buffer BUF ^ 1 while they run; after the last quarter the records of
  // step + 2 are requested into that register stage.
  auto run_step = [&](int step, auto buf_c) {
    constexpr int BUF = decltype(buf_c)::value;
    using NB = std::integral_constant<int, BUF ^ 1>;
    // the last steps' loads are clamped: loaded, never read
    const int s1 = step + 1 < nsteps ? step + 1 : nsteps - 1;
    const int s2 = step + 2 < nsteps ? step + 2 : nsteps - 1;
    load_a_lds<BM>(a16, lda, M, m0, s1, wave, lane, As_of(NB{}));
    __builtin_amdgcn_sched_barrier(0);
    const _Float16 *As = As_of(buf_c) + arow * BK;
    const _Float16 *Bs = Bs_of(buf_c) + brow * BSTRIDE + 8 * (lane >> 5);
    gq_half8 af[2][TM], bf[2][TN];
    auto read_frags = [&](int ks, int fb) {
      const int ch = (2 * ks + (lane >> 5)) ^ sw;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[fb][i] = *reinterpret_cast<const gq_half8 *>(As + 32 * i * BK + 8 * ch);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[fb][j] = *reinterpret_cast<const gq_half8 *>(Bs + 32 * j * BSTRIDE + 16 * ks);
    };
    read_frags(0, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read_frags(ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = gq_mfma32(af[ks & 1][i], bf[ks & 1][j], acc[i][j]);
      // dequantize a quarter of the next step's weight records (loaded a step
      // ago) into the other weight buffer while these MFMAs run
      store_w_part(ks, s1, BUF ^ 1, NB{});
      // the records of step + 2 reuse that register stage: request them once
      // the last quarter has been read
      if (ks == KS - 1) load_w_step(s2, BUF);
    }
    // the A tile of step + 1 (LDS DMA, issued before the 2 * WR record
    // loads) must land before any wave reads buffer BUF ^ 1
    __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * WR));  // vmcnt(2 * WR)
    __syncthreads();
  };

  // the tile's row scales go to LDS with the prologue (read back by the
  // epilogue, whose global stores would otherwise wait behind their loads)
  __shared__ __attribute__((aligned(16))) float rs_s[BM];
  const gq_f4 rs4 = ld_row_scales<BM>(rs, m0, tid, w);
  // prologue: step 0 in buffer 0, step 1 in register stage 1
  load_a_lds<BM>(a16, lda, M, m0, 0, wave, lane, As_0);
  load_w_step(0, 0);
  load_w_step(nsteps > 1 ? 1 : 0, 1);
#pragma unroll
  for (int q = 0; q < KS; ++q) store_w_part(q, 0, 0, B0{});
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  if (tid < BM / 4) *reinterpret_cast<gq_f4 *>(rs_s + 4 * tid) = rs4;
  __syncthreads();
  // nsteps is even (K is padded to whole 128-k chunks)
  for (int step = 0; step < nsteps; step += 2) {
    run_step(step, B0{});
    run_step(step + 1, B1{});
  }

  // D layout (32x32): lane l holds column l%32, rows 8*(v/4) + 4*(l/32) + v%4.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    // the row scales of this lane's 16 rows of MFMA tile row i (from LDS):
    // four runs of four consecutive rows; exact powers of two
    const int mb = m0 + (BM / 2) * wm + 32 * i + 4 * (lane >> 5);
    float rsv[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const gq_f4 t = *reinterpret_cast<const gq_f4 *>(rs_s + (mb - m0) + 8 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) rsv[4 * q + e] = t[e];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + (BN / 4) * wn + 32 * j + (lane & 31);
      if (n >= N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = mb + 8 * (v >> 2) + (v & 3);
        if (m < M) {
          const float o = acc[i][j][v] * rsv[v];
          if constexpr (CBF16)
            reinterpret_cast<uint16_t *>(c)[(size_t)m * N + n] = f32_to_bf16_rne(o);
          else
            reinterpret_cast<float *>(c)[(size_t)m * N + n] = o;
        }
      }
    }
  }
}

// ---- register-B kernel: 256 x 256 tiles, 4 waves of 128 x 128 ----------------
// The weight operand never goes through LDS: each wave loads, for each of its
// four 32-column blocks, the T16 code groups of its columns and dequantizes
// them straight into v_mfma_f32_32x32x16_f16 B fragments.  Only the
// activation tile is staged in LDS (LDS DMA, double-buffered, swizzled).
//
// k order inside a 64-k step: MFMA k-step ks (16 k) takes, in lane half kh,
// the 8 k at 32 (ks >> 1) + 16 kh + 8 (ks & 1).  For the weights this is T16
// lane slot g = 2 (ks >> 1) + kh, code-group slots 8 (ks & 1) .. + 7 (one
// dword of the group); for the activations it is 16-byte chunk
// 4 (ks >> 1) + 2 kh + (ks & 1) of the row -- the same k on both sides.  All
// eight k of a fragment lie in 32-block (ks >> 1) of the step.
template <int FMT, int NJ>
struct RStep;
template <int NJ>
struct RStep<GQ_FMT_Q4_0, NJ> {
  gq_u2 q[NJ][2];  // [column block][g = kh or 2 + kh]: the step's 8-byte code groups
  gq_u2 d[NJ];     // d0 d2 | d1 d3 of the column's chunk
};
template <int NJ>
struct RStep<GQ_FMT_Q8_0, NJ> {
  gq_u4 q[NJ][2];  // 16 int8 per lane slot
  gq_u2 d[NJ];
};
template <int NJ>
struct RStep<GQ_FMT_Q4_K, NJ> {
  gq_u2 q[NJ][2];
  gq_u4 meta[NJ];  // d, dmin, W1, W2, W3 of the column's super-block
};

// Buffer resource over the 4 GiB from p (raw: stride 0, the offset in
// bytes).  The register-B kernel addresses its operands as a 32-bit per-lane
// offset fixed for the whole K walk plus a uniform scalar offset per step, so
// a load costs no vector address arithmetic (the host checks that both the
// packed weights and the activations lie within 4 GiB).
GQ_DEV __amdgpu_buffer_rsrc_t gq_rsrc(const void *p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, -1, 0x00020000);
}
GQ_DEV gq_u2 ld8_b(const void *base, uint32_t vo, uint32_t so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(gq_rsrc(base), vo, so, 0);
  return gq_u2{v[0], v[1]};
}
GQ_DEV gq_u4 ld16_b(const void *base, uint32_t vo, uint32_t so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(gq_rsrc(base), vo, so, 0);
  return gq_u4{v[0], v[1], v[2], v[3]};
}

template <int FMT, int NJ>
GQ_DEV void load_rstep(const uint8_t *w, const uint32_t (&qo)[NJ], const uint32_t (&so)[NJ], int step,
                       RStep<FMT, NJ> &st) {
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if constexpr (FMT == GQ_FMT_Q4_0) {
      const uint32_t b = ((uint32_t)(step >> 1) << 10) + 8u * (uint32_t)(step & 1);
      st.q[j][0] = ld8_b(w, qo[j], b);
      st.q[j][1] = ld8_b(w, qo[j] + 512u, b);
      st.d[j] = ld8_b(w, so[j], (uint32_t)(step >> 1) * 128u);
    } else if constexpr (FMT == GQ_FMT_Q8_0) {
      const uint32_t b = ((uint32_t)(step >> 1) << 11) + ((uint32_t)(step & 1) << 10);
      st.q[j][0] = ld16_b(w, qo[j], b);
      st.q[j][1] = ld16_b(w, qo[j] + 512u, b);
      st.d[j] = ld8_b(w, so[j], (uint32_t)(step >> 1) * 128u);
    } else {
      const int m = step & 3;
      const uint32_t b = ((uint32_t)(step >> 2) << 11) + ((uint32_t)(m >> 1) << 10) + 8u * (uint32_t)(m & 1);
      st.q[j][0] = ld8_b(w, qo[j], b);
      st.q[j][1] = ld8_b(w, qo[j] + 512u, b);
      st.meta[j] = ld16_b(w, so[j], (uint32_t)(step >> 2) * 256u);
    }
  }
}

// The register-B kernel's activation tile loads (load_a_lds's rows and
// swizzle): per-lane offsets computed once, the step's columns a scalar offset.
template <int BM, int NW>
GQ_DEV void a_offsets(int lda, int M, int m0, int wave, int lane, uint32_t (&ao)[BM / (8 * NW)]) {
  constexpr int PER_WAVE = BM / (8 * NW);
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int row0 = 8 * (wave * PER_WAVE + i);
    const int c = (lane & 7) ^ a_swz(row0 + (lane >> 3));
    int m = m0 + row0 + (lane >> 3);
    if (m >= M) m = M - 1;  // clamped; rows >= M are never stored
    ao[i] = 2u * ((uint32_t)m * (uint32_t)lda + 8u * (uint32_t)c);
  }
}
template <int BM, int NW>
GQ_DEV void load_a_lds_b(const _Float16 *a, const uint32_t *ao, int step, int wave,
                         _Float16 *As) {
  constexpr int PER_WAVE = BM / (8 * NW);
#pragma unroll
  for (int i = 0; i < PER_WAVE; ++i) {
    const int row0 = 8 * (wave * PER_WAVE + i);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(gq_rsrc(a), (__attribute__((address_space(3))) void *)(As + row0 * BK), 16, ao[i],
                                             (uint32_t)step * (2u * BK), 0, 0);
  }
}

// Q4_K: the fp16 factors of the sub-block 2 (step & 3) + h of column block j
// (sc, -1024 sc, d, -dmin m), decoded once per K step.
struct QKf {
  gq_half2 sc2, nsc2, d2, mn2, mn16;  // mn16 = 16 mn2 (exact): for the 16 x elements
};
template <int NJ>
GQ_DEV void q4k_factors(const RStep<GQ_FMT_Q4_K, NJ> &st, int step, QKf (&f)[NJ][2]) {
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const uint32_t mv[4] = {st.meta[j][0], st.meta[j][1], st.meta[j][2], st.meta[j][3]};
    // the fp16 bits as they are (the reference's NaN-to-Inf conversion would
    // compile to branches here)
    const _Float16 hd = __builtin_bit_cast(_Float16, (uint16_t)(mv[0] & 0xFFFFu));
    const _Float16 ndmin = -__builtin_bit_cast(_Float16, (uint16_t)(mv[0] >> 16));
    // the step's two sub-blocks 2 t and 2 t + 1 (t = step & 3): byte t of meta
    // words 1 and 2 (6-bit scale, the min's low 2 bits on top) and of word 3
    // (the mins' high nibbles); both factors of a kind decoded as one fp16
    // pair: 1024 + code from the mantissa bits, minus 1024 (exact)
    const uint32_t sh = 8u * (uint32_t)(step & 3);
    const uint32_t b1 = (mv[1] >> sh) & 0xFFu, b2 = (mv[2] >> sh) & 0xFFu, b3 = (mv[3] >> sh) & 0xFFu;
    const uint32_t scp = (b1 & 63u) | ((b2 & 63u) << 16);
    const uint32_t mnp = ((b1 >> 6) | ((b3 & 15u) << 2)) | (((b2 >> 6) | ((b3 >> 4) << 2)) << 16);
    const gq_half2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
    const gq_half2 sc = gq_bits_h2(scp | 0x64006400u) + k1024;   // sc, exact
    const gq_half2 mn = gq_bits_h2(mnp | 0x64006400u) + k1024;   // m, exact
    const gq_half2 nsc = sc * gq_half2{(_Float16)-1024.0f, (_Float16)-1024.0f};  // exact
    const gq_half2 hm = mn * gq_half2{ndmin, ndmin};  // -(dmin m), the exact product rounded once
    const gq_half2 hm16 = hm * gq_half2{(_Float16)16.0f, (_Float16)16.0f};  // exact
    f[j][0] = QKf{__builtin_shufflevector(sc, sc, 0, 0), __builtin_shufflevector(nsc, nsc, 0, 0), gq_half2{hd, hd},
                  __builtin_shufflevector(hm, hm, 0, 0), __builtin_shufflevector(hm16, hm16, 0, 0)};
    f[j][1] = QKf{__builtin_shufflevector(sc, sc, 1, 1), __builtin_shufflevector(nsc, nsc, 1, 1), gq_half2{hd, hd},
                  __builtin_shufflevector(hm, hm, 1, 1), __builtin_shufflevector(hm16, hm16, 1, 1)};
  }
}

// B fragment of column block j, MFMA k-step ks, K step `step`: 8 fp16 values
// (c - bias) * scale (Q4_K: d sc c - dmin m, factors from q4k_factors), each
// rounded once.
template <int FMT, int NJ>
GQ_DEV gq_half8 rfrag(const RStep<FMT, NJ> &st, int j, int ks, int step, const QKf *qk, uint32_t mg) {
  const int h = ks >> 1;
  gq_half2 p[4];
  if constexpr (FMT == GQ_FMT_Q8_0) {
    const gq_u4 &q = st.q[j][h];
    const uint32_t w0 = q[2 * (ks & 1)] ^ 0x80808080u, w1 = q[2 * (ks & 1) + 1] ^ 0x80808080u;
    const uint32_t db = st.d[j][h];
    const gq_half2 d2 = h2_of_bits16((step & 1) ? (db >> 16) : db);
    const gq_half2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    bytes_to_magic(w0, p[0], p[1]);
    bytes_to_magic(w1, p[2], p[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = (p[i] + off) * d2;
  } else {
    // the 4-bit order (gq_nib_halves): pairs 1 and 3 are 1024 + 16 q, their
    // results 16 x the weight (the activations hold those k divided by 16)
    gq_nib_halves(st.q[j][h][ks & 1], mg, p);
    if constexpr (FMT == GQ_FMT_Q4_0) {
      const uint32_t db = st.d[j][h];
      const gq_half2 d2 = h2_of_bits16((step & 1) ? (db >> 16) : db);
      const gq_half2 off1 = {(_Float16)-1032.0f, (_Float16)-1032.0f};
      const gq_half2 off16 = {(_Float16)-1152.0f, (_Float16)-1152.0f};  // 16 (q - 8), exact
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i] = (p[i] + ((i & 1) ? off16 : off1)) * d2;
    } else {
      // sc q (or 16 sc q) is exact; then one rounding of d sc q - dmin m
      const QKf &f = qk[h];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        p[i] = __builtin_elementwise_fma(__builtin_elementwise_fma(p[i], f.sc2, f.nsc2), f.d2, (i & 1) ? f.mn16 : f.mn2);
    }
  }
  gq_half8 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = p[i][0];
    o[2 * i + 1] = p[i][1];
  }
  return o;
}

// Workgroup tile BM x BN, WM x WN waves; a wave owns (BM / WM) x (BN / WN) of C
// (TM x NJ MFMA tiles of 32 x 32).  256 x 256 with 2 x 4 waves: two waves per SIMD.
// PD: pipeline depth.  The activation tile of step s + PD - 1 is requested
// into one of PD LDS buffers when step s starts, and the weights of step
// s + PD into the register stage step s has just used (PD stages), so a
// step waits on loads issued PD - 1 steps earlier: depth 2 for large tiles,
// 3 or 4 for grids whose short steps would otherwise wait out each load's
// latency.
// KG: K groups.  KG groups of WM x WN waves share the workgroup's tile, group
// g taking the K steps g, g + KG, g + 2 KG, ... with its own activation
// buffers; the groups' accumulators are added through LDS at the end (group
// 0 stores).  Grids with one workgroup per CU (M = 512) otherwise run one
// wave per SIMD, each waiting out its loads' latency; KG groups put KG waves
// on every SIMD with no partial sums leaving the CU.  nsteps % KG == 0.
template <int FMT, int CBF16, int BM, int BN, int WM, int WN, int PD = 2, int KG = 1>
__global__ void __launch_bounds__(64 * WM * WN * KG)
__attribute__((amdgpu_waves_per_eu(WM * WN * KG / 4, WM * WN * KG / 4)))
k_gemm_rb(const uint8_t *__restrict__ w, uint32_t sc_off, const _Float16 *__restrict__ a16, int lda,
          void *__restrict__ c, const float *__restrict__ rs, int M, int N, int C, int nsteps, int tiles_m,
          int gm) {
  constexpr int KS = BK / 16;
  constexpr int NW = WM * WN, TM = BM / WM / 32, NJ = BN / WN / 32;  // waves per group, MFMA tiles per wave
  static_assert(TM >= 1 && NJ >= 1 && BM % (8 * NW) == 0, "tile shape");
  static_assert(PD >= 2 && PD <= 4, "pipeline depth");
  static_assert(KG == 1 || KG == 2 || KG == 4, "K groups");
  // one array per buffer: the buffer index is a compile-time constant
  // everywhere, so no wait for an in-flight DMA into another buffer is needed
  // (each K group uses its own BM x BK part of every buffer)
  __shared__ __attribute__((aligned(16))) _Float16 As_0[KG * BM * BK];
  __shared__ __attribute__((aligned(16))) _Float16 As_1[KG * BM * BK];
  __shared__ __attribute__((aligned(16))) _Float16 As_2[PD >= 3 ? KG * BM * BK : 8];
  __shared__ __attribute__((aligned(16))) _Float16 As_3[PD >= 4 ? KG * BM * BK : 8];
  const int kg = KG == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6) / NW);
  auto As_of = [&](auto b) -> _Float16 * {
    constexpr int v = decltype(b)::value;
    return (v == 0 ? As_0 : v == 1 ? As_1 : v == 2 ? As_2 : As_3) + kg * (BM * BK);
  };
  const int nl = nsteps / KG;  // this group's steps
  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using B2 = std::integral_constant<int, 2>;
  using B3 = std::integral_constant<int, 3>;
  constexpr int NA = BM / (8 * NW);  // activation-tile loads per thread and K step
  // loads a step may leave in flight at its end: the activation tiles of
  // steps s + 2 .. s + PD - 1 and the weights of steps s + 2 .. s + PD
  constexpr int pend = (PD - 2) * NA + (PD - 1) * 3 * NJ;
  static_assert(pend <= 63, "vmcnt immediate");
  constexpr int kWaitPend = 0x0F70 | (pend & 15) | ((pend >> 4) << 14);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) % NW);  // within the K group
  const int wm = wave / WN, wn = wave % WN;
  int mt, nt;
  tile_of_g(blockIdx.x, gridDim.x, tiles_m, (N + BN - 1) / BN, gm, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int ntiles = (int)gq_tiles(N);
  const int kh = lane >> 5, r = lane & 15;

  // per column block: byte offsets of this lane's T16 slot g = kh (the slot
  // 2 + kh is 512 bytes further) and of its row's scales, chunk 0
  uint32_t qo[NJ], so[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    int t = (n0 + (BN / WN) * wn + 32 * j + (lane & 31)) >> 4;
    if (t >= ntiles) t = ntiles - 1;  // clamped; those columns are never stored
    const uint32_t tc = (uint32_t)t * (uint32_t)C;
    const uint32_t slot = 16u * (16u * (uint32_t)kh + (uint32_t)r);
    if constexpr (FMT == GQ_FMT_Q4_0) {
      qo[j] = (tc << 10) + slot;
      so[j] = sc_off + tc * 128u + 8u * r;
    } else if constexpr (FMT == GQ_FMT_Q8_0) {
      qo[j] = (tc << 11) + slot;
      so[j] = sc_off + tc * 128u + 8u * r;
    } else {
      qo[j] = (tc << 11) + slot;
      so[j] = sc_off + tc * 256u + 16u * r;
    }
  }

  gq_f16v acc[TM][NJ];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  RStep<FMT, NJ> wst[PD];
  const uint32_t mg = gq_nib_magic();
  uint32_t ao[BM / (8 * NW)];
  a_offsets<BM, NW>(lda, M, m0, wave, lane, ao);
  const int arow = (BM / WM) * wm + (lane & 31);
  const int sw = a_swz(lane & 31);

  // the group's l-th step of K
  auto gstep = [&](int l) { return l * KG + kg; };
  // the group's step l (buffer and register stage l % PD; `step` the K step);
  // steps past the end are skipped by every wave alike
  auto run_step = [&](int l, auto buf_c) {
    constexpr int BUF = decltype(buf_c)::value;
    using NB = std::integral_constant<int, (BUF + PD - 1) % PD>;  // buffer of l + PD - 1
    const int step = gstep(l);
    const int s1 = gstep(l + PD - 1 < nl ? l + PD - 1 : nl - 1);
    const int s2 = gstep(l + PD < nl ? l + PD : nl - 1);
    load_a_lds_b<BM, NW>(a16, ao, s1, wave, As_of(NB{}));
    __builtin_amdgcn_sched_barrier(0);
    const _Float16 *As = As_of(buf_c) + arow * BK;
    RStep<FMT, NJ> &cur = wst[BUF];
    gq_half8 af[2][TM];
    auto read_a = [&](int ks, int fb) {
      const int ch = (4 * (ks >> 1) + 2 * kh + (ks & 1)) ^ sw;
#pragma unroll
      for (int i = 0; i < TM; ++i) af[fb][i] = *reinterpret_cast<const gq_half8 *>(As + 32 * i * BK + 8 * ch);
    };
    read_a(0, 0);
    QKf qk[NJ][2];
    if constexpr (FMT == GQ_FMT_Q4_K) q4k_factors<NJ>(cur, step, qk);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) read_a(ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const gq_half8 bf = rfrag<FMT, NJ>(cur, j, ks, step, qk[j], mg);
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = gq_mfma32(af[ks & 1][i], bf, acc[i][j]);
      }
    }
    // the register stage of this step is free: request step + PD into it
    load_rstep<FMT, NJ>(w, qo, so, s2, cur);
    // the activation tile and the weights of step + 1 must have landed
    __builtin_amdgcn_s_waitcnt(kWaitPend);
    __syncthreads();
  };

  // prologue: tiles 0 .. PD - 2 and weights 0 .. PD - 1 requested; step 0's
  // must land
  auto prime = [&](auto b) {
    constexpr int i = decltype(b)::value;
    const int st = gstep(i < nl ? i : nl - 1);
    if constexpr (i < PD - 1) load_a_lds_b<BM, NW>(a16, ao, st, wave, As_of(b));
    load_rstep<FMT, NJ>(w, qo, so, st, wst[i]);
  };
  // the tile's row scales, requested before the operands (the oldest load,
  // so the wait below covers it) and kept in LDS for the epilogue, whose
  // global stores would otherwise wait behind their loads
  __shared__ __attribute__((aligned(16))) float rs_s[BM];
  const gq_f4 rs4 = ld_row_scales<BM>(rs, m0, tid, w);
  prime(B0{});
  prime(B1{});
  if constexpr (PD >= 3) prime(B2{});
  if constexpr (PD >= 4) prime(B3{});
  __builtin_amdgcn_s_waitcnt(kWaitPend);
  if (tid < BM / 4) *reinterpret_cast<gq_f4 *>(rs_s + 4 * tid) = rs4;
  __syncthreads();
  for (int l = 0; l < nl; l += PD) {
    run_step(l, B0{});
    if (l + 1 < nl) run_step(l + 1, B1{});
    if constexpr (PD >= 3)
      if (l + 2 < nl) run_step(l + 2, B2{});
    if constexpr (PD >= 4)
      if (l + 3 < nl) run_step(l + 3, B3{});
  }
  if constexpr (KG > 1) {
    // the groups' sums, one MFMA tile at a time: groups 1 .. KG - 1 write
    // theirs (lane-contiguous float4s), group 0 adds them in group order
    __shared__ __attribute__((aligned(16))) gq_f4 xs[(KG - 1) * NW * 4 * 64];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if (kg > 0) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            xs[(((kg - 1) * NW + wave) * 4 + q) * 64 + lane] =
                gq_f4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
          for (int g = 0; g < KG - 1; ++g)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const gq_f4 t = xs[((g * NW + wave) * 4 + q) * 64 + lane];
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[i][j][4 * q + e] += t[e];
            }
        }
        __syncthreads();
      }
    if (kg > 0) return;
  }

  // C of this workgroup's rows through a buffer resource starting at row m0
  // (its range ends at row M) when a tile's offsets fit in 32 bits
  constexpr uint32_t ES = CBF16 ? 2u : 4u;
  const bool cfits = (size_t)N * BM * ES < ((size_t)1 << 31);
  const size_t crange = (size_t)(M - m0) * (size_t)N * ES;
  const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<uint8_t *>(c) + (size_t)m0 * N * ES, (short)0,
      (int)(crange < 0xFFFFFFFFu ? crange : 0xFFFFFFFFu), 0x00020000);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    // the row scales of this lane's 16 rows of MFMA tile row i (from LDS):
    // four runs of four consecutive rows; exact powers of two
    const int mb = m0 + (BM / WM) * wm + 32 * i + 4 * (lane >> 5);
    float rsv[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const gq_f4 t = *reinterpret_cast<const gq_f4 *>(rs_s + (mb - m0) + 8 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) rsv[4 * q + e] = t[e];
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int n = n0 + (BN / WN) * wn + 32 * j + (lane & 31);
      if (n >= N) continue;
      if (cfits) {
        // one per-lane offset per MFMA tile, the row of each value a scalar
        // offset; rows >= M lie beyond the resource's range, so the hardware
        // drops their stores
        const uint32_t vo = ((uint32_t)(mb - m0) * (uint32_t)N + (uint32_t)n) * ES;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const uint32_t so = (uint32_t)(8 * (v >> 2) + (v & 3)) * (uint32_t)N * ES;
          const float o = acc[i][j][v] * rsv[v];
          if constexpr (CBF16)
            __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_rne(o), cr, vo, so, 0);
          else
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), cr, vo, so, 0);
        }
        continue;
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = mb + 8 * (v >> 2) + (v & 3);
        if (m < M) {
          const float o = acc[i][j][v] * rsv[v];
          if constexpr (CBF16)
            reinterpret_cast<uint16_t *>(c)[(size_t)m * N + n] = f32_to_bf16_rne(o);
          else
            reinterpret_cast<float *>(c)[(size_t)m * N + n] = o;
        }
      }
    }
  }
}

// Activations -> fp16 [M][ldo] (ldo >= K, columns K..ldo-1 zero), one
// workgroup per row, with a per-row power-of-two scale: the row's largest
// magnitude is brought into [2^14, 2^15) before the one rounding to fp16, and
// rs[m] = 2^-s undoes it on the finished dot products (the GEMM epilogues).
// Multiplying by a power of two is exact, so rows inside fp16's range round
// as before, while rows with values beyond 65504 (outliers of the
// down-projection input, bf16 spikes) or far below 1 keep fp16's full
// relative precision instead of overflowing to Inf or going subnormal.
// q4perm: each run of 8 in the order of the 4-bit B fragments (gq_nib_halves) of the
// skinny and register-B GEMMs (element e holds k slot {0,2,4,6,1,3,5,7}[e], elements 2, 3, 6, 7
// divided by 16 -- exact, before the one rounding to fp16).
// 8 activations from offset off of a (bf16, fp16 or fp32: DT) as floats.  The
// conversion kernels issue all their loads unconditionally (addresses clamped into the row), so
// no load sits under a branch -- a branch around a load makes the compiler
// wait for every load issued before it, one round trip per load
template <int DT>
GQ_DEV void load8_t(const void *a, size_t off, float (&v)[8]) {
  if constexpr (DT == GQ_DT_BF16) {
    const gq_u4 u = gq_ld16(reinterpret_cast<const uint16_t *>(a) + off);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __uint_as_float(u[q] << 16);
      v[2 * q + 1] = __uint_as_float(u[q] & 0xFFFF0000u);
    }
  } else if constexpr (DT == GQ_DT_F16) {
    const gq_half8 h = *reinterpret_cast<const gq_half8 *>(reinterpret_cast<const _Float16 *>(a) + off);
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = (float)h[q];
  } else {
    const float *f = reinterpret_cast<const float *>(a) + off;
    const gq_f4 v0 = *reinterpret_cast<const gq_f4 *>(f), v1 = *reinterpret_cast<const gq_f4 *>(f + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = v0[q];
      v[4 + q] = v1[q];
    }
  }
}

constexpr int kConvThreads = 512, kConvRuns = 8;  // a row of up to 32768 elements stays in registers

GQ_DEV gq_half8 conv8(const float (&v)[8], float f, int q4perm) {
  constexpr int perm[8] = {0, 2, 4, 6, 1, 3, 5, 7};
  gq_half8 h;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = q4perm ? ((e & 2) ? v[perm[e]] * 0.0625f : v[perm[e]]) : v[e];
    h[e] = (_Float16)(x * f);
  }
  return h;
}

template <int DT, int RUNS>
__global__ void __launch_bounds__(kConvThreads) k_a_to_f16(const void *__restrict__ a, _Float16 *__restrict__ o,
                                                           float *__restrict__ rs, int K, int ldo, int q4perm) {
  __shared__ float wmax[kConvThreads / 64];
  const size_t m = blockIdx.x;
  const int tid = threadIdx.x;
  constexpr int SPAN = 8 * kConvThreads * kConvRuns;  // elements held in registers
  // K % 8 == 0 (host-checked), so a run of 8 is all inside or all past K
  float v[kConvRuns][8];
  float amax = 0.f;
#pragma unroll
  for (int r = 0; r < kConvRuns; ++r) {
    const int k0 = 8 * (tid + kConvThreads * r);
    if (r < RUNS) load8_t<DT>(a, m * K + (k0 < K ? k0 : 0), v[r]);  // (RUNS covers the row up to SPAN)
  }
#pragma unroll
  for (int r = 0; r < kConvRuns; ++r) {
    const int k0 = 8 * (tid + kConvThreads * r);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[r][e] = (r < RUNS && k0 < K) ? v[r][e] : 0.f;
      amax = fmaxf(amax, fabsf(v[r][e]));
    }
  }
  for (int k0 = SPAN + 8 * tid; k0 < K; k0 += 8 * kConvThreads) {  // (rows longer than SPAN)
    float u[8];
    load8_t<DT>(a, m * K + k0, u);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(u[e]));
  }
#pragma unroll
  for (int o2 = 32; o2 > 0; o2 >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o2, 64));
  if ((tid & 63) == 0) wmax[tid >> 6] = amax;
  __syncthreads();
  amax = wmax[0];
#pragma unroll
  for (int w = 1; w < kConvThreads / 64; ++w) amax = fmaxf(amax, wmax[w]);
  // s = 14 - floor(log2(amax)) from the exponent field (0 for a zero row,
  // Inf / NaN; clamped so 2^s and 2^-s stay normal floats)
  const uint32_t eb = (__float_as_uint(amax) >> 23) & 0xFFu;
  int sh = (eb == 0u || eb == 0xFFu) ? 0 : 14 - ((int)eb - 127);
  sh = sh < -100 ? -100 : sh > 100 ? 100 : sh;
  const float f = __uint_as_float((uint32_t)(127 + sh) << 23);
  if (tid == 0) rs[m] = __uint_as_float((uint32_t)(127 - sh) << 23);
#pragma unroll
  for (int r = 0; r < kConvRuns; ++r) {
    const int k0 = 8 * (tid + kConvThreads * r);
    if (k0 < ldo) *reinterpret_cast<gq_half8 *>(o + m * ldo + k0) = conv8(v[r], f, q4perm);
  }
  for (int k0 = SPAN + 8 * tid; k0 < ldo; k0 += 8 * kConvThreads) {
    float u[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (k0 < K) load8_t<DT>(a, m * K + k0, u);
    *reinterpret_cast<gq_half8 *>(o + m * ldo + k0) = conv8(u, f, q4perm);
  }
}

// Rows of up to 8192 padded elements: one wave per row (four rows per
// workgroup), the row held in registers (R runs of 8 per lane) and its
// largest magnitude reduced within the wave -- no LDS, no barrier.  The same
// scaling and rounding as k_a_to_f16.
template <int R, int DT>
__global__ void __launch_bounds__(256) k_a_to_f16_w(const void *__restrict__ a, _Float16 *__restrict__ o,
                                                    float *__restrict__ rs, int M, int K, int ldo, int q4perm) {
  const int lane = threadIdx.x & 63;
  const size_t m = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= (size_t)M) return;
  float v[R][8];
  float amax = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k0 = 8 * (lane + 64 * r);
    load8_t<DT>(a, m * K + (k0 < K ? k0 : 0), v[r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k0 = 8 * (lane + 64 * r);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[r][e] = k0 < K ? v[r][e] : 0.f;
      amax = fmaxf(amax, fabsf(v[r][e]));
    }
  }
#pragma unroll
  for (int o2 = 32; o2 > 0; o2 >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o2, 64));
  const uint32_t eb = (__float_as_uint(amax) >> 23) & 0xFFu;
  int sh = (eb == 0u || eb == 0xFFu) ? 0 : 14 - ((int)eb - 127);
  sh = sh < -100 ? -100 : sh > 100 ? 100 : sh;
  const float f = __uint_as_float((uint32_t)(127 + sh) << 23);
  if (lane == 0) rs[m] = __uint_as_float((uint32_t)(127 - sh) << 23);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k0 = 8 * (lane + 64 * r);
    if (k0 < ldo) *reinterpret_cast<gq_half8 *>(o + m * ldo + k0) = conv8(v[r], f, q4perm);
  }
}

// A -> fp16 [M][ldo] with per-row scales: k_a_to_f16_w for at least 1024 rows
// of up to 8192 padded columns (2048 x 4096 bf16: 13.5 -> 11.1 us with loads
// under branches), else k_a_to_f16 (one workgroup of 8 waves per row: fewer
// rows keep more waves busy) with the runs per thread the row needs
template <int DT>
int launch_a_to_f16_t(const void *a, _Float16 *o, float *rs, int M, int K, int ldo, int q4perm, hipStream_t s) {
  const unsigned g4 = (unsigned)((M + 3) / 4);
  if (M >= 1024 && ldo <= 2048)
    hipLaunchKernelGGL((k_a_to_f16_w<4, DT>), dim3(g4), dim3(256), 0, s, a, o, rs, M, K, ldo, q4perm);
  else if (M >= 1024 && ldo <= 4096)
    hipLaunchKernelGGL((k_a_to_f16_w<8, DT>), dim3(g4), dim3(256), 0, s, a, o, rs, M, K, ldo, q4perm);
  else if (M >= 1024 && ldo <= 8192)
    hipLaunchKernelGGL((k_a_to_f16_w<16, DT>), dim3(g4), dim3(256), 0, s, a, o, rs, M, K, ldo, q4perm);
  else if (K <= 8 * kConvThreads)
    hipLaunchKernelGGL((k_a_to_f16<DT, 1>), dim3((unsigned)M), dim3(kConvThreads), 0, s, a, o, rs, K, ldo, q4perm);
  else if (K <= 2 * 8 * kConvThreads)
    hipLaunchKernelGGL((k_a_to_f16<DT, 2>), dim3((unsigned)M), dim3(kConvThreads), 0, s, a, o, rs, K, ldo, q4perm);
  else if (K <= 4 * 8 * kConvThreads)
    hipLaunchKernelGGL((k_a_to_f16<DT, 4>), dim3((unsigned)M), dim3(kConvThreads), 0, s, a, o, rs, K, ldo, q4perm);
  else
    hipLaunchKernelGGL((k_a_to_f16<DT, kConvRuns>), dim3((unsigned)M), dim3(kConvThreads), 0, s, a, o, rs, K, ldo,
                       q4perm);
  return gq_last_launch();
}

int launch_a_to_f16(const void *a, int a_dtype, _Float16 *o, float *rs, int M, int K, int ldo, int q4perm,
                    hipStream_t s) {
  if (a_dtype == GQ_DT_BF16) return launch_a_to_f16_t<GQ_DT_BF16>(a, o, rs, M, K, ldo, q4perm, s);
  if (a_dtype == GQ_DT_F16) return launch_a_to_f16_t<GQ_DT_F16>(a, o, rs, M, K, ldo, q4perm, s);
  return launch_a_to_f16_t<GQ_DT_F32>(a, o, rs, M, K, ldo, q4perm, s);
}

template <int FMT, int CBF16, int BM, int BN>
int launch_cfg(const void *packed, const _Float16 *a16, int lda, void *c, const float *rs, int M, int N, int K,
               hipStream_t s) {
  auto kern = k_gemm_t16<FMT, CBF16, BM, BN>;
  const int C = (int)gq_chunks(FMT, K);
  const int nsteps = (int)(gq_kpad(FMT, K) / BK);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  if ((size_t)tiles_m * (size_t)tiles_n > 0x7FFFFFFFu) return GQ_ERR_INVALID_ARGS;  // (one grid dimension)
  hipLaunchKernelGGL(kern, dim3((unsigned)(tiles_m * tiles_n)), dim3(NTHR), 0, s, (const uint8_t *)packed,
                     (uint32_t)gq_sc_plane_offset(FMT, N, K), a16, lda, c, rs, M, N, C, nsteps, tiles_m);
  return gq_last_launch();
}

// pd_default: the pipeline depth of the shape (GQ_GEMM_PD=2|3|4 overrides it,
// for tuning)
template <int FMT, int CBF16, int BM, int BN, int WM, int WN, int KG = 1>
int launch_rb(const void *packed, const _Float16 *a16, int lda, void *c, const float *rs, int M, int N, int K,
              hipStream_t s, int pd_default = 4) {
  const int C = (int)gq_chunks(FMT, K);
  const int nsteps = (int)(gq_kpad(FMT, K) / BK);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  if ((size_t)tiles_m * (size_t)tiles_n > 0x7FFFFFFFu) return GQ_ERR_INVALID_ARGS;  // (one grid dimension)
  const char *e = getenv("GQ_GEMM_PD");
  const int pd = e ? atoi(e) : pd_default;
  // tile order in groups of 4 M tiles (GQ_GEMM_GM=n overrides, 0: plain
  // column-major order): 4096 x 14336 x 4096 442 vs 453 us in an alternating
  // A/B on one box; no change at 2048 rows (8 M tiles)
  const char *eg = getenv("GQ_GEMM_GM");
  const int gm = eg ? atoi(eg) : 4;
#define GQ_LAUNCH_RB(PD)                                                                                        \
  hipLaunchKernelGGL((k_gemm_rb<FMT, CBF16, BM, BN, WM, WN, PD, KG>), dim3((unsigned)(tiles_m * tiles_n)),      \
                     dim3(64 * WM * WN * KG), 0, s, (const uint8_t *)packed, (uint32_t)gq_sc_plane_offset(FMT, N, K), \
                     a16, lda, c, rs, M, N, C, nsteps, tiles_m, gm)
  // the depths whose LDS fits (activation buffers, the K groups' exchange,
  // the row scales); a deeper request falls back to the deepest that fits
  constexpr auto lds = [](int d) { return d * KG * BM * BK * 2 + (KG - 1) * WM * WN * 4096 + BM * 4; };
  constexpr int kLds = 160 * 1024;
  if (KG > 1 && nsteps % KG) return GQ_ERR_INVALID_ARGS;
  if constexpr (lds(4) <= kLds) {
    if (pd == 4) {
      GQ_LAUNCH_RB(4);
      return gq_last_launch();
    }
  }
  if constexpr (lds(3) <= kLds) {
    if (pd >= 3) {
      GQ_LAUNCH_RB(3);
      return gq_last_launch();
    }
  }
  GQ_LAUNCH_RB(2);
#undef GQ_LAUNCH_RB
  return gq_last_launch();
}

// Kernel and tile shape (measured on MI355X, M = 64 .. 2048 x N = 4096 / 14336):
//  13: register-B kernel, 128 x 256 on 8 waves of 128 x 32 (the 1 x 8 grid on
//      half the rows: each weight dequantized once), depth 4, for >= 192
//      workgroups: 4-7 % faster than 4 in an interleaved A/B (512 x 14336 x
//      4096 Q4_0 / Q4_K / Q8_0 66.4 / 73.7 / 69.9 vs 71.3 / 76.7 / 73.5 us,
//      2048 x 4096 x 4096 Q4_0 76.2 vs 81.8, 1024 x 14336 124.6 vs 133.8)
//  12: register-B kernel, 256 x 256 on 8 waves of 256 x 32 (448 workgroups at
//      2048 x 14336): each wave dequantizes its B fragments for all 256 rows,
//      so no two waves convert the same weights (twice the activation-fragment
//      LDS reads of the 2 x 4 wave grid, half its dequantization VALU);
//      2-8 % faster than 0 (2 x 4 waves) and 3 (LDS-B) for every format
//   0: register-B kernel, 256 x 256, 2 x 4 waves of 128 x 64
//   3: LDS-B kernel, 256 x 256
//  14: register-B, 64 x 128 on 4 waves of 64 x 32 (1 x 4), depth 4, for >= 192
//      workgroups where 128 x 128 gives fewer: 512 x 4096 x 4096 Q4_0 / Q4_K
//      37.0 / 38.3 us vs 40.9 / 41.9 for 9, 2048 x 1024 x 4096 40.5 vs 44.9
//   4: register-B, 256 x 128 (2 x 4 waves), the former choice of 13's grids
//   6: register-B, 128 x 128, for >= 192 workgroups (1024 x 4096, 256 x 14336)
//   9: register-B, 128 x 64 (4 waves), the former choice of 14's grids (512 x
//      4096: 50 vs 56 us with 128 x 128; 128 x 14336: 48 vs 54 us)
//  11: register-B, 64 x 64 (4 waves), smaller problems (M <= 256 at N = 4096:
//      40-43 us vs 49-53)
//  17: 128 x 128 on 1 x 4 waves in 2 K groups (8 waves), depth 4, where 6
//      was chosen: 1024 x 4096 x 4096 Q4_0 / Q4_K / Q8_0 49 / 53-56 / 53 us
//      against 57 / 64-65 / 57-58 for 6; 768 x 4096 42-45 vs 48; 256 x
//      14336 44-45 vs 47-50 (conversion included, graph replays)
//  15: 64 x 128 on 1 x 4 waves in 4 K groups (16 waves), depth 3, for every
//      smaller grid: 512 x 4096 x 4096 30-34 us against 36-39 (14); 256 x
//      4096 24-26 vs 32-36 (11 / skinny); 64 x 14336 22-24 vs 30-34
//      (skinny).  2 K groups (18) ran the same at 512 rows and 1-5 % slower
//      below; 2 K groups on 128 x 256 (16) no faster than 13.
// The register-B kernel runs with pipeline depth 4 (1-3 % faster than 2 on
// the shapes measured), except 256 x 256: depth 3 on the 1 x 8 grid, 2 on the
// 2 x 4 grid (at 4 its Q8_0 and Q4_K instances spill registers).  1, 2 (LDS-B
// 256 x 128, 128 x 128) and 5, 7, 8, 10 (other register-B shapes) are kept for
// tuning through GQ_GEMM_TILE.
int pick_tile(int fmt, int M, int N, int K) {
  auto wgs = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  const int nsteps = (int)(gq_kpad(fmt, K) / BK);
  if (const char *e = getenv("GQ_GEMM_TILE")) {
    const int t = atoi(e);
    // K-group shapes need the K steps to divide among the groups
    if (t == 15 && nsteps % 4) return 14;
    if ((t == 16 || t == 17 || t == 18) && nsteps % 2) return t == 16 ? 13 : t == 17 ? 6 : 14;
    return t;
  }
  if (wgs(256, 256) >= 384) return 12;
  if (wgs(128, 256) >= 192) return 13;
  if (wgs(128, 128) >= 192) return nsteps % 2 ? 6 : 17;
  if (nsteps % 4 == 0) return 15;
  if (wgs(64, 128) >= 192) return 14;
  return 11;
}

template <int FMT, int CBF16>
int launch_fmt(const void *packed, const _Float16 *a16, int lda, void *c, const float *rs, int M, int N, int K,
               hipStream_t s) {
  switch (pick_tile(FMT, M, N, K)) {
  case 0: return launch_rb<FMT, CBF16, 256, 256, 2, 4>(packed, a16, lda, c, rs, M, N, K, s, 2);
  case 4: return launch_rb<FMT, CBF16, 256, 128, 2, 4>(packed, a16, lda, c, rs, M, N, K, s);
  case 5: return launch_rb<FMT, CBF16, 128, 256, 2, 4>(packed, a16, lda, c, rs, M, N, K, s);
  case 6: return launch_rb<FMT, CBF16, 128, 128, 2, 4>(packed, a16, lda, c, rs, M, N, K, s);
  case 7: return launch_rb<FMT, CBF16, 128, 128, 2, 2>(packed, a16, lda, c, rs, M, N, K, s);
  case 8: return launch_rb<FMT, CBF16, 256, 128, 4, 2>(packed, a16, lda, c, rs, M, N, K, s);
  case 9: return launch_rb<FMT, CBF16, 128, 64, 2, 2>(packed, a16, lda, c, rs, M, N, K, s);
  case 10: return launch_rb<FMT, CBF16, 64, 128, 2, 4>(packed, a16, lda, c, rs, M, N, K, s);
  case 11: return launch_rb<FMT, CBF16, 64, 64, 2, 2>(packed, a16, lda, c, rs, M, N, K, s);
  case 12: return launch_rb<FMT, CBF16, 256, 256, 1, 8>(packed, a16, lda, c, rs, M, N, K, s, 3);
  case 13: return launch_rb<FMT, CBF16, 128, 256, 1, 8>(packed, a16, lda, c, rs, M, N, K, s);
  case 14: return launch_rb<FMT, CBF16, 64, 128, 1, 4>(packed, a16, lda, c, rs, M, N, K, s);
  case 15: return launch_rb<FMT, CBF16, 64, 128, 1, 4, 4>(packed, a16, lda, c, rs, M, N, K, s);
  case 16: return launch_rb<FMT, CBF16, 128, 256, 1, 8, 2>(packed, a16, lda, c, rs, M, N, K, s, 3);
  case 17: return launch_rb<FMT, CBF16, 128, 128, 1, 4, 2>(packed, a16, lda, c, rs, M, N, K, s);
  case 18: return launch_rb<FMT, CBF16, 64, 128, 1, 4, 2>(packed, a16, lda, c, rs, M, N, K, s);
  default: return launch_rb<FMT, CBF16, 128, 128, 2, 4>(packed, a16, lda, c, rs, M, N, K, s);
  case 3: return launch_cfg<FMT, CBF16, 256, 256>(packed, a16, lda, c, rs, M, N, K, s);
  case 1: return launch_cfg<FMT, CBF16, 256, 128>(packed, a16, lda, c, rs, M, N, K, s);
  case 2: return launch_cfg<FMT, CBF16, 128, 128>(packed, a16, lda, c, rs, M, N, K, s);
  }
}

template <int FMT>
int launch_gemm(const void *packed, const _Float16 *a16, int lda, void *c, const float *rs, int c_dtype, int M, int N,
                int K, hipStream_t s) {
  return c_dtype == GQ_DT_BF16 ? launch_fmt<FMT, 1>(packed, a16, lda, c, rs, M, N, K, s)
                               : launch_fmt<FMT, 0>(packed, a16, lda, c, rs, M, N, K, s);
}

}  // namespace

extern "C" size_t gq_gemm_workspace_bytes(int fmt, size_t M, size_t K) {
  // activations are first written as fp16 [M][padded K (+ 8 for the skinny
  // kernel)] unless they are fp16 of the padded width already and in k order
  // fp16 A, then the M row scales (padded by one tile: the GEMM epilogues read
  // them four rows at a time)
  if (!gq_fmt_valid(fmt) || M > GQ_MAX_DIM || K > GQ_MAX_DIM) return 0;
  return gq_align256(M * (gq_kpad(fmt, K) + 8) * 2) + gq_align256((M + 256) * 4);
}

// Whether gq_gemm converts A (into the workspace) for this call: always on
// the skinny route; on the tiled route unless A is fp16 of the padded width
// and the kernel takes it in k order (not the 4-bit register-B kernels).
static bool gemm_converts_a(int fmt, size_t M, size_t N, size_t K, int a_dtype) {
  int ct = 0, nck = 0;
  if (gq_gemm_skinny_plan(fmt, M, N, K, &ct, &nck) == GQ_OK) return true;
  const int tile = pick_tile(fmt, (int)M, (int)N, (int)K);
  const bool q4 = (fmt == GQ_FMT_Q4_0 || gq_fmt_is_q4k(fmt)) && tile != 1 && tile != 2 && tile != 3;
  return a_dtype != GQ_DT_F16 || gq_kpad(fmt, K) != K || q4;
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
  // the kernel addresses the packed tensor with 32-bit offsets
  GQ_CHECK(gq_packed_bytes(fmt, N, K) < ((size_t)1 << 32), GQ_ERR_INVALID_ARGS);
  hipStream_t s = (hipStream_t)stream;
  // Few rows: the tiled GEMM gives N / 64 .. N / 128 workgroups, each walking
  // all of K (37-55 us at 4096 x 4096 or 14336 x 4096 for any M <= 256); the
  // skinny kernel takes the shapes gq_gemm_skinny_plan accepts (4096 x 4096:
  // 10 / 14 / 16 us at M = 17 / 64 / 128; 14336 x 4096: 19 / 27 us at
  // M = 17 / 64).
  const size_t Kp = gq_kpad(fmt, K);
  int sk_ct = 0, sk_nck = 0;
  if (gq_gemm_skinny_plan(fmt, M, N, K, &sk_ct, &sk_nck) == GQ_OK) {
    // A in the skinny kernel's order, always through the workspace, rows 16
    // bytes longer than a multiple of 4 KiB: each A load reads 16 rows, and at
    // a 4 KiB-multiple stride they collide in the memory hierarchy (64 x 4096:
    // 19.9 -> 14.9 us; pads of 128 or 256 bytes measured no faster than none,
    // so the collision is not one of whole cache lines; the tiled GEMM gains
    // from no pad and keeps the plain stride)
    const size_t ldo = Kp + 8;
    const size_t need = gq_gemm_workspace_bytes(fmt, M, K);
    if (!ws) {
      GQ_TRY(gq_default_workspace(need, &ws));
      ws_bytes = need;
    }
    GQ_CHECK(ws_bytes >= need, GQ_ERR_WORKSPACE);
    const int q4 = fmt == GQ_FMT_Q4_0 || gq_fmt_is_q4k(fmt);
    float *rs = (float *)((uint8_t *)ws + gq_align256(M * ldo * 2));
    GQ_TRY(launch_a_to_f16(a, a_dtype, (_Float16 *)ws, rs, (int)M, (int)K, (int)ldo, q4, s));
    return gq_launch_gemm_skinny(fmt, packed, (const _Float16 *)ws, (int)ldo, c, rs, c_dtype == GQ_DT_BF16, (int)M, (int)N,
                                 (int)K, s);
  }
  // Q6_K has no tiled kernel (gq_matmul runs the batch GEMV per 16 rows)
  GQ_CHECK(!gq_fmt_is_q6k(fmt), GQ_ERR_UNSUPPORTED);
  const _Float16 *a16 = (const _Float16 *)a;
  const float *rs = nullptr;
  // the register-B kernel takes the 4-bit formats' B fragments in the
  // gq_nib_halves order, so their activations are staged in that order; fp16
  // activations of the padded width are used as they are otherwise
  const int tile = pick_tile(fmt, (int)M, (int)N, (int)K);
  const int q4 = (fmt == GQ_FMT_Q4_0 || gq_fmt_is_q4k(fmt)) && tile != 1 && tile != 2 && tile != 3;
  // (the register-B kernel addresses the activations with 32-bit offsets)
  GQ_CHECK(tile == 1 || tile == 2 || tile == 3 || M * Kp * 2 < ((size_t)1 << 32), GQ_ERR_INVALID_ARGS);
  if (gemm_converts_a(fmt, M, N, K, a_dtype)) {
    const size_t need = gq_gemm_workspace_bytes(fmt, M, K);
    if (!ws) {
      GQ_TRY(gq_default_workspace(need, &ws));
      ws_bytes = need;
    }
    GQ_CHECK(ws_bytes >= need, GQ_ERR_WORKSPACE);
    float *rsw = (float *)((uint8_t *)ws + gq_align256(M * Kp * 2));
    GQ_TRY(launch_a_to_f16(a, a_dtype, (_Float16 *)ws, rsw, (int)M, (int)K, (int)Kp, q4, s));
    a16 = (const _Float16 *)ws;
    rs = rsw;
  }
  const int lda = (int)Kp;
  switch (fmt) {
  case GQ_FMT_Q4_0: return launch_gemm<GQ_FMT_Q4_0>(packed, a16, lda, c, rs, c_dtype, (int)M, (int)N, (int)K, s);
  case GQ_FMT_Q8_0: return launch_gemm<GQ_FMT_Q8_0>(packed, a16, lda, c, rs, c_dtype, (int)M, (int)N, (int)K, s);
  default: return launch_gemm<GQ_FMT_Q4_K>(packed, a16, lda, c, rs, c_dtype, (int)M, (int)N, (int)K, s);
  }
}

// ---- allocation-free form of gq_gemm ------------------------------------------
// The activation conversion (fp16 A and its row scales) lives in a file-scope
// device array instead of a workspace: one copy per GPU, held until the process
// ends.  Host code never passes the array's name to a kernel (on the host it is
// only a stand-in for the symbol): its device address is looked up once per
// device with hipGetSymbolAddress, with that device current, and kept.
namespace {
constexpr size_t kGemmScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kGemmScratchBytes];
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices];
}  // namespace

extern "C" size_t gq_gemm_static_max_bytes(void) { return kGemmScratchBytes; }

extern "C" int gq_gemm_static(int fmt, const void *packed, const void *a, int a_dtype, void *c, int c_dtype, size_t M,
                              size_t N, size_t K, void *stream) {
  GQ_TRY(gq_check_shape(fmt, N, K));
  GQ_CHECK(M <= GQ_MAX_DIM, GQ_ERR_INVALID_ARGS);
  // the scratch holds the A conversion, when the call makes one:
  // gq_gemm_workspace_bytes = M * (padded K + 8) * 2 + (M + 256) * 4 bytes,
  // each term rounded up to 256
  if (gq_fmt_valid(fmt) && K > 0 && gemm_converts_a(fmt, M, N, K, a_dtype))
    GQ_CHECK(gq_gemm_workspace_bytes(fmt, M, K) <= kGemmScratchBytes, GQ_ERR_WORKSPACE);
  int dev = 0;
  GQ_TRY(gq_hip_status(hipGetDevice(&dev)));
  GQ_CHECK(dev >= 0 && dev < kMaxDevices, GQ_ERR_NO_DEVICE);
  void *ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
      void *p = nullptr;
      GQ_TRY(gq_hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))));
      g_scratch_ptr[dev] = p;
    }
    ptr = g_scratch_ptr[dev];
  }
  return gq_gemm(fmt, packed, a, a_dtype, c, c_dtype, M, N, K, ptr, kGemmScratchBytes, stream);
}
