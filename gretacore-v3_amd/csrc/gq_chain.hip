// gq_chain.hip -- a decode step's chain of GEMVs in one persistent launch.
//
// The reference runs every projection of a decode step as its own launch
// (BlockScheduler: q, k, v, o, gate, up, down per layer,
// block_scheduler.cpp:1831-1894, 2769-2775, 2967-3003), and so do gq_gemv /
// gq_gemv_multi / gq_gemv_swiglu: each launch pays the dispatch gap between
// dependent kernels (~1.8 us on MI355X, as long as streaming 14 MB) plus its
// own ramp and tail.  Weight streaming does not depend on the activations, so
// here one launch runs an ordered list of GEMV "ops" (include/gq_chain.h) and
// an op's weight loads are issued before its inputs exist.
//
// Design (batch 1, int8 matrix cores as gq_gemv.hip's kernel):
//  * Persistent grid, one workgroup per CU (all resident at once; the host
//    checks the occupancy): 8 compute waves that split K, and one control
//    wave.  The ops are cut into units (NACC 16-row output tiles over the op's
//    whole K), numbered in op order; workgroup g takes units g, g + G, ...
//  * A compute wave holds two register sets of weight chunks: while it
//    computes unit j it already has unit j + G's loads in flight, which so
//    also cover the wait for that unit's inputs.
//  * The control wave never has weight loads in flight, so its waits are
//    short: it polls the dependencies, copies the op's x into LDS (LDS DMA,
//    with the GQA map applied to the addresses), and finishes every unit: the
//    K-split reduction, RMS factor, residual or SwiGLU, the stores, a release
//    fence and the op's counter.  It does this for unit j while the compute
//    waves already consume unit j + G (the partial sums are double-buffered).
//  * The activations are split into int8 limbs once per op and wave (every
//    unit of an op reads the same x), not once per unit.
//  * Dependencies: a unit whose op names op d waits until d's counter
//    reaches d's unit count, then acquires (invalidating this CU's caches, so
//    the other workgroups' outputs are read from memory).  Units are taken in
//    op order, ops depend only on earlier ops and all workgroups are
//    resident, so the waits end; each is also bounded: past the spin limit it
//    sets an error flag and every later wait returns at once, so the kernel
//    always drains.
#include <stdlib.h>

#include <map>
#include <mutex>
#include <vector>

#include "gq_gemv_i8.h"
#include "../../include/gq_chain.h"

namespace {

constexpr int kCW = 8;   // compute waves (the K split)
constexpr int kAcc = 4;  // output tiles (accumulators) per unit at most

// chunk slots per compute wave and register set (two sets are held)
template <int FMT>
struct ChainSlots;
template <>
struct ChainSlots<GQ_FMT_Q4_0> {
  static constexpr int S = 8;  // 5 VGPRs each
};
template <>
struct ChainSlots<GQ_FMT_Q8_0> {
  static constexpr int S = 4;  // 9 VGPRs each
};
template <>
struct ChainSlots<GQ_FMT_Q4_K> {
  static constexpr int S = 4;  // 12 VGPRs each
};
int chain_slots(int f) { return f == GQ_FMT_Q4_0 ? 8 : 4; }

// Device op record (the host builds it from gq_chain_op).
struct ChainOpD {
  const uint8_t *w, *w2;  // matrix (SwiGLU: gate), up matrix or null
  const float *x, *gamma, *resid;
  float *y;
  uint64_t sc_off;       // scale-plane offset of the tensor (w2: same shape)
  int N, K, C, Crow;     // rows, K of this op, its chunks, chunks per row of the tensor
  int cbase, nck;        // first chunk of the op in a row, chunks per wave (ceil(C / kCW))
  int nacc, pair;        // accumulators per unit (SwiGLU: gate, up alternate), SwiGLU flag
  int unit0, units;      // first unit (global numbering), unit count
  int dep[3];
  int xhd, xgrp;         // GQA read of x (0: none)
  int pad[3];
};
static_assert(sizeof(ChainOpD) == 128, "op record size");

// the op table's pointers are device memory: global-address-space views of
// them, so their accesses are global (not flat) memory instructions
template <typename T>
GQ_DEV const GQ_GLOBAL T *gmem(const T *p) {
  return (const GQ_GLOBAL T *)p;
}
template <typename T>
GQ_DEV GQ_GLOBAL T *gmem_w(T *p) {
  return (GQ_GLOBAL T *)p;
}

// Two ops whose inputs stage identically: same x, RMSNorm weight, GQA map and
// K slices, and the second depends on nothing the first did not (its inputs
// were complete when the first staged them).
GQ_DEV bool same_input(const ChainOpD &a, const ChainOpD &b) {
  return a.x == b.x && a.gamma == b.gamma && a.K == b.K && a.C == b.C && a.xhd == b.xhd && a.xgrp == b.xgrp &&
         a.dep[0] == b.dep[0] && a.dep[1] == b.dep[1] && a.dep[2] == b.dep[2];
}

GQ_DEV unsigned ld_agent(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

template <int FMT>
__global__ void __launch_bounds__(64 * (kCW + 1), 1)
k_chain(const ChainOpD *__restrict__ ops, int n_ops, int total, unsigned *__restrict__ done, unsigned *__restrict__ err,
        float eps, unsigned spin_limit, int xs_bytes) {
  using F = Fmt<FMT>;
  constexpr int NS = ChainSlots<FMT>::S;
  constexpr int LKMAX = F::CK * NS;  // a compute wave's K slice at most
  constexpr int TPR = (LKMAX + 511) / 512;  // 8-element runs per lane
  constexpr float OFF = (FMT == GQ_FMT_Q4_0) ? 8.f : (FMT == GQ_FMT_Q4_K) ? 1.f : 0.f;
  extern __shared__ __attribute__((aligned(16))) unsigned char gq_dyn_lds[];
  __shared__ float red[2][kCW][kAcc][16];  // partial sums, double-buffered by unit parity
  __shared__ float ssred[kCW];              // per-wave sums of squares of the op's x
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool ctl = wave == kCW;
  const int g = lane >> 4, r = lane & 15;
  const int G = (int)gridDim.x;
  float *const xs = reinterpret_cast<float *>(gq_dyn_lds);  // the op's x (fp32)
  const XlLayout L = xl_layout(LKMAX, 1);
  unsigned char *const lbase = gq_dyn_lds + xs_bytes + (size_t)(ctl ? 0 : wave) * L.wave_bytes;
  int8_t *const lm = reinterpret_cast<int8_t *>(lbase);
  float *const lsc = reinterpret_cast<float *>(lbase + L.scl_off);
  const int8_t *const lzero = reinterpret_cast<const int8_t *>(lbase + L.zero_off);
  if (!ctl)
    for (int o = 16 * lane; o < L.lk; o += 1024)  // the zero A rows, once
      *reinterpret_cast<gq_u4 *>(lbase + L.zero_off + o) = gq_u4{0u, 0u, 0u, 0u};
  const uint32_t qlane = 16u * (uint32_t)lane;
  const uint32_t slane = FMT == GQ_FMT_Q4_K ? 16u * (uint32_t)r : 8u * (uint32_t)r + 4u * (uint32_t)(g >> 1);

  int oi = 0;  // op of the last unit looked up (units ascend: scan forward)
  auto op_of = [&](int u) {
    while (oi + 1 < n_ops && u >= ops[oi + 1].unit0) ++oi;
    return oi;
  };
  // Chunk slot s of unit u: accumulator a = s / nck, chunk i = s % nck of
  // this wave's K slice.  Slots past the unit's accumulators or the slice
  // re-read a valid chunk: the loads are unconditional.
  auto issue = [&](int u, Chunk<FMT>(&ch)[NS]) {
    const ChainOpD &op = ops[op_of(u)];
    const int j = u - op.unit0;
    const int ntiles = (int)gq_tiles(op.N);
    const int c0 = (op.C * wave) / kCW, c1 = (op.C * (wave + 1)) / kCW;
    const int nw = c1 - c0;
    const int tpu = op.pair ? op.nacc >> 1 : op.nacc;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      int a = s / op.nck, i = s % op.nck;
      a = a < op.nacc ? a : op.nacc - 1;
      i = i < nw ? i : (nw > 0 ? nw - 1 : 0);
      const uint8_t *wm = (op.pair && (a & 1)) ? op.w2 : op.w;
      int t = j * tpu + (op.pair ? a >> 1 : a);
      t = t < ntiles ? t : ntiles - 1;
      const size_t ci = (size_t)t * op.Crow + op.cbase + c0 + i;
      load_chunk<FMT>(wm + ci * F::QB, wm + op.sc_off + ci * F::SB, qlane, slane, ch[s]);
    }
  };

  int cur_op = -1;
  auto process = [&](int u, Chunk<FMT>(&cur)[NS], Chunk<FMT>(&nxt)[NS], auto parity) {
    constexpr int P = decltype(parity)::value;
    const int o = op_of(u);
    const ChainOpD &op = ops[o];
    const int j = u - op.unit0;
    const int c0 = (op.C * wave) / kCW, c1 = (op.C * (wave + 1)) / kCW;
    const int nw = ctl ? 0 : c1 - c0;
    const bool norm = op.gamma != nullptr;

    if (o != cur_op && (cur_op < 0 || !same_input(ops[cur_op], op))) {  // (wave-uniform)
      // ---- a new op: its inputs, then its x -> LDS, then int8 limbs ---------
      if (ctl) {
        if (lane == 0) {
          for (int q = 0; q < 3; ++q) {
            const int d = op.dep[q];
            if (d < 0) continue;
            const unsigned need = (unsigned)ops[d].units;
            unsigned spins = 0;
            while (ld_agent(done + d) < need) {
              if (ld_agent(err) != 0u) break;  // an earlier wait gave up: drain
              if (++spins > spin_limit) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
              }
              __builtin_amdgcn_s_sleep(1);
            }
          }
        }
        // acquire: this CU's L1 and its XCD's L2 drop what other workgroups'
        // stores made stale, for every wave of the workgroup
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        // x -> LDS: 16 bytes per lane per instruction (LDS DMA, no registers);
        // the GQA map keeps runs of 4 together (head_dim % 8 == 0)
        for (int k0 = 0; k0 < op.K; k0 += 256) {
          int k = k0 + 4 * lane;
          k = k < op.K ? k : 0;
          if (op.xhd > 0) k = (k / (op.xhd * op.xgrp)) * op.xhd + k % op.xhd;
          __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(op.x + k),
                                           (__attribute__((address_space(3))) void *)(xs + k0), 16, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      }
      __syncthreads();
      if (!ctl) {
        const int k0 = c0 * F::CK, LK = nw * F::CK;
        float4 gv[TPR][2];
        if (norm) {
#pragma unroll
          for (int i = 0; i < TPR; ++i) {
            const int e8 = lane + 64 * i;
            const int k = (8 * e8 < LK && k0 + 8 * e8 < op.K) ? k0 + 8 * e8 : 0;
            const GQ_GLOBAL gq_f4 *gp = (const GQ_GLOBAL gq_f4 *)gmem(op.gamma + k);
            const gq_f4 g0 = gp[0], g1 = gp[1];
            gv[i][0] = float4{g0[0], g0[1], g0[2], g0[3]};
            gv[i][1] = float4{g1[0], g1[1], g1[2], g1[3]};
          }
        }
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < TPR; ++i) {
          const int e8 = lane + 64 * i;
          const bool in = 8 * e8 < LK && k0 + 8 * e8 < op.K;  // (K % 32 == 0: runs are whole)
          const float4 a0 = *reinterpret_cast<const float4 *>(xs + (in ? k0 + 8 * e8 : 0));
          const float4 a1 = *reinterpret_cast<const float4 *>(xs + (in ? k0 + 8 * e8 + 4 : 4));
          float v[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
          float amax = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            v[e] = in ? v[e] : 0.f;
            ss += v[e] * v[e];
            amax = fmaxf(amax, fabsf(v[e]));
          }
          if (norm) {  // x * gamma; the 1 / rms factor is applied after the K reduction
            const float gg[8] = {gv[i][0].x, gv[i][0].y, gv[i][0].z, gv[i][0].w,
                                 gv[i][1].x, gv[i][1].y, gv[i][1].z, gv[i][1].w};
            amax = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              v[e] *= gg[e];
              amax = fmaxf(amax, fabsf(v[e]));
            }
          }
          amax = quad_max(amax);
          const float inv = amax > 0.f ? 127.0f * __builtin_amdgcn_rcpf(amax) : 0.f;
          const float sx = amax * (1.0f / 127.0f);
          uint32_t la[2], lb[2];
          const int t8 = split8(v, inv, la, lb);
          const float sm = (float)quad_sum(t8) * (sx * (1.0f / 254.0f));
          if (in) {
            *reinterpret_cast<gq_u2 *>(lm + 8 * e8) = gq_u2{la[0], la[1]};
            *reinterpret_cast<gq_u2 *>(lm + L.lk + 8 * e8) = gq_u2{lb[0], lb[1]};
            if ((lane & 3) == 0)
              *reinterpret_cast<gq_f4 *>(lsc + 4 * (e8 >> 2)) = gq_f4{sx, sm, sx * (1.0f / 254.0f), 0.f};
          }
        }
        ss = wave_sum(ss);
        if (lane == 0) ssred[wave] = ss;
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
      }
    }
    if (o != cur_op) {
      // (a new op on the same input keeps the staged limbs; its dependencies
      // were those of the op that staged them, or later ones already met)
      cur_op = o;
    }

    if (!ctl) {
      // ---- the next unit's weights, then this unit's chunks ---------------------
      issue(u + G < total ? u + G : u, nxt);  // (the last unit re-reads its own chunks)
      // A operand: lane (r, g) is combination c = r >> 2 = (block h, limb l)
      // of the batch row (r & 3 == 0), with data where its lane group covers
      // block h of the MFMA pair, zeros otherwise (as gq_gemv.hip's kernel)
      const int c = r >> 2, h = c >> 1, l = c & 1;
      const bool act = ((g >> 1) == h) && (r & 3) == 0;
      const int8_t *abase = act ? lm + (size_t)l * L.lk + 32 * h + 16 * (g & 1) : lzero;
      const int hp = g >> 1, lp = g & 1;
      float tot[kAcc];
#pragma unroll
      for (int q = 0; q < kAcc; ++q) tot[q] = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int a = s / op.nck, i = s % op.nck;
        if (a >= op.nacc || i >= nw) continue;
        const Chunk<FMT> &cc = cur[s];
        float acc = 0.f, cor = 0.f;
#pragma unroll
        for (int m = 0; m < F::STEPS; ++m) {
          const int koff = i * F::CK + 64 * m;
          const int blk = i * (F::CK / 32) + 2 * m + hp;
          const gq_i4 av = *reinterpret_cast<const gq_i4 *>(abase + koff);
          const float2 sv = *reinterpret_cast<const float2 *>(lsc + 4 * blk + 2 * lp);
          gq_i4 bop;
          float ws, wmn = 0.f;
          if constexpr (FMT == GQ_FMT_Q4_0) {
            bop = codes16(cc.q[2 * m], cc.q[2 * m + 1]);
            ws = m ? h16hi(cc.d) : h16lo(cc.d);
            wmn = ws;
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
            wmn = h16hi(cc.meta[0]) * (float)((byte >> 6) | (b3 << 2));
          }
          const gq_i4 D = mfma_i8(av, bop);
          acc += (ws * sv.x) * (float)D[0];
          if constexpr (FMT != GQ_FMT_Q8_0) cor += wmn * sv.y;
        }
        const float val = acc - OFF * cor;
#pragma unroll
        for (int q = 0; q < kAcc; ++q) tot[q] += (a == q) ? val : 0.f;
      }
#pragma unroll
      for (int q = 0; q < kAcc; ++q) {
        const float p = sum_lane_groups(tot[q]);
        if (g == 0) red[P][wave][q][r] = p;
      }
    }
    __syncthreads();
    if (!ctl) return;

    // ---- control wave: finish the unit ------------------------------------------
    float inv = 1.f;
    if (norm) {
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < kCW; ++q) t += ssred[q];
      inv = 1.0f / sqrtf(t / (float)op.K + eps);
    }
    const int tpu = op.pair ? op.nacc >> 1 : op.nacc;
    if (lane < 16) {
      float part[kAcc];
#pragma unroll
      for (int q = 0; q < kAcc; ++q) {
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kCW; ++w) sum += red[P][w][q][r];
        part[q] = sum * inv;
      }
#pragma unroll
      for (int q = 0; q < kAcc; ++q) {
        if (q >= tpu) continue;
        const size_t row = (size_t)(j * tpu + q) * 16 + r;
        if (row >= (size_t)op.N) continue;
        float out;
        if (op.pair) {  // accumulators 2q (gate) and 2q + 1 (up)
          const float gt = part[(2 * q) % kAcc], up = part[(2 * q + 1) % kAcc];
          out = gt / (1.0f + expf(-gt)) * up;
        } else {
          out = part[q] + (op.resid ? gmem(op.resid)[row] : 0.f);
        }
        // agent-scope store: written through this XCD's L2 to memory, where
        // the other XCDs read it
        __hip_atomic_store(op.y + row, out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    // publish: once the stores are complete (vmcnt(0): the control wave has no
    // other memory operation in flight), the op's counter.  (A release fence
    // would also write back this XCD's whole L2, which costs microseconds;
    // the only data published is the write-through stores above.)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (lane == 0) __hip_atomic_fetch_add(done + o, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };

  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  Chunk<FMT> cA[NS], cB[NS];
  int u = (int)blockIdx.x;
  if (u >= total) return;
  if (!ctl) issue(u, cA);
  while (true) {
    process(u, cA, cB, P0{});
    u += G;
    if (u >= total) break;
    process(u, cB, cA, P1{});
    u += G;
    if (u >= total) break;
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // (the last, redundant prefetch lands before the wave ends)
}

// ---- host side ------------------------------------------------------------------
struct ChainHdr {  // the plan, kept on the host per workspace
  int fmt, n_ops, total, grid, xs_bytes, lds_bytes;
  float eps;
  unsigned spin_limit;
  size_t done_off, err_off, ops_off;
};
std::mutex g_chain_mutex;
std::map<const void *, ChainHdr> g_chain_plans;

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

int chain_fmt(int fmt) { return gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt; }

// Device ops for the caller's ops: ops whose K needs more chunks per wave
// than the slots hold are cut into column ranges chained through resid.
int build_ops(int fmt, const gq_chain_op *ops, int n_ops, std::vector<ChainOpD> &out, int *max_k) {
  const int f = chain_fmt(fmt);
  GQ_CHECK(f == GQ_FMT_Q4_0 || f == GQ_FMT_Q8_0 || f == GQ_FMT_Q4_K, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(ops && n_ops >= 1, GQ_ERR_INVALID_ARGS);
  const int S = chain_slots(f);
  const int ck = (int)gq_chunk_k(f);
  std::vector<int> last(n_ops, -1);  // device index of each caller op's final range
  int unit0 = 0;
  *max_k = 0;
  out.clear();
  for (int i = 0; i < n_ops; ++i) {
    const gq_chain_op &p = ops[i];
    GQ_CHECK(p.w && p.x && p.y && p.N > 0 && p.K > 0, GQ_ERR_INVALID_ARGS);
    const size_t kt = p.k_total ? p.k_total : (size_t)p.K + p.k_offset;
    GQ_TRY(gq_check_shape(f, p.N, kt));
    GQ_CHECK(p.k_offset % (uint32_t)ck == 0 && p.K % 32 == 0 && p.k_offset + (size_t)p.K <= kt, GQ_ERR_INVALID_ARGS);
    GQ_CHECK(!(p.w_up && p.resid), GQ_ERR_INVALID_ARGS);
    GQ_CHECK(p.x_head_dim == 0 || (p.x_head_dim % 8 == 0 && p.x_group > 0), GQ_ERR_INVALID_ARGS);
    for (int q = 0; q < 3; ++q) GQ_CHECK(p.dep[q] < i && p.dep[q] >= -1, GQ_ERR_INVALID_ARGS);
    const int C = (int)((p.K + ck - 1) / ck);
    const int nck_full = (C + kCW - 1) / kCW;
    const int pieces = (nck_full + S - 1) / S;
    // a cut op must be linear in x: no norm, GQA map or SwiGLU
    GQ_CHECK(pieces == 1 || (!p.gamma && !p.w_up && p.x_head_dim == 0), GQ_ERR_UNSUPPORTED);
    const int cper = (C + pieces - 1) / pieces;
    for (int pc = 0; pc < pieces; ++pc) {
      ChainOpD d{};
      const int cb = pc * cper, ce = (pc + 1) * cper < C ? (pc + 1) * cper : C;
      d.w = (const uint8_t *)p.w;
      d.w2 = (const uint8_t *)p.w_up;
      d.x = p.x + (size_t)cb * ck;
      d.gamma = p.gamma;
      d.resid = pc == 0 ? p.resid : p.y;  // later ranges add to the earlier ones
      d.y = p.y;
      d.sc_off = gq_sc_plane_offset(f, p.N, kt);
      d.N = (int)p.N;
      d.K = pc + 1 < pieces ? (ce - cb) * ck : (int)p.K - cb * ck;
      d.C = ce - cb;
      d.Crow = (int)gq_chunks(f, kt);
      d.cbase = (int)(p.k_offset / (uint32_t)ck) + cb;
      d.nck = (d.C + kCW - 1) / kCW;
      int nacc = S / d.nck;
      nacc = nacc < kAcc ? nacc : kAcc;
      if (p.w_up) {
        nacc &= ~1;
        GQ_CHECK(nacc >= 2, GQ_ERR_UNSUPPORTED);  // (K too long for a SwiGLU pair)
      }
      d.nacc = nacc;
      d.pair = p.w_up ? 1 : 0;
      const int tpu = d.pair ? nacc / 2 : nacc;
      d.units = (int)((gq_tiles(p.N) + tpu - 1) / tpu);
      d.unit0 = unit0;
      unit0 += d.units;
      if (pc == 0) {
        for (int q = 0; q < 3; ++q) d.dep[q] = p.dep[q] >= 0 ? last[p.dep[q]] : -1;
      } else {
        d.dep[0] = (int)out.size() - 1;
        d.dep[1] = d.dep[2] = -1;
      }
      d.xhd = (int)p.x_head_dim;
      d.xgrp = (int)p.x_group;
      *max_k = d.K > *max_k ? d.K : *max_k;
      out.push_back(d);
    }
    last[i] = (int)out.size() - 1;
  }
  return GQ_OK;
}

size_t chain_ws_bytes(size_t n_dev_ops) {
  return 256 /* counters' line */ + al256(n_dev_ops * 4) + 256 /* error flag */ + al256(n_dev_ops * sizeof(ChainOpD));
}

template <int FMT>
int chain_lds(int xs_bytes) {
  using F = Fmt<FMT>;
  return xs_bytes + kCW * xl_layout(F::CK * ChainSlots<FMT>::S, 1).wave_bytes;
}

template <int FMT>
int chain_launch(const ChainHdr &h, const uint8_t *ws, hipStream_t s) {
  hipLaunchKernelGGL(k_chain<FMT>, dim3((unsigned)h.grid), dim3(64 * (kCW + 1)), (size_t)h.lds_bytes, s,
                     (const ChainOpD *)(ws + h.ops_off), h.n_ops, h.total, (unsigned *)(ws + h.done_off),
                     (unsigned *)(ws + h.err_off), h.eps, h.spin_limit, h.xs_bytes);
  return gq_last_launch();
}

template <int FMT>
int chain_occupancy(int lds, int *per_cu) {
  return gq_hip_status(hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, k_chain<FMT>, 64 * (kCW + 1),
                                                                    (size_t)lds));
}

}  // namespace

extern "C" int gq_gemv_chain_workspace_bytes(int fmt, const gq_chain_op *ops, int n_ops, size_t *bytes) {
  GQ_CHECK(bytes, GQ_ERR_INVALID_ARGS);
  std::vector<ChainOpD> d;
  int mk = 0;
  GQ_TRY(build_ops(fmt, ops, n_ops, d, &mk));
  *bytes = chain_ws_bytes(d.size());
  return GQ_OK;
}

extern "C" int gq_gemv_chain_plan(int fmt, const gq_chain_op *ops, int n_ops, float eps, void *ws, size_t ws_bytes) {
  GQ_CHECK(ws, GQ_ERR_INVALID_ARGS);
  std::vector<ChainOpD> d;
  int max_k = 0;
  GQ_TRY(build_ops(fmt, ops, n_ops, d, &max_k));
  GQ_CHECK(ws_bytes >= chain_ws_bytes(d.size()), GQ_ERR_WORKSPACE);
  ChainHdr h{};
  h.fmt = chain_fmt(fmt);
  h.n_ops = (int)d.size();
  h.total = d.back().unit0 + d.back().units;
  h.eps = eps;
  h.xs_bytes = (int)((max_k + 255) / 256 * 256 * 4);  // (the DMA writes whole 256-element runs)
  h.lds_bytes = h.fmt == GQ_FMT_Q4_0 ? chain_lds<GQ_FMT_Q4_0>(h.xs_bytes)
                : h.fmt == GQ_FMT_Q8_0 ? chain_lds<GQ_FMT_Q8_0>(h.xs_bytes)
                                       : chain_lds<GQ_FMT_Q4_K>(h.xs_bytes);
  GQ_CHECK(h.lds_bytes <= 160 * 1024 - 8192, GQ_ERR_UNSUPPORTED);  // (x too long for the LDS copy)
  int per_cu = 0;
  switch (h.fmt) {
  case GQ_FMT_Q4_0: GQ_TRY(chain_occupancy<GQ_FMT_Q4_0>(h.lds_bytes, &per_cu)); break;
  case GQ_FMT_Q8_0: GQ_TRY(chain_occupancy<GQ_FMT_Q8_0>(h.lds_bytes, &per_cu)); break;
  default: GQ_TRY(chain_occupancy<GQ_FMT_Q4_K>(h.lds_bytes, &per_cu)); break;
  }
  const int cus = gq_device_cus();
  GQ_CHECK(per_cu >= 1 && cus > 0, GQ_ERR_UNSUPPORTED);
  h.grid = cus;  // one workgroup per CU: every workgroup resident at once
  const char *e = getenv("GQ_CHAIN_SPIN");
  h.spin_limit = e ? (unsigned)strtoul(e, nullptr, 0) : (1u << 22);
  h.done_off = 256;
  h.err_off = h.done_off + al256(d.size() * 4);
  h.ops_off = h.err_off + 256;
  GQ_TRY(gq_hip_status(hipMemcpy((uint8_t *)ws + h.ops_off, d.data(), d.size() * sizeof(ChainOpD),
                                 hipMemcpyHostToDevice)));
  std::lock_guard<std::mutex> lock(g_chain_mutex);
  g_chain_plans[ws] = h;
  return GQ_OK;
}

extern "C" int gq_gemv_chain_run(const void *ws, void *stream) {
  GQ_CHECK(ws, GQ_ERR_INVALID_ARGS);
  ChainHdr h;
  {
    std::lock_guard<std::mutex> lock(g_chain_mutex);
    auto it = g_chain_plans.find(ws);
    GQ_CHECK(it != g_chain_plans.end(), GQ_ERR_INVALID_ARGS);  // no plan in this workspace
    h = it->second;
  }
  hipStream_t s = (hipStream_t)stream;
  const uint8_t *w = (const uint8_t *)ws;
  // counters and the error flag start at zero (a kernel, not a memset node)
  GQ_TRY(gq_fill_zero((float *)(w + h.done_off), (h.ops_off - h.done_off) / 4, s));
  switch (h.fmt) {
  case GQ_FMT_Q4_0: return chain_launch<GQ_FMT_Q4_0>(h, w, s);
  case GQ_FMT_Q8_0: return chain_launch<GQ_FMT_Q8_0>(h, w, s);
  default: return chain_launch<GQ_FMT_Q4_K>(h, w, s);
  }
}

extern "C" int gq_gemv_chain_error(const void *ws, int *error) {
  GQ_CHECK(ws && error, GQ_ERR_INVALID_ARGS);
  ChainHdr h;
  {
    std::lock_guard<std::mutex> lock(g_chain_mutex);
    auto it = g_chain_plans.find(ws);
    GQ_CHECK(it != g_chain_plans.end(), GQ_ERR_INVALID_ARGS);
    h = it->second;
  }
  unsigned v = 0;
  GQ_TRY(gq_hip_status(hipMemcpy(&v, (const uint8_t *)ws + h.err_off, 4, hipMemcpyDeviceToHost)));
  *error = v ? 1 : 0;
  return GQ_OK;
}
