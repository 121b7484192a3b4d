// gq_chain.hip -- a decode step's chain of GEMVs in one persistent launch.
//
// The reference runs every projection of a decode step as its own launch
// (BlockScheduler: q, k, v, o, gate, up, down per layer,
// block_scheduler.cpp:1831-1894, 2769-2775, 2967-3003), and so do gq_gemv /
// gq_gemv_multi / gq_gemv_swiglu: each launch pays the dispatch gap between
// dependent kernels (~1.6 us on MI355X, as long as streaming 12 MB) plus its
// own ramp and tail.  Weight streaming does not depend on the activations, so
// here one launch runs an ordered list of GEMV "ops" (include/gq_chain.h) and
// the weights of later ops are in flight while an op waits for its inputs.
//
// Design (batch 1, int8 matrix cores as gq_gemv.hip's kernel):
//  * Persistent grid, one workgroup per CU (all resident at once; the host
//    checks the occupancy): kCW = 4 compute waves, one per SIMD, that split
//    K, and one control wave.  An op is cut into units -- one 16-row output
//    tile over the op's K (SwiGLU: the same tile of gate and of up) --
//    numbered in op order, and workgroup g takes units g, g + G, ..., so the
//    units of every op are spread over all CUs.
//  * A compute wave walks one stream of chunk loads: its K slice of every
//    unit of its workgroup, in order.  A register ring keeps NSLOT chunks in
//    flight: when the wave consumes stream position p it requests position
//    p + NSLOT, whichever unit or op that is.  The ring is indexed by
//    compile-time slot numbers (the loop body is unrolled NSLOT times) and
//    every request is unconditional (past the end it re-reads a valid chunk),
//    so the waits on the loads stay in issue order.
//  * The control wave never holds weight loads, so its waits are short.  Per
//    activation stage (ops that read the same input: q, k and v of a layer)
//    it waits until the ops the stage depends on are complete, copies x into
//    LDS (LDS DMA, with the GQA map applied to the addresses) and the RMSNorm
//    weight, computes 1 / rms and posts x * gamma; each compute wave then
//    splits its K slice per 32-block into the two int8 limbs the matrix
//    cores take (the GEMV's split).  Per unit it sums the compute waves' partial tiles, applies
//    1 / rms, the residual or SwiGLU, and stores the rows.
//  * Compute and control waves meet only through LDS counters: a ring of kRed
//    partial-tile slots (arrivals / slots freed), the posted stage and the
//    compute waves' release of the stage's x once they have converted it.  The control
//    wave's global latencies therefore never stall the weight stream; the
//    compute waves wait only for a stage's limbs or a free slot.
//  * Completion of an op: the control wave stores its rows with agent-scope
//    (write-through) stores and, when its workgroup moves to another op,
//    waits for them (vmcnt(0)) and sets its flag for the op.  A stage whose
//    ops name op d waits until every workgroup holding units of d has set its
//    flag, and reads the outputs of other workgroups with agent-scope loads.  Units are taken in op
//    order, ops depend only on earlier ops and all workgroups are resident,
//    so the waits end; each is also bounded: past the spin limit it sets an
//    error flag and every later wait returns at once, so the kernel always
//    drains.
#include <stdlib.h>

#include <map>
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "gq_gemv_i8.h"
#include "../../include/gq_chain.h"

namespace {

constexpr int kCW = 4;              // compute waves (the K split), one per SIMD
constexpr int kRed = 4;             // partial-tile slots between compute and control waves
constexpr int kMaxPieceK = 16384;   // longest K of one device op (LDS holds its x and limbs)
constexpr int kMaxGrid = 256;       // workgroups at most (one per CU); completion flags per op

// register ring per format: NSLOT chunks in flight per compute wave, LPC loads
// per chunk (NSLOT * LPC <= 63, the vmcnt range)
template <int FMT>
struct Ring;
template <>
struct Ring<GQ_FMT_Q4_0> {
  static constexpr int NSLOT = 20;  // 5 VGPRs per chunk
};
template <>
struct Ring<GQ_FMT_Q8_0> {
  static constexpr int NSLOT = 12;  // 9 VGPRs
};
template <>
struct Ring<GQ_FMT_Q4_K> {
  static constexpr int NSLOT = 12;  // 12 VGPRs
};

// Device op record (the host builds it from gq_chain_op).
struct ChainOpD {
  const uint8_t *w, *w2;  // matrix (SwiGLU: gate), up matrix or null
  const float *x, *gamma, *resid;
  float *y;
  uint64_t sc_off;       // scale-plane offset of the tensor (w2: same shape)
  int N, K, C, Crow;     // rows, K of this op, its chunks, chunks per row of the tensor
  int cbase, pair;       // first chunk of the op in a row, SwiGLU flag
  int unit0, units;      // first unit (global numbering), unit count (= row tiles)
  int dep[3];
  int xhd, xgrp;         // GQA read of x (0: none)
  int stage;             // activation stage (ops of one stage read the same input)
  int pad[4];
};
static_assert(sizeof(ChainOpD) == 128, "op record size");

// LDS words shared by the compute and control waves of a workgroup
struct ChainSync {
  unsigned xready;    // activation stages posted by the control wave
  unsigned released;  // stages whose x the compute waves have converted (kCW per stage)
  unsigned freed;     // units whose partial-tile slot the control wave has read
  unsigned lerr;      // a wait of this workgroup gave up
  unsigned arrive[kRed];  // partial tiles written into each slot (kCW per use)
};

// the op table's pointers are device memory: global-address-space views of
// them, so their accesses are global (not flat) memory instructions
#define GQ_CONST __attribute__((address_space(4)))
template <typename T>
GQ_DEV const GQ_GLOBAL T *gmem(const T *p) {
  return (const GQ_GLOBAL T *)p;
}

// Two ops whose inputs stage identically: same x, RMSNorm weight, GQA map and
// K range, and the same dependencies (its inputs complete when the first's are).
__host__ __device__ inline bool same_input(const ChainOpD &a, const ChainOpD &b) {
  return a.x == b.x && a.gamma == b.gamma && a.K == b.K && a.C == b.C && a.xhd == b.xhd && a.xgrp == b.xgrp &&
         a.dep[0] == b.dep[0] && a.dep[1] == b.dep[1] && a.dep[2] == b.dep[2];
}

GQ_DEV unsigned ld_agent(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
GQ_DEV unsigned lds_ld(const unsigned *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
GQ_DEV void lds_st(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
GQ_DEV void lds_add(unsigned *p, unsigned v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// LDS writes of this wave complete before what follows (no vector-memory
// wait: the compute waves keep their weight loads in flight)
GQ_DEV void lds_order() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Waits (bounded) until the LDS word reaches v; false if it gave up or an
// earlier wait of the workgroup did.
GQ_DEV bool lds_wait_ge(const unsigned *p, unsigned v, ChainSync *sy, unsigned spin_limit) {
  unsigned spins = 0;
  while (lds_ld(p) < v) {
    if (lds_ld(&sy->lerr) != 0u) return false;
    if (++spins > spin_limit) {
      lds_st(&sy->lerr, 1u);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

template <typename F, int... I>
GQ_DEV void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
GQ_DEV void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS layout (dynamic part): x * gamma as fp32 [kx]; per compute wave its
// limbs: limb a [sl], limb b [sl], per 32-block float4 (s, S, s / 254, 0)
// [sl / 32] (sl: the longest K slice of a wave); a zero region [zl]
struct ChainLds {
  int kx, sl, zl;
  int xs, lw, wb, lz, bytes;
};
__host__ __device__ inline ChainLds chain_lds_layout(int kx, int sl, int zl) {
  ChainLds L;
  L.kx = kx;
  L.sl = sl;
  L.zl = zl;
  L.xs = 0;
  L.lw = L.xs + 4 * kx;
  L.wb = 2 * sl + 16 * (sl / 32);
  L.lz = L.lw + kCW * L.wb;
  L.bytes = L.lz + zl;
  return L;
}

constexpr int kXB = 16;    // float4 loads per lane in one batch of the control wave's x copy
constexpr int kObuf = 64;  // finished rows (16-row tiles) the control wave holds before storing

template <int FMT>
__global__ void __launch_bounds__(64 * (kCW + 1), 1)
k_chain(const ChainOpD *__restrict__ ops_in, int n_ops, int total, unsigned *__restrict__ done, unsigned *__restrict__ err,
        float eps, unsigned spin_limit, ChainLds LL) {
  using F = Fmt<FMT>;
  constexpr int NSLOT = Ring<FMT>::NSLOT;
  // the op table does not change during the launch: read it through the
  // constant address space, so its loads are scalar (SMEM) and never wait on
  // the weight loads in flight
  const GQ_CONST ChainOpD *const ops = (const GQ_CONST ChainOpD *)(ops_in);
  constexpr float OFF = (FMT == GQ_FMT_Q4_0) ? 8.f : (FMT == GQ_FMT_Q4_K) ? 1.f : 0.f;
  extern __shared__ __attribute__((aligned(16))) unsigned char gq_dyn_lds[];
  __shared__ float red[kRed][kCW][2][16];  // partial tiles (gate, up) per slot and compute wave
  __shared__ ChainSync sy;
  __shared__ float obuf[kObuf][16];  // finished rows of the current op, not yet stored
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool ctl = wave == kCW;
  const int g = lane >> 4, r = lane & 15;
  const int G = (int)gridDim.x;
  float *const xs = reinterpret_cast<float *>(gq_dyn_lds + LL.xs);
  const int8_t *const lz = reinterpret_cast<const int8_t *>(gq_dyn_lds + LL.lz);

  if (ctl) {
    for (int o = 16 * lane; o < LL.zl; o += 1024)  // the zero A rows
      *reinterpret_cast<gq_u4 *>(gq_dyn_lds + LL.lz + o) = gq_u4{0u, 0u, 0u, 0u};
    if (lane == 0) {
      sy.xready = sy.released = sy.freed = sy.lerr = 0u;
#pragma unroll
      for (int q = 0; q < kRed; ++q) sy.arrive[q] = 0u;
    }
  }
  __syncthreads();
  if ((int)blockIdx.x >= total) return;

  if (!ctl) {
    // ====================== compute waves ======================================
    const uint32_t qlane = 16u * (uint32_t)lane;
    const uint32_t slane = FMT == GQ_FMT_Q4_K ? 16u * (uint32_t)r : 8u * (uint32_t)r + 4u * (uint32_t)(g >> 1);
    // A operand: lane (r, g) is combination c = r >> 2 = (block h, limb l) of
    // the batch row (r & 3 == 0), with data where its lane group covers block
    // h of the MFMA pair, zeros otherwise (as gq_gemv.hip's kernel)
    const int c = r >> 2, h = c >> 1, l = c & 1;
    const bool act = ((g >> 1) == h) && (r & 3) == 0;
    const int hp = g >> 1, lp = g & 1;
    // this wave's limbs (its K slice of the current stage)
    int8_t *const lw = reinterpret_cast<int8_t *>(gq_dyn_lds + LL.lw + wave * LL.wb);
    float *const lsw = reinterpret_cast<float *>(gq_dyn_lds + LL.lw + wave * LL.wb + 2 * LL.sl);
    const int8_t *const abase = act ? lw + (size_t)l * LL.sl + 32 * h + 16 * (g & 1) : lz;
    const int astep = act ? 1 : 0;  // the zero rows do not move with the chunk

    // stream cursor: unit u (>= total: past the end), its op o, entry e of E
    struct Cur {
      int u, o, e, E, nw, c0;
    };
    auto enter = [&](Cur &cu, int u) {
      cu.u = u;
      cu.e = 0;
      if (u >= total) {
        cu.E = 1;
        return;
      }
      while (cu.o + 1 < n_ops && u >= ops[cu.o + 1].unit0) ++cu.o;
      const GQ_CONST ChainOpD &op = ops[cu.o];
      cu.c0 = (op.C * wave) / kCW;
      cu.nw = (op.C * (wave + 1)) / kCW - cu.c0;
      cu.E = (cu.nw > 0 ? cu.nw : 1) * (op.pair ? 2 : 1);
    };
    auto advance = [&](Cur &cu) {
      if (++cu.e >= cu.E && cu.u < total) enter(cu, cu.u + G);
    };
    // entry e of a unit: matrix (SwiGLU: gate, up alternate) and chunk of the slice
    auto entry = [&](const GQ_CONST ChainOpD &op, int e, int &a, int &i) {
      a = op.pair ? (e & 1) : 0;
      i = op.pair ? (e >> 1) : e;
    };

    Chunk<FMT> ring[NSLOT];
    auto issue = [&](Cur &cu, Chunk<FMT> &slot) {
      const GQ_CONST ChainOpD &op = ops[cu.o];
      int t = 0, a = 0, i = 0;
      if (cu.u < total) {
        t = cu.u - op.unit0;
        entry(op, cu.e, a, i);
        i = i < cu.nw ? i : 0;  // (a wave without chunks re-reads chunk c0 < C)
      }
      const uint8_t *wm = a ? op.w2 : op.w;
      const size_t ci = (size_t)t * (size_t)op.Crow + (size_t)(op.cbase + cu.c0 + i);
      load_chunk<FMT>(wm + ci * F::QB, wm + op.sc_off + ci * F::SB, qlane, slane, slot);
      advance(cu);
    };

    Cur ic, cc;
    ic.o = cc.o = 0;
    enter(ic, (int)blockIdx.x);
    enter(cc, (int)blockIdx.x);
    int stage = -1;        // stage whose limbs this wave reads
    unsigned nstage = 0;   // stages posted that this wave has waited for
    unsigned nunit = 0;    // units of this workgroup finished by this wave
    float tot[2] = {0.f, 0.f};

    auto consume = [&](Chunk<FMT> &slot) {
      const GQ_CONST ChainOpD &op = ops[cc.o];
      if (cc.e == 0) {
        if (op.stage != stage) {  // (wave-uniform) a new stage: wait for its limbs
          ++nstage;
          lds_wait_ge(&sy.xready, nstage, &sy, spin_limit);
          stage = op.stage;
          // x * gamma of this wave's K slice -> two int8 limbs per 32-block
          // (8 elements per lane, a quad of lanes per block); past K: zero
          const int ls = cc.nw * F::CK, kb0 = cc.c0 * F::CK;
          for (int kb = 0; kb < ls; kb += 512) {
            const int kk = kb + 8 * lane, k = kb0 + kk;
            float v[8];
            if (kk < ls && k < op.K) {
              const gq_f4 a0 = *reinterpret_cast<const gq_f4 *>(xs + k);
              const gq_f4 a1 = *reinterpret_cast<const gq_f4 *>(xs + k + 4);
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                v[e] = a0[e];
                v[4 + e] = a1[e];
              }
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) v[e] = 0.f;
            }
            // a NaN or Inf in the block: zero limbs, sx NaN or Inf, NaN outputs
            const float amax = quad_max(abs_max_bits8(v));
            const float rinv = amax > 0.f ? 127.0f * __builtin_amdgcn_rcpf(amax) : 0.f;
            const float sx = amax * (1.0f / 127.0f);
            uint32_t pa[2], pb[2];
            const int t8 = split8(v, rinv, pa, pb);
            const float sm = (float)quad_sum(t8) * (sx * (1.0f / 254.0f));
            if (kk < ls) {
              *reinterpret_cast<gq_u2 *>(lw + kk) = gq_u2{pa[0], pa[1]};
              *reinterpret_cast<gq_u2 *>(lw + LL.sl + kk) = gq_u2{pb[0], pb[1]};
              if ((lane & 3) == 0)
                *reinterpret_cast<gq_f4 *>(lsw + 4 * (kk >> 5)) = gq_f4{sx, sm, sx * (1.0f / 254.0f), 0.f};
            }
          }
          // x may be replaced by the next stage's once every wave has converted it
          lds_order();
          if (lane == 0) lds_add(&sy.released, 1u);
        }
        tot[0] = tot[1] = 0.f;
      }
      int a, i;
      entry(op, cc.e, a, i);
      if (i < cc.nw) {
        const int kc = i * F::CK;  // first k of the chunk in this wave's slice
        float acc = 0.f, cor = 0.f;
#pragma unroll
        for (int m = 0; m < F::STEPS; ++m) {
          const int koff = astep * (kc + 64 * m) + (1 - astep) * (64 * m);
          const int blk = kc / 32 + 2 * m + hp;
          const gq_i4 av = *reinterpret_cast<const gq_i4 *>(abase + koff);
          const float2 sv = *reinterpret_cast<const float2 *>(lsw + 4 * blk + 2 * lp);
          gq_i4 bop;
          float ws, wmn = 0.f;
          if constexpr (FMT == GQ_FMT_Q4_0) {
            bop = codes16(slot.q[2 * m], slot.q[2 * m + 1]);
            ws = m ? h16hi(slot.d) : h16lo(slot.d);
            wmn = ws;
          } else if constexpr (FMT == GQ_FMT_Q8_0) {
            const gq_u4 &qq = m ? slot.q1 : slot.q0;
            bop = gq_i4{(int)qq[0], (int)qq[1], (int)qq[2], (int)qq[3]};
            ws = m ? h16hi(slot.d) : h16lo(slot.d);
          } else {
            const uint32_t w0 = (m < 2) ? slot.qa[2 * (m & 1)] : slot.qb[2 * (m & 1)];
            const uint32_t w1 = (m < 2) ? slot.qa[2 * (m & 1) + 1] : slot.qb[2 * (m & 1) + 1];
            bop = codes16(w0, w1);
            const uint32_t wsc = hp ? slot.meta[2] : slot.meta[1];
            const uint32_t byte = (wsc >> (8 * m)) & 0xFFu;
            const uint32_t b3 = (slot.meta[3] >> (8 * m + 4 * hp)) & 15u;
            ws = h16lo(slot.meta[0]) * (float)(byte & 63u);
            wmn = h16hi(slot.meta[0]) * (float)((byte >> 6) | (b3 << 2));
          }
          const gq_i4 D = mfma_i8(av, bop);
          acc += (ws * sv.x) * (float)D[0];
          if constexpr (FMT != GQ_FMT_Q8_0) cor += wmn * sv.y;
        }
        const float val = acc - OFF * cor;
        if (a) tot[1] += val;
        else tot[0] += val;
      }
      if (cc.e == cc.E - 1) {
        // ---- the unit's partial tile -> a slot for the control wave ------------
        const float p0 = sum_lane_groups(tot[0]);
        const float p1 = op.pair ? sum_lane_groups(tot[1]) : 0.f;
        const int slot_i = (int)(nunit % kRed);
        if (nunit >= kRed) lds_wait_ge(&sy.freed, nunit + 1 - kRed, &sy, spin_limit);
        if (g == 0) {
          red[slot_i][wave][0][r] = p0;
          red[slot_i][wave][1][r] = p1;
        }
        lds_order();
        if (lane == 0) lds_add(&sy.arrive[slot_i], 1u);
        ++nunit;
      }
      advance(cc);
    };

    static_for<NSLOT>([&](auto s) { issue(ic, ring[decltype(s)::value]); });
    while (cc.u < total) {
      static_for<NSLOT>([&](auto s) {
        constexpr int S = decltype(s)::value;
        if (cc.u < total) consume(ring[S]);
        issue(ic, ring[S]);
      });
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the surplus loads land before the wave ends
    if (lds_ld(&sy.lerr) != 0u) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // ====================== control wave ==========================================
  int o = 0;            // op of the current unit
  int cnt_op = -1;      // op whose finished units are not yet counted
  unsigned cnt = 0;     // how many
  int stage = -1;
  unsigned nstage = 0;  // stages posted
  unsigned n = 0;       // units of this workgroup finished
  float inv = 1.f;      // 1 / rms of the current stage (1 without RMSNorm)
  bool bad = false;     // a wait gave up: skip the rest of the waits

  int nbuf = 0;          // rows held in obuf (tiles of op cnt_op)
  int tbuf0 = 0;         // tile of the first of them (the tiles of a workgroup step by G)
  // stores the held rows (agent scope: written through this XCD's L2 to
  // memory, where the other XCDs read them)
  auto flush = [&]() {
    if (nbuf == 0) return;
    const GQ_CONST ChainOpD &op = ops[cnt_op];
    for (int b = 0; b < nbuf; ++b) {
      const int row = 16 * (tbuf0 + b * G) + r;
      if (lane < 16 && row < op.N) __hip_atomic_store(op.y + row, obuf[b][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    nbuf = 0;
  };
  auto publish = [&]() {
    if (cnt_op >= 0 && cnt > 0) {
      flush();
      // the rows' stores complete, then the count
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      // (one flag per workgroup and op: 256 atomic adds on one word
      // serialise at the memory side, ~25 ns each)
      if (lane == 0) __hip_atomic_store(done + (size_t)cnt_op * kMaxGrid + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
    }
    cnt = 0;
  };

  for (int u = (int)blockIdx.x; u < total; u += G, ++n) {
    while (o + 1 < n_ops && u >= ops[o + 1].unit0) ++o;
    const GQ_CONST ChainOpD &op = ops[o];
    if (o != cnt_op) {
      publish();
      cnt_op = o;
    }
    if (op.stage != stage) {
      // ---- a new stage: its inputs complete, x -> LDS, limbs ------------------
      // the compute waves are done with the previous stage's limbs
      if (!bad && nstage > 0) bad = !lds_wait_ge(&sy.released, kCW * nstage, &sy, spin_limit);
      for (int q = 0; q < 3 && !bad; ++q) {
        const int d = op.dep[q];
        if (d < 0) continue;
        // op d is complete when every workgroup that holds units of it has
        // set its flag (workgroup g holds unit u iff u % G == g)
        const int d0 = ops[d].unit0, dn = ops[d].units;
        unsigned spins = 0;
        while (true) {
          bool ok = true;
          for (int g0 = 0; g0 < G; g0 += 64) {
            const int gg = g0 + lane;
            const bool holds = gg < G && (dn >= G || ((gg - d0 % G + G) % G) < dn);
            if (holds && ld_agent(done + (size_t)d * kMaxGrid + gg) == 0u) ok = false;
          }
          if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
          if (ld_agent(err) != 0u || lds_ld(&sy.lerr) != 0u) {
            bad = true;
            break;
          }
          if (++spins > spin_limit) {
            __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            bad = true;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
      if (bad) lds_st(&sy.lerr, 1u);
      // Inputs written by other workgroups are read with agent-scope loads
      // (sc1: never served from a stale line of this XCD's L2), so no
      // acquire fence -- which would invalidate the whole L2 -- is needed.
      // x * gamma -> LDS, in batches of kXB float4 loads per lane (all
      // requested, then used); the GQA map keeps runs of 4 together
      // (head_dim % 8 == 0).  Plain loads, not LDS DMA: a DMA in flight would
      // make every later LDS access of this wave wait on vmcnt, i.e. on the
      // write-through stores of the finished rows.
      const bool norm = op.gamma != nullptr;
      float ss = 0.f;
      for (int k0 = 0; k0 < op.K; k0 += 256 * kXB) {
        gq_f4 xv[kXB], gv[kXB];
#pragma unroll
        for (int j = 0; j < kXB; ++j) {
          int k = k0 + 256 * j + 4 * lane;
          k = k < op.K ? k : 0;
          const int km = op.xhd > 0 ? (k / (op.xhd * op.xgrp)) * op.xhd + k % op.xhd : k;
          const unsigned long long *xp = reinterpret_cast<const unsigned long long *>(op.x + km);
          const unsigned long long v0 = __hip_atomic_load(xp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          const unsigned long long v1 = __hip_atomic_load(xp + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          xv[j] = gq_f4{__uint_as_float((unsigned)v0), __uint_as_float((unsigned)(v0 >> 32)),
                        __uint_as_float((unsigned)v1), __uint_as_float((unsigned)(v1 >> 32))};
          if (norm) gv[j] = *reinterpret_cast<const GQ_GLOBAL gq_f4 *>(gmem(op.gamma + k));
        }
#pragma unroll
        for (int j = 0; j < kXB; ++j) {
          const int k = k0 + 256 * j + 4 * lane;
          if (k < op.K) {
            gq_f4 v = xv[j];
            ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
            if (norm) v = v * gv[j];
            *reinterpret_cast<gq_f4 *>(xs + k) = v;
          }
        }
      }
      // RMSNorm: 1 / rms scales the finished dot products
      inv = norm ? 1.0f / sqrtf(wave_sum(ss) / (float)op.K + eps) : 1.f;
      lds_order();
      ++nstage;
      if (lane == 0) lds_st(&sy.xready, nstage);
      stage = op.stage;
    }

    // ---- finish unit n: the compute waves' partial tiles -----------------------
    const int t = u - op.unit0;
    const int row = 16 * t + r;
    float res = 0.f;
    if (lane < 16 && row < op.N && op.resid && !op.pair)  // (requested before the wait)
      res = __uint_as_float(__hip_atomic_load(reinterpret_cast<const unsigned *>(op.resid) + row, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT));
    const int slot_i = (int)(n % kRed);
    if (!bad) bad = !lds_wait_ge(&sy.arrive[slot_i], kCW * (n / kRed + 1), &sy, spin_limit);
    float p0 = 0.f, p1 = 0.f;
    if (lane < 16) {
#pragma unroll
      for (int w = 0; w < kCW; ++w) {
        p0 += red[slot_i][w][0][r];
        p1 += red[slot_i][w][1][r];
      }
    }
    lds_order();
    if (lane == 0) lds_st(&sy.freed, n + 1);
    if (nbuf == kObuf) flush();
    if (nbuf == 0) tbuf0 = t;
    if (lane < 16) {
      float out;
      if (op.pair) {
        const float gt = p0 * inv, up = p1 * inv;
        out = gt / (1.0f + expf(-gt)) * up;
      } else {
        out = p0 * inv + res;
      }
      obuf[nbuf][r] = out;
    }
    ++nbuf;
    ++cnt;
  }
  publish();
  if (bad || lds_ld(&sy.lerr) != 0u) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- host side ------------------------------------------------------------------
struct ChainHdr {  // the plan, kept on the host per workspace
  int fmt, n_ops, total, grid;
  ChainLds lds;
  float eps;
  unsigned spin_limit;
  size_t done_off, err_off, ops_off;
};
std::mutex g_chain_mutex;
std::map<const void *, ChainHdr> g_chain_plans;

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

int chain_fmt(int fmt) { return gq_fmt_is_q4k(fmt) ? GQ_FMT_Q4_K : fmt; }

// Write hazards between ops: the kernel orders an op after the ops it
// depends on (transitively) and after nothing else, so an op whose y overlaps
// a buffer an earlier op reads (x, gamma, resid) or writes (y) must reach
// that op through its dependencies; otherwise the two may run at the same
// time inside the one launch.  Returns GQ_ERR_INVALID_ARGS for such a pair.
int check_hazards(const gq_chain_op *ops, int n_ops) {
  struct Range {
    uintptr_t a, b;
  };
  auto rng = [](const void *p, size_t n_floats) {
    return Range{(uintptr_t)p, (uintptr_t)p + 4 * n_floats};
  };
  auto meets = [](Range u, Range v) { return u.a < v.b && v.a < u.b; };
  // anc[i][j]: op j precedes op i through dependencies
  std::vector<std::vector<char>> anc(n_ops, std::vector<char>(n_ops, 0));
  for (int i = 0; i < n_ops; ++i) {
    for (int q = 0; q < 3; ++q) {
      const int d = ops[i].dep[q];
      if (d < 0 || d >= i) continue;  // (bad indices are rejected with the op)
      anc[i][d] = 1;
      for (int j = 0; j < d; ++j) anc[i][j] |= anc[d][j];
    }
  }
  auto xlen = [](const gq_chain_op &o) {
    return o.x_head_dim && o.x_group ? (size_t)o.x_head_dim * (o.K / ((size_t)o.x_head_dim * o.x_group))
                                     : (size_t)o.K;
  };
  for (int i = 0; i < n_ops; ++i) {
    const gq_chain_op &p = ops[i];
    const Range yi = rng(p.y, p.N);
    // (an op's own y must not alias its inputs)
    GQ_CHECK(!meets(yi, rng(p.x, xlen(p))) && !(p.gamma && meets(yi, rng(p.gamma, p.K))) &&
                 !(p.resid && meets(yi, rng(p.resid, p.N))),
             GQ_ERR_INVALID_ARGS);
    for (int j = 0; j < i; ++j) {
      const gq_chain_op &o = ops[j];
      const bool hit = meets(yi, rng(o.y, o.N)) || meets(yi, rng(o.x, xlen(o))) ||
                       (o.gamma && meets(yi, rng(o.gamma, o.K))) || (o.resid && meets(yi, rng(o.resid, o.N)));
      GQ_CHECK(!hit || anc[i][j], GQ_ERR_INVALID_ARGS);
    }
  }
  return GQ_OK;
}

// Device ops for the caller's ops: ops whose K exceeds kMaxPieceK are cut
// into column ranges chained through resid; consecutive ops with the same
// input share an activation stage.  Also returns the LDS layout.
int build_ops(int fmt, const gq_chain_op *ops, int n_ops, std::vector<ChainOpD> &out, ChainLds *lds) {
  const int f = chain_fmt(fmt);
  GQ_CHECK(f == GQ_FMT_Q4_0 || f == GQ_FMT_Q8_0 || f == GQ_FMT_Q4_K, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(ops && n_ops >= 1, GQ_ERR_INVALID_ARGS);
  const int ck = (int)gq_chunk_k(f);
  const int max_c = kMaxPieceK / ck;
  std::vector<int> last(n_ops, -1);  // device index of each caller op's final range
  int unit0 = 0, kx = 0, sl = 0, zl = 0;
  out.clear();
  GQ_TRY(check_hazards(ops, n_ops));
  for (int i = 0; i < n_ops; ++i) {
    const gq_chain_op &p = ops[i];
    GQ_CHECK(p.w && p.x && p.y && p.N > 0 && p.K > 0, GQ_ERR_INVALID_ARGS);
    // the kernel reads x with 8-byte and gamma with 16-byte vector loads
    GQ_CHECK((uintptr_t)p.x % 16 == 0 && (uintptr_t)p.gamma % 16 == 0, GQ_ERR_INVALID_ARGS);
    GQ_CHECK((uintptr_t)p.y % 4 == 0 && (uintptr_t)p.resid % 4 == 0, GQ_ERR_INVALID_ARGS);
    const size_t kt = p.k_total ? p.k_total : (size_t)p.K + p.k_offset;
    GQ_TRY(gq_check_shape(f, p.N, kt));
    GQ_CHECK(p.k_offset % (uint32_t)ck == 0 && p.K % 32 == 0 && p.k_offset + (size_t)p.K <= kt, GQ_ERR_INVALID_ARGS);
    GQ_CHECK(!(p.w_up && p.resid), GQ_ERR_INVALID_ARGS);
    GQ_CHECK(p.x_head_dim == 0 || (p.x_head_dim % 8 == 0 && p.x_group > 0), GQ_ERR_INVALID_ARGS);
    for (int q = 0; q < 3; ++q) GQ_CHECK(p.dep[q] < i && p.dep[q] >= -1, GQ_ERR_INVALID_ARGS);
    const int C = (int)((p.K + ck - 1) / ck);
    const int pieces = (C + max_c - 1) / max_c;
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
      d.pair = p.w_up ? 1 : 0;
      d.units = (int)gq_tiles(p.N);
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
      d.stage = out.empty() ? 0 : (same_input(out.back(), d) ? out.back().stage : out.back().stage + 1);
      const int kp = d.C * ck;
      kx = kp > kx ? kp : kx;
      const int slice = (d.C + kCW - 1) / kCW * ck;
      sl = slice > sl ? slice : sl;
      zl = ck;  // (the zero A rows: one chunk's 64-k steps)
      out.push_back(d);
    }
    last[i] = (int)out.size() - 1;
  }
  *lds = chain_lds_layout(kx, sl, zl);
  return GQ_OK;
}

size_t chain_ws_bytes(size_t n_dev_ops) {
  return 256 + al256(n_dev_ops * kMaxGrid * 4) /* completion flags */ + 256 /* error flag */ +
         al256(n_dev_ops * sizeof(ChainOpD));
}

template <int FMT>
int chain_launch(const ChainHdr &h, const uint8_t *ws, hipStream_t s) {
  hipLaunchKernelGGL(k_chain<FMT>, dim3((unsigned)h.grid), dim3(64 * (kCW + 1)), (size_t)h.lds.bytes, s,
                     (const ChainOpD *)(ws + h.ops_off), h.n_ops, h.total, (unsigned *)(ws + h.done_off),
                     (unsigned *)(ws + h.err_off), h.eps, h.spin_limit, h.lds);
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
  ChainLds lds;
  GQ_TRY(build_ops(fmt, ops, n_ops, d, &lds));
  // (x too long for the LDS copy; 8 KiB stay for the static arrays: partial
  // tiles, counters, held rows)
  GQ_CHECK(lds.bytes <= 160 * 1024 - 8192, GQ_ERR_UNSUPPORTED);
  *bytes = chain_ws_bytes(d.size());
  return GQ_OK;
}

extern "C" int gq_gemv_chain_plan(int fmt, const gq_chain_op *ops, int n_ops, float eps, void *ws, size_t ws_bytes) {
  GQ_CHECK(ws, GQ_ERR_INVALID_ARGS);
  std::vector<ChainOpD> d;
  ChainHdr h{};
  GQ_TRY(build_ops(fmt, ops, n_ops, d, &h.lds));
  GQ_CHECK(h.lds.bytes <= 160 * 1024 - 8192, GQ_ERR_UNSUPPORTED);
  GQ_CHECK(ws_bytes >= chain_ws_bytes(d.size()), GQ_ERR_WORKSPACE);
  h.fmt = chain_fmt(fmt);
  h.n_ops = (int)d.size();
  h.total = d.back().unit0 + d.back().units;
  h.eps = eps;
  int per_cu = 0;
  switch (h.fmt) {
  case GQ_FMT_Q4_0: GQ_TRY(chain_occupancy<GQ_FMT_Q4_0>(h.lds.bytes, &per_cu)); break;
  case GQ_FMT_Q8_0: GQ_TRY(chain_occupancy<GQ_FMT_Q8_0>(h.lds.bytes, &per_cu)); break;
  default: GQ_TRY(chain_occupancy<GQ_FMT_Q4_K>(h.lds.bytes, &per_cu)); break;
  }
  const int cus = gq_device_cus();
  GQ_CHECK(per_cu >= 1 && cus > 0, GQ_ERR_UNSUPPORTED);
  h.grid = cus < kMaxGrid ? cus : kMaxGrid;  // one workgroup per CU: every workgroup resident at once
  const char *e = getenv("GQ_CHAIN_SPIN");
  h.spin_limit = e ? (unsigned)strtoul(e, nullptr, 0) : (1u << 22);
  h.done_off = 256;
  h.err_off = h.done_off + al256(d.size() * kMaxGrid * 4);
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
