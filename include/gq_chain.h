/*
 * gq_chain.h -- a decode step's GEMVs as one persistent launch (libgq.so).
 *
 * No counterpart in the reference: the reference launches every projection
 * of a decode step separately (src/inference/src/block_scheduler.cpp:
 * 1831-1894, 2769-2775, 2967-3003, through GretaCompute::gemm).  A chain
 * runs an ordered list of batch-1 GEMV "ops" of one GGUF-native format in
 * one launch; each op names the earlier ops whose outputs it reads, and its
 * weights stream while those are still being computed.
 *
 * Op semantics (K values of x, N of y, W the op's T16 tensor, N x K):
 *   t   = x, or x read through a GQA map: t[k] = x[(k / (hd * grp)) * hd + k % hd]
 *         (x_head_dim = hd, x_group = grp; 0, 0: no map)
 *   t   = t * gamma / sqrt(sum(t^2) / K + eps)     if gamma != NULL (RMSNorm)
 *   y   = W t (+ resid)                            or, with w_up != NULL,
 *   y   = silu(W t) * (W_up t),  silu(g) = g / (1 + e^-g)
 * K may be a column range of a wider tensor: k_offset (a multiple of the
 * format's 128- or 256-element chunk) and k_total (the tensor's K) select
 * columns [k_offset, k_offset + K) of an N x k_total tensor; x then holds
 * those K values.  The library splits ops whose K exceeds its per-launch
 * limit into such ranges itself (chained through resid).
 *
 * Ordering: inside the one launch an op runs after the ops it depends on
 * (transitively) and is unordered with every other op.  So an op whose y
 * overlaps a buffer that an earlier op reads (x, gamma, resid) or writes (y)
 * must depend on that op, directly or through other ops; the plan refuses
 * such a pair otherwise (GQ_ERR_INVALID_ARGS), as it refuses a y that
 * aliases the op's own inputs.  Alignment: x and gamma 16 bytes (vector
 * loads), resid and y 4 bytes.
 */
#ifndef GQ_CHAIN_H
#define GQ_CHAIN_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gq_chain_op {
  const void *w;      /* T16 weights (the chain's format) */
  const void *w_up;   /* SwiGLU: the up matrix (same shape), else NULL */
  const float *x;     /* input (K values; with a GQA map, hd * (K / (hd * grp)) values) */
  const float *gamma; /* RMSNorm weight (K values) or NULL */
  const float *resid; /* added to y (N values) or NULL; not with w_up */
  float *y;           /* output, N values (must not alias x, gamma or resid of this op) */
  uint32_t N, K;
  uint32_t k_offset, k_total; /* column range of a wider tensor (0, 0: the whole K) */
  uint32_t x_head_dim, x_group;
  int32_t dep[3]; /* earlier ops (indices) whose y this op reads, -1: none */
} gq_chain_op;

/* Device workspace bytes of a plan for these ops. */
int gq_gemv_chain_workspace_bytes(int fmt, const gq_chain_op *ops, int n_ops, size_t *bytes);
/* Builds a plan in d_workspace: checks the ops (format Q4_0 / Q8_0 / Q4_K /
 * Q4_K_GGML, shapes, dependencies pointing backwards), cuts them into units
 * and uploads the op table (synchronous).  The plan stays valid while the
 * ops' buffers do; run it any number of times. */
int gq_gemv_chain_plan(int fmt, const gq_chain_op *ops, int n_ops, float eps, void *d_workspace,
                       size_t workspace_bytes);
/* Runs a plan on `stream`: resets its counters with a fill kernel, then one
 * persistent launch (no memset, no allocation: capturable into a HIP graph).
 * Concurrent runs of one plan race. */
int gq_gemv_chain_run(const void *d_workspace, void *stream);
/* After a run has completed: 0 if every dependency wait ended normally, 1 if
 * one gave up after its bounded spin (the outputs are then undefined).
 * Synchronous (reads one word). */
int gq_gemv_chain_error(const void *d_workspace, int *error);

#ifdef __cplusplus
}
#endif
#endif
