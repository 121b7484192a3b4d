/* gq_probe.h -- calibration kernels of lib/libgqcalib.so (not part of the
 * product boundary; the benchmark times them beside the decode GEMV to state
 * its read ceiling).
 *
 * gq_probe_read: wgs workgroups of waves_per_wg waves stream `bytes` (a
 * multiple of 16) of src as the decode GEMV streams its weights (each wave a
 * contiguous share of whole KiB, at most 16 KiB, all loads issued up front);
 * out (wgs * waves_per_wg words) is never written in practice, it keeps the
 * loads live.  gq_probe_empty: the same grid doing nothing.  All return 0 or
 * a GQ_ERR_* status. */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int gq_probe_read(const void *d_src, size_t bytes, int wgs, int waves_per_wg, uint32_t *d_out, void *stream);
int gq_probe_empty(int wgs, int waves_per_wg, void *stream);
/* Effective shader clock under matrix-core load: wgs workgroups of 4 waves
 * run `iters` x 4 dependent-chain MFMAs on changing operands; d_out[0..3]
 * receives the shader-clock counter (s_memtime) and the 100 MHz counter
 * (s_memrealtime) before and after workgroup 0's loop (d_out holds 5 words). */
int gq_probe_clock(unsigned long long *d_out, int wgs, int iters, void *stream);

#ifdef __cplusplus
}
#endif
