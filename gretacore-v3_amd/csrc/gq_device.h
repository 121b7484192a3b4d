// gq_device.h -- device helpers for CDNA4 (gfx950): fp16 decoding with the
// reference's semantics, nibble/byte -> fp16 operand construction and MFMA
// wrappers.  Wave64 throughout.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gq_layout.h"

typedef _Float16 gq_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 gq_half2 __attribute__((ext_vector_type(2)));
typedef float gq_f4 __attribute__((ext_vector_type(4)));
typedef float gq_f16v __attribute__((ext_vector_type(16)));
typedef int gq_i4 __attribute__((ext_vector_type(4)));
typedef int gq_i16v __attribute__((ext_vector_type(16)));
typedef uint32_t gq_u4 __attribute__((ext_vector_type(4)));
typedef uint32_t gq_u2 __attribute__((ext_vector_type(2)));

#define GQ_DEV static __device__ __forceinline__

// fp16 -> fp32 with the reference's semantics (weight_loader.cpp:91-110):
// finite values and infinities convert exactly (the hardware conversion keeps
// fp16 subnormals), every exponent-31 input becomes +-Inf (NaN payloads are
// dropped exactly as the reference does).
GQ_DEV float gq_h2f(uint32_t h16) {
  h16 &= 0xFFFFu;
  if ((h16 & 0x7C00u) == 0x7C00u)
    return __uint_as_float(((h16 & 0x8000u) << 16) | 0x7F800000u);
  _Float16 hv = __builtin_bit_cast(_Float16, (uint16_t)h16);
  return (float)hv;
}
// Same, for a scale that only feeds a GEMV/GEMM: the NaN->Inf rule is kept so
// results match the reference semantics on every input.
GQ_DEV float gq_scale_h2f(uint32_t h16) { return gq_h2f(h16); }

GQ_DEV uint32_t gq_h2_bits(gq_half2 v) { return __builtin_bit_cast(uint32_t, v); }
GQ_DEV gq_half2 gq_bits_h2(uint32_t v) { return __builtin_bit_cast(gq_half2, v); }

GQ_DEV gq_f4 gq_mfma16(const gq_half8 &a, const gq_half8 &b, const gq_f4 &c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
GQ_DEV gq_f16v gq_mfma32(const gq_half8 &a, const gq_half8 &b, const gq_f16v &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

GQ_DEV gq_u4 gq_ld16(const void *p) { return *reinterpret_cast<const gq_u4 *>(p); }
// Streaming loads for data read exactly once (weights): non-temporal, so they
// do not evict reusable lines from L2 / the Infinity Cache.
// Streaming loads of device memory.  The pointer is cast to the global
// address space: a pointer the compiler cannot trace to a kernel argument
// (one read from a table in memory) would otherwise become a flat access,
// which also counts against the LDS counter and defeats load pipelining.
#define GQ_GLOBAL __attribute__((address_space(1)))
GQ_DEV gq_u4 gq_ld16_nt(const void *p) {
  return __builtin_nontemporal_load((const GQ_GLOBAL gq_u4 *)p);
}
GQ_DEV uint32_t gq_ld4_nt(const void *p) {
  return __builtin_nontemporal_load((const GQ_GLOBAL uint32_t *)p);
}
GQ_DEV gq_u2 gq_ld8(const void *p) { return *reinterpret_cast<const gq_u2 *>(p); }
