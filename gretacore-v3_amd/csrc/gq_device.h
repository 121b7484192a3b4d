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

// 4-bit codes straight to fp16: OR-ing a code into the low mantissa bits of
// 1024.0 (0x6400) gives 1024 + q.  Of a code-group word (slots 0..3 in the
// low nibbles of bytes 0..3, slots 4..7 in the high nibbles) four and-or ops
// give the halves (s0, s2), (s4, s6) * 16, (s1, s3), (s5, s7) * 16 -- the high
// nibbles come out as 1024 + 16 q.  Formats that use this order stage their
// activations in the same order, with the "* 16" positions divided by 16
// (exact), so each product is unchanged: element e of a run of 8 holds slot
// {0, 2, 4, 6, 1, 3, 5, 7}[e], elements 2, 3, 6, 7 scaled by 16.
// The magic is held in a VGPR (mg): a VOP3 and-or can then take the mask as its
// one scalar operand and stays a single instruction.
GQ_DEV uint32_t gq_nib_magic() {
  uint32_t v;
  asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(v));
  return v;
}
GQ_DEV void gq_nib_halves(uint32_t w, uint32_t mg, gq_half2 (&p)[4]) {
  const uint32_t v = w >> 8;
  p[0] = gq_bits_h2((w & 0x000F000Fu) | mg);
  p[1] = gq_bits_h2((w & 0x00F000F0u) | mg);
  p[2] = gq_bits_h2((v & 0x000F000Fu) | mg);
  p[3] = gq_bits_h2((v & 0x00F000F0u) | mg);
}

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
