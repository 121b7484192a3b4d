// gq_layout.h -- the GGUF block formats handled by this library and the
// wavefront-tiled ("T16") layout they are repacked into at load time.
// Shared by host and device code.
//
// GGUF formats (row-major W[N][K], ne0 = K contiguous), as the reference's
// loader sizes them (src/inference/src/weight_loader.cpp:38-82):
//   Q4_0  32 weights / 18 B : fp16 d | 16 B nibbles (byte j: elem j low, j+16 high)
//   Q8_0  32 weights / 34 B : fp16 d | 32 x int8
//   Q4_K 256 weights / 144 B: fp16 d | fp16 dmin | 12 B 6-bit codes | 128 B nibbles
//
// T16 layout.  Rows are grouped into row tiles of 16 (N is padded up to a
// multiple of 16 with all-zero rows).  The K axis is cut into chunks; every
// chunk of a row tile is one contiguous 1 KiB (or 2 KiB) record, so one
// dwordx4 load per lane streams it with perfect coalescing.  Within a chunk,
// lane l = 16*g + r of a wavefront owns row r; for each int8-MFMA step m
// (64 k) it holds the 16 elements 16*(g&1) .. +15 of 32-element (sub-)block
// 2m + (g>>1) -- the lane's share of a v_mfma_i32_16x16x64_i8 B operand.
//
//  code group: 16 four-bit codes in 8 bytes, byte b = slot 8(b>>2)+(b&3) in the
//  low nibble and slot 8(b>>2)+(b&3)+4 in the high nibble, so that one AND
//  (and one shift) per word yields 4 codes as bytes in slot order.
//
//  Q4_0: chunk = 4 blocks (128 k, two MFMA steps).  C = ceil(K/128).
//    qs plane  [tile][C][64 lanes][2 steps][8 B code group]      1024 B/chunk
//    d plane   [tile][C][16 rows][d0 d2 d1 d3] fp16               128 B/chunk
//  Q8_0: chunk = 4 blocks (128 k).
//    qs plane  [tile][C][2 steps][64 lanes][16 x int8]            2048 B/chunk
//    d plane   as Q4_0                                            128 B/chunk
//  Q4_K: chunk = 1 super-block (256 k, four MFMA steps).  S = K/256.
//    qs plane  [tile][S][2 step pairs][64 lanes][2 steps][8 B]    2048 B/chunk
//    meta plane [tile][S][16 rows][16 B]: d, dmin (fp16) | W1 | W2 | W3 with
//              byte i of W1 = sc[2i]   | (m[2i]   & 3) << 6
//              byte i of W2 = sc[2i+1] | (m[2i+1] & 3) << 6
//              byte i of W3 = (m[2i] >> 2) | (m[2i+1] >> 2) << 4   256 B/chunk
//  Q6_K: chunk = 1 super-block (256 k).  Codes c = low 4 bits | high 2 bits << 4.
//    qs plane  [tile][S] 3072 B: the low nibbles as Q4_K code groups (2048 B),
//              then per lane and MFMA step the 16 high 2-bit fields in one word
//              [64 lanes][4 steps][4 B]: byte b holds, at bits 2q..2q+1, the
//              high bits of slot 4q + b (the slot whose low nibble the Q4 code
//              group extraction puts in byte b of word q)
//    scale plane [tile][S] 288 B: [16 rows][16 x int8 scale] then [16 rows][fp16 d]
// Padding blocks (K not a multiple of 128 for Q4_0/Q8_0) carry d = 0 and zero
// codes, so they add exact zeros.  Bytes per weight are unchanged by the
// repack: 0.5625 (Q4_0, Q4_K), 1.0625 (Q8_0) and 0.8203 (Q6_K).
#ifndef GQ_LAYOUT_H
#define GQ_LAYOUT_H
#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define GQ_LHD __host__ __device__ static inline
#else
#define GQ_LHD static inline
#endif

#define GQ_TILE_ROWS 16

// Format ids: the GGML type ids (weight_loader.cpp:15-33), plus one id each for
// the llama.cpp canonical Q4_K and Q6_K layouts.
#define GQ_FMT_Q4_0 2
#define GQ_FMT_Q8_0 8
#define GQ_FMT_Q4_K 12
#define GQ_FMT_Q6_K 14
#define GQ_FMT_Q4_K_GGML 112
#define GQ_FMT_Q6_K_GGML 114

GQ_LHD int gq_fmt_is_q4k(int fmt) {
  return fmt == GQ_FMT_Q4_K || fmt == GQ_FMT_Q4_K_GGML;
}
GQ_LHD int gq_fmt_is_q6k(int fmt) {
  return fmt == GQ_FMT_Q6_K || fmt == GQ_FMT_Q6_K_GGML;
}
// formats with a T16 layout (repack, dequant of packed data, GEMV)
GQ_LHD int gq_fmt_valid(int fmt) {
  return fmt == GQ_FMT_Q4_0 || fmt == GQ_FMT_Q8_0 || gq_fmt_is_q4k(fmt) || gq_fmt_is_q6k(fmt);
}
GQ_LHD size_t gq_block_elems(int fmt) { return (gq_fmt_is_q4k(fmt) || gq_fmt_is_q6k(fmt)) ? 256 : 32; }
GQ_LHD size_t gq_block_bytes(int fmt) {
  return fmt == GQ_FMT_Q4_0 ? 18 : fmt == GQ_FMT_Q8_0 ? 34 : gq_fmt_is_q6k(fmt) ? 210 : 144;
}
// k elements per T16 chunk
GQ_LHD size_t gq_chunk_k(int fmt) { return (gq_fmt_is_q4k(fmt) || gq_fmt_is_q6k(fmt)) ? 256 : 128; }
// bytes of the qs plane and of the scale plane per (tile, chunk)
GQ_LHD size_t gq_chunk_qs_bytes(int fmt) {
  return fmt == GQ_FMT_Q4_0 ? 1024 : gq_fmt_is_q6k(fmt) ? 3072 : 2048;
}
GQ_LHD size_t gq_chunk_sc_bytes(int fmt) {
  return gq_fmt_is_q4k(fmt) ? 256 : gq_fmt_is_q6k(fmt) ? 288 : 128;
}

GQ_LHD size_t gq_tiles(size_t N) { return (N + GQ_TILE_ROWS - 1) / GQ_TILE_ROWS; }
GQ_LHD size_t gq_chunks(int fmt, size_t K) {
  size_t ck = gq_chunk_k(fmt);
  return (K + ck - 1) / ck;
}
// offset of the scale plane within a repacked tensor
GQ_LHD size_t gq_sc_plane_offset(int fmt, size_t N, size_t K) {
  return gq_tiles(N) * gq_chunks(fmt, K) * gq_chunk_qs_bytes(fmt);
}
GQ_LHD size_t gq_packed_bytes(int fmt, size_t N, size_t K) {
  return gq_tiles(N) * gq_chunks(fmt, K) *
         (gq_chunk_qs_bytes(fmt) + gq_chunk_sc_bytes(fmt));
}
GQ_LHD size_t gq_layout_gguf_bytes(int fmt, size_t N, size_t K) {
  return N * (K / gq_block_elems(fmt)) * gq_block_bytes(fmt);
}

#endif
