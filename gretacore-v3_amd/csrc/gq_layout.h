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
// multiple of 16 with all-zero rows).  Within a tile, lane l = 16*g + r of a
// wavefront owns row r and "word slot" g (g = 0..3).  The K axis is cut into
// chunks; every chunk of a row tile is one contiguous 1 KiB (or 2 KiB) record so
// that one dwordx4 load per lane streams it with perfect coalescing.
//
//  canonical word: a 32-bit word that holds 8 consecutive elements e0..e7 of a
//  32-element (sub-)block, element i at nibble position (i>>1) | ((i&1)<<2).
//  Then ((w >> 4s) & 0x000F000F) holds elements (2s, 2s+1) in its two 16-bit
//  halves, which turns into an fp16 pair with one OR and one packed subtract.
//
//  Q4_0: chunk = 4 blocks (128 k).  C = ceil(K/128) chunks per row.
//    qs plane   [tile][C][64 lanes][4 words] : lane l word j = canonical word g of
//               block 4c+j of row r                                 1024 B/chunk
//    d plane    [tile][C][16 rows][4] fp16                           128 B/chunk
//  Q8_0: chunk = 4 blocks (128 k).
//    qs plane   [tile][C][2 parts][64 lanes][16 B] : part p lane l = bytes
//               8g..8g+7 of block 4c+2p then of block 4c+2p+1 of row r
//                                                                   2048 B/chunk
//    d plane    as Q4_0                                              128 B/chunk
//  Q4_K: chunk = 1 super-block (256 k).  S = K/256 chunks per row.
//    qs plane   [tile][S][2 halves][64 lanes][16 B] : half h lane l = the 4
//               canonical words of sub-block 2g+h of row r           2048 B/chunk
//    meta plane [tile][S][16 rows][16 B] : d, dmin (fp16) | W1 | W2 | W3 with
//               byte g of W1 = sc[2g]   | (m[2g]   & 3) << 6
//               byte g of W2 = sc[2g+1] | (m[2g+1] & 3) << 6
//               byte g of W3 = (m[2g] >> 2) | (m[2g+1] >> 2) << 4    256 B/chunk
// Padding blocks (K not a multiple of 128 for Q4_0/Q8_0) carry d = 0 and zero
// weights, so they add exact zeros.  Bytes per weight are unchanged by the
// repack: 0.5625 (Q4_0, Q4_K) and 1.0625 (Q8_0).
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

// Format ids: the GGML type ids (weight_loader.cpp:15-33), plus one id for the
// llama.cpp canonical Q4_K layout.
#define GQ_FMT_Q4_0 2
#define GQ_FMT_Q8_0 8
#define GQ_FMT_Q4_K 12
#define GQ_FMT_Q4_K_GGML 112

GQ_LHD int gq_fmt_valid(int fmt) {
  return fmt == GQ_FMT_Q4_0 || fmt == GQ_FMT_Q8_0 || fmt == GQ_FMT_Q4_K ||
         fmt == GQ_FMT_Q4_K_GGML;
}
GQ_LHD int gq_fmt_is_q4k(int fmt) {
  return fmt == GQ_FMT_Q4_K || fmt == GQ_FMT_Q4_K_GGML;
}
GQ_LHD size_t gq_block_elems(int fmt) { return gq_fmt_is_q4k(fmt) ? 256 : 32; }
GQ_LHD size_t gq_block_bytes(int fmt) {
  return fmt == GQ_FMT_Q4_0 ? 18 : fmt == GQ_FMT_Q8_0 ? 34 : 144;
}
// k elements per T16 chunk
GQ_LHD size_t gq_chunk_k(int fmt) { return gq_fmt_is_q4k(fmt) ? 256 : 128; }
// bytes of the qs plane and of the scale plane per (tile, chunk)
GQ_LHD size_t gq_chunk_qs_bytes(int fmt) { return fmt == GQ_FMT_Q4_0 ? 1024 : 2048; }
GQ_LHD size_t gq_chunk_sc_bytes(int fmt) { return gq_fmt_is_q4k(fmt) ? 256 : 128; }

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
// nibble position of element i (0..7) inside a canonical word
GQ_LHD int gq_canon_pos(int i) { return (i >> 1) | ((i & 1) << 2); }

#endif
