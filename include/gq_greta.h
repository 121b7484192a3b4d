/*
 * gq_greta.h -- C ABI of the .greta weight-file writer and reader in libgq.so.
 *
 * Reference interfaces replaced (paths relative to leaatimberini/gretacore-v3):
 *   - tools/quantize/greta_quantize_gguf.cpp:17-124 (main: GGUF -> .greta of
 *     load_tensor_int4 records) -> gq_greta_write(kind GQ_LOAD_INT4), the same
 *     container and records.
 *   - the reader the reference lacks, and a cache of the T16 tiled layout:
 *     gq_greta_write(kind GQ_LOAD_QUANT) stores every Q4_0 / Q8_0 / Q4_K /
 *     Q6_K tensor already repacked (no GPU needed to write it), and
 *     gq_greta_load uploads a record with no conversion.
 *
 * Container (little-endian): "GRETA_W\0", u32 json_len, json, u32 n_tensors,
 * then per tensor: u32 name_len, name, u32 dtype (GretaDataType), u32 rank,
 * u64 dims[rank], u32 group_size, u32 num_heads, u64 w_size, u64 s_size,
 * u64 h_size, and the three arrays.
 */
#ifndef GQ_GRETA_H
#define GQ_GRETA_H
#include <stddef.h>
#include <stdint.h>

#include "gq_gguf.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gq_greta gq_greta; /* opaque */

/* record dtypes (GretaDataType values) */
#define GQ_GRETA_INT4 4
#define GQ_GRETA_Q4_K 5
#define GQ_GRETA_Q4_0 8
#define GQ_GRETA_Q8_0 9
#define GQ_GRETA_Q4_K_GGML 10
#define GQ_GRETA_Q6_K 11
#define GQ_GRETA_Q6_K_GGML 12

typedef struct {
  char name[256];      /* NUL-terminated (truncated if longer) */
  uint32_t dtype;      /* GQ_GRETA_* */
  uint32_t n_dims;
  uint64_t shape[8];   /* GGUF order: shape[0] contiguous */
  uint32_t group_size, num_heads;
  uint64_t w_bytes, s_bytes, h_bytes;
  int32_t fmt;         /* T16 records: GQ_FMT_* of the tiles; INT4: -1 */
  uint64_t N, K;       /* T16 records: rows, row length */
} gq_greta_tensor;

/* Writes a .greta file from an open GGUF.  kind GQ_LOAD_QUANT: T16 records
 * (host repack, no GPU); kind GQ_LOAD_INT4: the reference tool's INT4 records
 * (converted on the GPU).  Tensors that cannot be converted are skipped;
 * *written (may be NULL) receives the record count.  Errors: gq_gguf_error(g). */
int gq_greta_write(gq_gguf *g, const char *path, int kind, size_t *written);

/* Opens a .greta file (memory-mapped, lengths bounds-checked; T16 records of
 * another layout version are refused).  On failure *out is NULL and
 * gq_greta_open_error() has the message. */
int gq_greta_open(const char *path, gq_greta **out);
const char *gq_greta_open_error(void);
void gq_greta_close(gq_greta *h);
const char *gq_greta_error(const gq_greta *h);
size_t gq_greta_tensor_count(const gq_greta *h);
int gq_greta_tensor_info(const gq_greta *h, size_t index, gq_greta_tensor *out);
int gq_greta_find(const gq_greta *h, const char *name, size_t *index);
/* Config from the file's json (T16 files); the reference defaults otherwise. */
int gq_greta_get_config(const gq_greta *h, gq_gguf_config *out);
/* Uploads a record into caller-owned device memory: d_w (w_bytes), d_s
 * (s_bytes, NULL when 0), d_h (h_bytes, NULL when 0).  Synchronous. */
int gq_greta_load(const gq_greta *h, const char *name, void *d_w, size_t w_cap, void *d_s, size_t s_cap, void *d_h,
                  size_t h_cap);

#ifdef __cplusplus
}
#endif
#endif
