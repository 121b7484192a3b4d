/*
 * gq_gguf.h -- C ABI of the GGUF weight loader in libgq.so.
 *
 * Reference interfaces replaced (paths relative to leaatimberini/gretacore-v3):
 *   - src/inference/include/gcore/inference/weight_loader.hpp:24-86 and
 *     src/inference/src/weight_loader.cpp:218-504 (GGUFLoader::open,
 *     list_tensors, get_config)  -> gq_gguf_open / gq_gguf_tensor_info /
 *     gq_gguf_get_config / gq_gguf_vocab_token
 *   - weight_loader.cpp:517-1008 (load_tensor, load_tensor_fp16,
 *     load_tensor_int8, load_tensor_int4) -> gq_gguf_load (kinds F32, F16,
 *     INT8, INT4) into caller-owned device memory
 *   - the GGUF-native upload that the reference lacks -> gq_gguf_load with
 *     kind QUANT (raw Q4_0 / Q8_0 / Q4_K blocks repacked on the GPU to T16).
 * The C++ classes (gcore::inference::GGUFLoader) wrap the same code.
 *
 * Loads are synchronous (the reference copies with hipMemcpy): on return the
 * destination holds the converted tensor.  A handle may be used by one thread
 * at a time.
 */
#ifndef GQ_GGUF_H
#define GQ_GGUF_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gq_gguf gq_gguf; /* opaque */

typedef struct {
  char name[256];    /* NUL-terminated (names are at most 512 bytes in GGUF;
                        longer ones are truncated here) */
  char dtype[16];    /* "F32", "F16", "Q4_0", "Q8_0", "Q4_K", "Q6_K", "UNKNOWN" */
  uint32_t ggml_type;
  uint32_t n_dims;
  uint64_t shape[8]; /* shape[0] = ne0, the contiguous dimension */
  uint64_t offset;   /* absolute file offset of the data */
  uint64_t size_bytes;
} gq_gguf_tensor;

typedef struct {
  uint32_t dim, num_heads, num_heads_kv, num_layers, vocab_size, hidden_dim, head_dim, max_seq_len;
  float rope_base, rms_eps;
} gq_gguf_config;

/* load kinds */
#define GQ_LOAD_F32 0   /* load_tensor: fp32 [n] */
#define GQ_LOAD_F16 1   /* load_tensor_fp16: fp16 [n] (+ GQA K/V transpose) */
#define GQ_LOAD_INT8 2  /* load_tensor_int8: int8 [n] + fp32 scales [ceil(n/32)] */
#define GQ_LOAD_INT4 3  /* load_tensor_int4: packed [ceil(n/2)] + scales + head scales */
#define GQ_LOAD_QUANT 4 /* load_tensor_quant: T16 bytes of gq_packed_size */

typedef struct {
  uint64_t n_elem;
  uint64_t bytes;        /* main destination */
  uint64_t scale_bytes;  /* INT8 / INT4 */
  uint32_t num_heads;    /* INT4: head scale count when has_head_scales */
  int32_t has_head_scales;
  int32_t is_qkv;
  int32_t transpose;     /* GQA K/V transpose applied */
  int32_t fmt;           /* QUANT: GQ_FMT_* of the T16 data */
  uint64_t N, K;         /* QUANT: rows, row length */
} gq_gguf_plan;

/* Opens and parses a GGUF file (memory-mapped).  On failure *out is NULL and
 * the status is GQ_ERR_INVALID_ARGS; gq_gguf_open_error() has the message. */
int gq_gguf_open(const char *path, gq_gguf **out);
const char *gq_gguf_open_error(void); /* message of this thread's last failed open */
void gq_gguf_close(gq_gguf *g);
/* Message of the last failed call on this handle ("" if none). */
const char *gq_gguf_error(const gq_gguf *g);

size_t gq_gguf_tensor_count(const gq_gguf *g);
int gq_gguf_tensor_info(const gq_gguf *g, size_t index, gq_gguf_tensor *out);
/* Index of a tensor by name; GQ_ERR_INVALID_ARGS if absent. */
int gq_gguf_find(const gq_gguf *g, const char *name, size_t *index);
int gq_gguf_get_config(const gq_gguf *g, gq_gguf_config *out);
/* Vocabulary entry i (tokenizer.ggml.tokens); the pointer lives as long as g. */
int gq_gguf_vocab_token(const gq_gguf *g, size_t i, const char **s, size_t *len);
/* Q4_K code layout: 0 = reference (default), 1 = llama.cpp. */
int gq_gguf_set_q4k_layout(gq_gguf *g, int ggml);
/* Copies a tensor's stored bytes to host memory (capacity >= size_bytes). */
int gq_gguf_read_raw(const gq_gguf *g, const char *name, void *dst, size_t capacity);

/* Sizes of a load of `kind`, and the checks it will make (type, GQA shape,
 * head-scale range). */
int gq_gguf_plan_load(const gq_gguf *g, const char *name, int kind, gq_gguf_plan *plan);
/* Loads into caller-owned device memory of at least the planned sizes:
 * d_out (plan.bytes), d_scales (plan.scale_bytes, INT8/INT4 else NULL),
 * d_head_scales (plan.num_heads floats when plan.has_head_scales, else NULL). */
int gq_gguf_load(const gq_gguf *g, const char *name, int kind, void *d_out, size_t out_bytes, void *d_scales,
                 size_t scale_bytes, void *d_head_scales, size_t head_scale_bytes);

/* GQ_LOAD_QUANT of n tensors in one pass: no counterpart in the reference
 * (whose loader, and gq_gguf_load, take one tensor per call and return when
 * it is on the device).  Here the pinned staging ring stays full across the
 * tensors, so a layer's many small tensors load at the large-tensor rate.
 * d_outs[i] holds out_bytes[i] >= the planned bytes of names[i].  Every name
 * is planned and checked before any data moves (GQ_ERR_INVALID_ARGS, nothing
 * loaded); returns when all tensors are on the device.  A transfer error
 * (GQ_ERR_HIP) may leave the tensors before the failing one loaded. */
int gq_gguf_load_quant_many(const gq_gguf *g, size_t n, const char *const *names, void *const *d_outs,
                            const size_t *out_bytes);

#ifdef __cplusplus
}
#endif
#endif
