// ref_harness.cpp -- exposes the reference's own CPU functions for this path
// through a C ABI so tests can pin the oracle against them.
//
// TEST INFRASTRUCTURE ONLY.  This translation unit compiles the reference's
// source files where they lie under the reference tree (REF_ROOT, passed by
// oracle/Makefile); no reference source is copied into this repository.  The
// functions exposed are file-static in the reference, which is why the .cpp is
// included rather than linked.
#include REF_WEIGHT_LOADER_CPP
#include "gcore/rt/ref/cpu_reference.hpp"

#include <cstring>
#include <fstream>

extern "C" {

// weight_loader.cpp:91-110
float gqref_fp16_to_fp32(uint16_t h) { return gcore::inference::fp16_to_fp32(h); }
// weight_loader.cpp:112-123
uint16_t gqref_fp32_to_fp16(float f) { return gcore::inference::fp32_to_fp16(f); }
// weight_loader.cpp:125-156
void gqref_dequant_q4_k(const uint8_t *blocks, size_t n_blocks, float *out) {
  for (size_t b = 0; b < n_blocks; ++b)
    gcore::inference::dequantize_q4_k_block(blocks + b * 144, out + b * 256, 256);
}
// weight_loader.cpp:158-177
void gqref_dequant_q6_k(const uint8_t *blocks, size_t n_blocks, float *out) {
  for (size_t b = 0; b < n_blocks; ++b)
    gcore::inference::dequantize_q6_k_block(blocks + b * 210, out + b * 256, 256);
}
// cpu_reference.hpp:19-38, 40-51, 56-66
uint16_t gqref_float_to_half(float f) { return gcore::rt::ref::CpuReference::float_to_half(f); }
float gqref_half_to_float(uint16_t h) { return gcore::rt::ref::CpuReference::half_to_float(h); }
void gqref_gemm(const float *A, const float *B, float *C, int M, int N, int K) {
  gcore::rt::ref::CpuReference::gemm(A, B, C, M, N, K);
}

// GGUFLoader::open / list_tensors / get_config (weight_loader.cpp:467-519):
// parse a GGUF file and report the tensor table and the llama.* config, so the
// build's own parser can be compared with the reference's on the same files.
// Returns the tensor count (or -1) and writes up to `cap` entries.
struct gqref_tensor {
  char name[128];
  char dtype[16];
  uint64_t shape[4];
  uint32_t n_dims;
  uint64_t offset;
  uint64_t size_bytes;
};
struct gqref_config {
  uint32_t dim, num_heads, num_heads_kv, num_layers, vocab_size, hidden_dim,
      head_dim, max_seq_len;
  float rope_base, rms_eps;
};
int gqref_gguf_parse(const char *path, gqref_tensor *out, int cap,
                     gqref_config *cfg, char *err, int err_cap) {
  gcore::inference::GGUFLoader l;
  std::string e;
  if (!l.open(path, &e)) {
    if (err && err_cap > 0) {
      std::strncpy(err, e.c_str(), err_cap - 1);
      err[err_cap - 1] = 0;
    }
    return -1;
  }
  auto ts = l.list_tensors();
  for (int i = 0; i < (int)ts.size() && i < cap; ++i) {
    std::memset(&out[i], 0, sizeof(out[i]));
    std::strncpy(out[i].name, ts[i].name.c_str(), sizeof(out[i].name) - 1);
    std::strncpy(out[i].dtype, ts[i].dtype.c_str(), sizeof(out[i].dtype) - 1);
    out[i].n_dims = (uint32_t)ts[i].shape.size();
    for (size_t d = 0; d < ts[i].shape.size() && d < 4; ++d)
      out[i].shape[d] = ts[i].shape[d];
    out[i].offset = ts[i].offset;
    out[i].size_bytes = ts[i].size_bytes;
  }
  if (cfg) {
    auto c = l.get_config();
    cfg->dim = c.dim; cfg->num_heads = c.num_heads; cfg->num_heads_kv = c.num_heads_kv;
    cfg->num_layers = c.num_layers; cfg->vocab_size = c.vocab_size;
    cfg->hidden_dim = c.hidden_dim; cfg->head_dim = c.head_dim;
    cfg->max_seq_len = c.max_seq_len; cfg->rope_base = c.rope_base; cfg->rms_eps = c.rms_eps;
  }
  return (int)ts.size();
}

// GGUFLoader::load_tensor / _fp16 / _int8 / _int4 (weight_loader.cpp:517-1008),
// the reference's own loader run end to end (it allocates device Buffers, so
// this needs a GPU).  kind: 0 fp32, 1 fp16, 2 int8, 3 int4.  Device results
// are copied back into the host arrays (capacities in bytes); the sizes are
// returned.  Returns 0 on success, -1 on failure.
int gqref_gguf_load(const char *path, const char *name, int kind, void *out, uint64_t out_cap,
                    uint64_t *out_bytes, float *scales, uint64_t scales_cap, uint64_t *scales_bytes,
                    float *head_scales, uint64_t head_cap, uint64_t *head_count, char *err, int err_cap) {
  gcore::inference::GGUFLoader l;
  std::string e;
  auto fail = [&]() {
    if (err && err_cap > 0) {
      std::strncpy(err, e.c_str(), err_cap - 1);
      err[err_cap - 1] = 0;
    }
    return -1;
  };
  if (!l.open(path, &e)) return fail();
  gcore::rt::hip::Buffer b, s, h;
  bool ok = false;
  if (kind == 0) ok = l.load_tensor(name, b, &e);
  else if (kind == 1) ok = l.load_tensor_fp16(name, b, &e);
  else if (kind == 2) ok = l.load_tensor_int8(name, b, s, &e);
  else if (kind == 3) ok = l.load_tensor_int4(name, b, s, h, &e);
  if (!ok) return fail();
  *out_bytes = b.size();
  if (b.size() > out_cap || !b.copy_to_host(out, b.size(), &e)) return fail();
  *scales_bytes = 0;
  *head_count = 0;
  if (kind >= 2) {
    *scales_bytes = s.size();
    if (s.size() > scales_cap || !s.copy_to_host(scales, s.size(), &e)) return fail();
  }
  if (kind == 3 && h.size() > 0) {
    *head_count = h.size() / 4;
    if (h.size() > head_cap || !h.copy_to_host(head_scales, h.size(), &e)) return fail();
  }
  return 0;
}
}
