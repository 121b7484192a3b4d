// C ABI over gcore::inference::GGUFLoader (declared in gq_gguf.h).
#include <cstring>
#include <string>
#include <vector>

#include "gcore/inference/greta_file.hpp"
#include "gcore/inference/weight_loader.hpp"
#include "gq.h"
#include "gq_gguf.h"
#include "gq_greta.h"

using gcore::inference::GGUFLoader;
using gcore::inference::GretaLoader;

struct gq_gguf {
  GGUFLoader loader;
  std::vector<gcore::inference::TensorInfo> tensors;
  std::vector<uint32_t> types;
  gcore::inference::ModelConfig config;
  mutable std::string err;
};

struct gq_greta {
  GretaLoader loader;
  mutable std::string err;
};

namespace {
thread_local std::string g_open_err;
thread_local std::string g_greta_open_err;

void fill_config(const gcore::inference::ModelConfig &c, gq_gguf_config *out) {
  out->dim = c.dim;
  out->num_heads = c.num_heads;
  out->num_heads_kv = c.num_heads_kv;
  out->num_layers = c.num_layers;
  out->vocab_size = c.vocab_size;
  out->hidden_dim = c.hidden_dim;
  out->head_dim = c.head_dim;
  out->max_seq_len = c.max_seq_len;
  out->rope_base = c.rope_base;
  out->rms_eps = c.rms_eps;
}

bool kind_of(int k, GGUFLoader::LoadKind *out) {
  switch (k) {
  case GQ_LOAD_F32: *out = GGUFLoader::LoadKind::F32; return true;
  case GQ_LOAD_F16: *out = GGUFLoader::LoadKind::F16; return true;
  case GQ_LOAD_INT8: *out = GGUFLoader::LoadKind::INT8; return true;
  case GQ_LOAD_INT4: *out = GGUFLoader::LoadKind::INT4; return true;
  case GQ_LOAD_QUANT: *out = GGUFLoader::LoadKind::QUANT; return true;
  default: return false;
  }
}
}  // namespace

extern "C" {

int gq_gguf_open(const char *path, gq_gguf **out) {
  if (!out) return GQ_ERR_INVALID_ARGS;
  *out = nullptr;
  if (!path) return GQ_ERR_INVALID_ARGS;
  auto *g = new gq_gguf();
  std::string e;
  if (!g->loader.open(path, &e)) {
    g_open_err = e.empty() ? "GGUF open failed" : e;
    delete g;
    return GQ_ERR_INVALID_ARGS;
  }
  g->tensors = g->loader.list_tensors();
  for (auto &t : g->tensors) g->types.push_back((uint32_t)g->loader.ggml_type(t.name));
  g->config = g->loader.get_config();
  g_open_err.clear();
  *out = g;
  return GQ_OK;
}

const char *gq_gguf_open_error(void) { return g_open_err.c_str(); }

void gq_gguf_close(gq_gguf *g) { delete g; }

const char *gq_gguf_error(const gq_gguf *g) { return g ? g->err.c_str() : ""; }

size_t gq_gguf_tensor_count(const gq_gguf *g) { return g ? g->tensors.size() : 0; }

int gq_gguf_tensor_info(const gq_gguf *g, size_t index, gq_gguf_tensor *out) {
  if (!g || !out || index >= g->tensors.size()) return GQ_ERR_INVALID_ARGS;
  const auto &t = g->tensors[index];
  std::memset(out, 0, sizeof(*out));
  std::strncpy(out->name, t.name.c_str(), sizeof(out->name) - 1);
  std::strncpy(out->dtype, t.dtype.c_str(), sizeof(out->dtype) - 1);
  out->ggml_type = g->types[index];
  out->n_dims = (uint32_t)t.shape.size();
  for (size_t i = 0; i < t.shape.size() && i < 8; ++i) out->shape[i] = t.shape[i];
  out->offset = t.offset;
  out->size_bytes = t.size_bytes;
  return GQ_OK;
}

int gq_gguf_find(const gq_gguf *g, const char *name, size_t *index) {
  if (!g || !name || !index) return GQ_ERR_INVALID_ARGS;
  for (size_t i = 0; i < g->tensors.size(); ++i)
    if (g->tensors[i].name == name) {
      *index = i;
      return GQ_OK;
    }
  g->err = std::string("tensor not found: ") + name;
  return GQ_ERR_INVALID_ARGS;
}

int gq_gguf_get_config(const gq_gguf *g, gq_gguf_config *out) {
  if (!g || !out) return GQ_ERR_INVALID_ARGS;
  fill_config(g->config, out);
  return GQ_OK;
}

int gq_gguf_vocab_token(const gq_gguf *g, size_t i, const char **s, size_t *len) {
  if (!g || !s || !len || i >= g->config.vocabulary.size()) return GQ_ERR_INVALID_ARGS;
  *s = g->config.vocabulary[i].data();
  *len = g->config.vocabulary[i].size();
  return GQ_OK;
}

int gq_gguf_set_q4k_layout(gq_gguf *g, int ggml) {
  if (!g || (ggml != 0 && ggml != 1)) return GQ_ERR_INVALID_ARGS;
  g->loader.set_q4k_layout_ggml(ggml != 0);
  return GQ_OK;
}

int gq_gguf_read_raw(const gq_gguf *g, const char *name, void *dst, size_t capacity) {
  if (!g || !name || !dst) return GQ_ERR_INVALID_ARGS;
  std::vector<uint8_t> raw;
  if (!g->loader.read_raw(name, raw, &g->err)) return GQ_ERR_INVALID_ARGS;
  if (raw.size() > capacity) {
    g->err = "read_raw: destination too small";
    return GQ_ERR_INVALID_ARGS;
  }
  std::memcpy(dst, raw.data(), raw.size());
  return GQ_OK;
}

int gq_gguf_plan_load(const gq_gguf *g, const char *name, int kind, gq_gguf_plan *plan) {
  GGUFLoader::LoadKind k;
  if (!g || !name || !plan) return GQ_ERR_INVALID_ARGS;
  if (!kind_of(kind, &k)) return GQ_ERR_UNSUPPORTED;
  GGUFLoader::LoadPlan p;
  if (!g->loader.plan(name, k, &p, &g->err)) return GQ_ERR_INVALID_ARGS;
  std::memset(plan, 0, sizeof(*plan));
  plan->n_elem = p.n_elem;
  plan->bytes = p.bytes;
  plan->scale_bytes = p.scale_bytes;
  plan->num_heads = p.num_heads;
  plan->has_head_scales = p.has_head_scales;
  plan->is_qkv = p.is_qkv;
  plan->transpose = p.transpose;
  plan->fmt = p.fmt;
  plan->N = p.N;
  plan->K = p.K;
  return GQ_OK;
}

int gq_gguf_load(const gq_gguf *g, const char *name, int kind, void *d_out, size_t out_bytes, void *d_scales,
                 size_t scale_bytes, void *d_head_scales, size_t head_scale_bytes) {
  GGUFLoader::LoadKind k;
  if (!g || !name) return GQ_ERR_INVALID_ARGS;
  if (!kind_of(kind, &k)) return GQ_ERR_UNSUPPORTED;
  GGUFLoader::LoadPlan p;
  if (!g->loader.plan(name, k, &p, &g->err)) return GQ_ERR_INVALID_ARGS;
  if (!d_out || out_bytes < p.bytes || (p.scale_bytes && (!d_scales || scale_bytes < p.scale_bytes)) ||
      (p.has_head_scales && (!d_head_scales || head_scale_bytes < (size_t)p.num_heads * 4))) {
    g->err = "gq_gguf_load: destination missing or smaller than planned";
    return GQ_ERR_INVALID_ARGS;
  }
  if (!g->loader.load_into(name, k, p, d_out, d_scales, d_head_scales, &g->err)) return GQ_ERR_HIP;
  return GQ_OK;
}

int gq_gguf_load_quant_many(const gq_gguf *g, size_t n, const char *const *names, void *const *d_outs,
                            const size_t *out_bytes) {
  if (!g) return GQ_ERR_INVALID_ARGS;
  if (n == 0) return GQ_OK;
  if (!names || !d_outs || !out_bytes) return GQ_ERR_INVALID_ARGS;
  std::vector<std::string> nm(n);
  for (size_t i = 0; i < n; ++i) {
    if (!names[i]) return GQ_ERR_INVALID_ARGS;
    nm[i] = names[i];
  }
  // the checks (names, types, sizes) before any transfer
  for (size_t i = 0; i < n; ++i) {
    GGUFLoader::LoadPlan p;
    if (!g->loader.plan(nm[i], GGUFLoader::LoadKind::QUANT, &p, &g->err)) return GQ_ERR_INVALID_ARGS;
    if (!d_outs[i] || out_bytes[i] < p.bytes) {
      g->err = "gq_gguf_load_quant_many: destination missing or smaller than planned: " + nm[i];
      return GQ_ERR_INVALID_ARGS;
    }
  }
  if (!g->loader.load_quant_many(nm.data(), d_outs, out_bytes, n, &g->err)) return GQ_ERR_HIP;
  return GQ_OK;
}

// ---- .greta files -------------------------------------------------------------

int gq_greta_write(gq_gguf *g, const char *path, int kind, size_t *written) {
  if (written) *written = 0;
  if (!g || !path) return GQ_ERR_INVALID_ARGS;
  gcore::inference::GretaWriteKind k;
  if (kind == GQ_LOAD_QUANT) k = gcore::inference::GretaWriteKind::T16;
  else if (kind == GQ_LOAD_INT4) k = gcore::inference::GretaWriteKind::INT4;
  else return GQ_ERR_UNSUPPORTED;
  size_t n = 0;
  if (!gcore::inference::write_greta(g->loader, path, k, &n, &g->err)) return GQ_ERR_INVALID_ARGS;
  if (written) *written = n;
  return GQ_OK;
}

int gq_greta_open(const char *path, gq_greta **out) {
  if (!out) return GQ_ERR_INVALID_ARGS;
  *out = nullptr;
  if (!path) return GQ_ERR_INVALID_ARGS;
  auto *h = new gq_greta();
  std::string e;
  if (!h->loader.open(path, &e)) {
    g_greta_open_err = e.empty() ? ".greta open failed" : e;
    delete h;
    return GQ_ERR_INVALID_ARGS;
  }
  g_greta_open_err.clear();
  *out = h;
  return GQ_OK;
}

const char *gq_greta_open_error(void) { return g_greta_open_err.c_str(); }

void gq_greta_close(gq_greta *h) { delete h; }

const char *gq_greta_error(const gq_greta *h) { return h ? h->err.c_str() : ""; }

size_t gq_greta_tensor_count(const gq_greta *h) { return h ? h->loader.records().size() : 0; }

int gq_greta_tensor_info(const gq_greta *h, size_t index, gq_greta_tensor *out) {
  if (!h || !out || index >= h->loader.records().size()) return GQ_ERR_INVALID_ARGS;
  const auto &r = h->loader.records()[index];
  std::memset(out, 0, sizeof(*out));
  std::strncpy(out->name, r.name.c_str(), sizeof(out->name) - 1);
  out->dtype = r.dtype;
  out->n_dims = (uint32_t)r.shape.size();
  for (size_t i = 0; i < r.shape.size() && i < 8; ++i) out->shape[i] = r.shape[i];
  out->group_size = r.group_size;
  out->num_heads = r.num_heads;
  out->w_bytes = r.w_size;
  out->s_bytes = r.s_size;
  out->h_bytes = r.h_size;
  out->fmt = gcore::inference::greta_fmt_of_dtype(r.dtype);
  if (out->fmt >= 0 && !r.shape.empty() && r.shape[0]) {
    uint64_t n = 1;
    for (uint64_t d : r.shape) n *= d;
    out->K = r.shape[0];
    out->N = n / r.shape[0];
  }
  return GQ_OK;
}

int gq_greta_find(const gq_greta *h, const char *name, size_t *index) {
  if (!h || !name || !index) return GQ_ERR_INVALID_ARGS;
  const auto &recs = h->loader.records();
  for (size_t i = 0; i < recs.size(); ++i)
    if (recs[i].name == name) {
      *index = i;
      return GQ_OK;
    }
  h->err = std::string("tensor not found: ") + name;
  return GQ_ERR_INVALID_ARGS;
}

int gq_greta_get_config(const gq_greta *h, gq_gguf_config *out) {
  if (!h || !out) return GQ_ERR_INVALID_ARGS;
  fill_config(h->loader.get_config(), out);
  return GQ_OK;
}

int gq_greta_load(const gq_greta *h, const char *name, void *d_w, size_t w_cap, void *d_s, size_t s_cap, void *d_h,
                  size_t h_cap) {
  if (!h || !name) return GQ_ERR_INVALID_ARGS;
  size_t i;
  if (gq_greta_find(h, name, &i) != GQ_OK) return GQ_ERR_INVALID_ARGS;
  const auto &r = h->loader.records()[i];
  if (!d_w || w_cap < r.w_size || (r.s_size && (!d_s || s_cap < r.s_size)) ||
      (r.h_size && (!d_h || h_cap < r.h_size))) {
    h->err = "gq_greta_load: destination missing or smaller than the record";
    return GQ_ERR_INVALID_ARGS;
  }
  if (!h->loader.load_into(name, d_w, w_cap, d_s, s_cap, d_h, h_cap, &h->err)) return GQ_ERR_HIP;
  return GQ_OK;
}

}  // extern "C"
