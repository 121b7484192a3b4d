// GGUF loader with the reference's WeightLoader / GGUFLoader behaviour
// (src/inference/src/weight_loader.cpp:218-1008, factory :1043-1053).
//
// The file is memory-mapped and parsed with bounds checks; tensor data is
// copied to the GPU as stored and converted there by libgq's bit-exact
// kernels (dequant, fp16 truncation, GQA transpose, INT8/INT4 requant, head
// scales, T16 repack).
#include "gcore/inference/weight_loader.hpp"

#include "gcore/inference/greta_file.hpp"

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdlib>
#include <cstring>
#include <iostream>

#include "gq.h"
#include "upload.hpp"

namespace gcore::inference {

namespace {

// GGML type ids (weight_loader.cpp:15-33).
enum : uint32_t {
  T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8,
  T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14,
};

// Block geometry used for size_bytes (weight_loader.cpp:38-82): unknown types
// have a 32-element block of 0 bytes.
size_t type_block_elems(uint32_t t) {
  switch (t) {
  case T_F32: case T_F16: return 1;
  case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
  default: return 32;
  }
}
size_t type_block_bytes(uint32_t t) {
  switch (t) {
  case T_F32: return 4;
  case T_F16: return 2;
  case T_Q4_0: return 18;
  case T_Q4_1: return 20;
  case T_Q8_0: return 34;
  case T_Q4_K: return 144;
  case T_Q5_K: return 176;
  case T_Q6_K: return 210;
  default: return 0;
  }
}
// Type names reported in TensorInfo::dtype (weight_loader.cpp:179-194), plus
// "Q8_0", which the reference reports as "UNKNOWN".
const char *type_name(uint32_t t) {
  switch (t) {
  case T_F32: return "F32";
  case T_F16: return "F16";
  case T_Q4_0: return "Q4_0";
  case T_Q8_0: return "Q8_0";
  case T_Q4_K: return "Q4_K";
  case T_Q6_K: return "Q6_K";
  default: return "UNKNOWN";
  }
}

constexpr uint64_t kMaxLen = 1000000;  // string / array length limit (:236-256)

// Bounds-checked little-endian cursor over the mapped file.
struct Cursor {
  const uint8_t *p;
  size_t n, pos = 0;
  bool ok = true;
  bool take(void *dst, size_t k) {
    if (!ok || k > n - pos) return ok = false;
    if (dst) std::memcpy(dst, p + pos, k);
    pos += k;
    return true;
  }
  bool skip(uint64_t k) {
    if (!ok || k > n - pos) return ok = false;
    pos += (size_t)k;
    return true;
  }
  template <typename T> bool get(T &v) { return take(&v, sizeof(T)); }
};

// Scalar GGUF value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32,
// 7 bool, 10 u64, 11 i64, 12 f64; 8 string, 9 array.
size_t scalar_bytes(uint32_t t) {
  switch (t) {
  case 0: case 1: case 7: return 1;
  case 2: case 3: return 2;
  case 4: case 5: case 6: return 4;
  case 10: case 11: case 12: return 8;
  default: return 0;
  }
}

bool skip_value(Cursor &c, uint32_t t, int depth) {
  if (size_t b = scalar_bytes(t)) return c.skip(b);
  if (t == 8) {
    uint64_t len;
    return c.get(len) && len <= kMaxLen && c.skip(len);
  }
  if (t == 9 && depth < 4) {
    uint32_t at;
    uint64_t len;
    if (!c.get(at) || !c.get(len) || len > kMaxLen) return false;
    if (size_t b = scalar_bytes(at)) return c.skip(len * b);
    for (uint64_t i = 0; i < len; ++i)
      if (!skip_value(c, at, depth + 1)) return false;
    return true;
  }
  return false;
}

// Numeric value as double (integer or float types); false for strings,
// arrays and bools.
bool read_number(Cursor &c, uint32_t t, double &out) {
  switch (t) {
  case 0: { uint8_t v; if (!c.get(v)) return false; out = v; return true; }
  case 1: { int8_t v; if (!c.get(v)) return false; out = v; return true; }
  case 2: { uint16_t v; if (!c.get(v)) return false; out = v; return true; }
  case 3: { int16_t v; if (!c.get(v)) return false; out = v; return true; }
  case 4: { uint32_t v; if (!c.get(v)) return false; out = v; return true; }
  case 5: { int32_t v; if (!c.get(v)) return false; out = v; return true; }
  case 6: { float v; if (!c.get(v)) return false; out = v; return true; }
  case 10: { uint64_t v; if (!c.get(v)) return false; out = (double)v; return true; }
  case 11: { int64_t v; if (!c.get(v)) return false; out = (double)v; return true; }
  case 12: { double v; if (!c.get(v)) return false; out = v; return true; }
  default: return false;
  }
}

bool is_float_type(uint32_t t) { return t == 6 || t == 12; }

void set_err(std::string *err, const std::string &msg) {
  if (err) *err = msg;
}

// Device allocation released on scope exit (after the device is idle).
struct DevMem {
  void *p = nullptr;
  ~DevMem() {
    if (p) (void)hipFree(p);
  }
  bool alloc(size_t bytes, std::string *err) {
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
      p = nullptr;
      set_err(err, std::string("hipMalloc failed: ") + hipGetErrorString(e));
      return false;
    }
    return true;
  }
};

bool hip_ok(hipError_t e, const char *what, std::string *err) {
  if (e == hipSuccess) return true;
  set_err(err, std::string(what) + ": " + hipGetErrorString(e));
  return false;
}
bool gq_ok(int st, const char *what, std::string *err) {
  if (st == GQ_OK) return true;
  std::string m = std::string(what) + ": " + gq_status_string(st);
  const char *h = gq_last_error();
  if (h && *h) m += std::string(" (") + h + ")";
  set_err(err, m);
  return false;
}

bool is_kv_name(const std::string &n) {
  return n.find("attn_k.weight") != std::string::npos || n.find("attn_v.weight") != std::string::npos;
}
bool is_qkv_name(const std::string &n) {
  return n.find("attn_q") != std::string::npos || n.find("attn_k") != std::string::npos ||
         n.find("attn_v") != std::string::npos;
}

}  // namespace

struct GGUFLoader::Impl {
  std::string path;
  int fd = -1;
  const uint8_t *map = nullptr;
  size_t map_size = 0;
  std::vector<TensorInfo> tensors;
  std::vector<uint32_t> types;  // GGML type id per tensor
  ModelConfig config;
  size_t data_offset = 0;
  bool loaded = false;
  bool q4k_ggml = false;
  std::unique_ptr<Uploader> up;  // pinned staging ring, created at the first load

  Uploader &uploader() {
    if (!up) up = std::make_unique<Uploader>();
    up->bind_file(fd, map, map_size);  // slices of the mapping are read with pread
    return *up;
  }
  bool upload(void *dst, const uint8_t *src, size_t bytes, std::string *err) {
    return uploader().copy(dst, src, bytes, err);
  }

  ~Impl() { close(); }
  void close() {
    if (map) munmap(const_cast<uint8_t *>(map), map_size);
    if (fd >= 0) ::close(fd);
    map = nullptr;
    map_size = 0;
    fd = -1;
    tensors.clear();
    types.clear();
    loaded = false;
  }

  // llama.* keys and the vocabulary (weight_loader.cpp:272-427).
  bool parse_kv(Cursor &c, std::string *err) {
    uint64_t klen;
    if (!c.get(klen) || klen > 1024) return set_err(err, "GGUF: bad key length"), false;
    std::string key(klen, '\0');
    if (!c.take(&key[0], klen)) return set_err(err, "GGUF: truncated key"), false;
    uint32_t vt;
    if (!c.get(vt)) return set_err(err, "GGUF: truncated value type"), false;

    uint32_t *u32_field = nullptr;
    float *f32_field = nullptr;
    if (key == "llama.embedding_length") u32_field = &config.dim;
    else if (key == "llama.feed_forward_length") u32_field = &config.hidden_dim;
    else if (key == "llama.block_count") u32_field = &config.num_layers;
    else if (key == "llama.attention.head_count") u32_field = &config.num_heads;
    else if (key == "llama.attention.head_count_kv") u32_field = &config.num_heads_kv;
    else if (key == "llama.context_length") u32_field = &config.max_seq_len;
    else if (key == "llama.rope.freq_base") f32_field = &config.rope_base;
    else if (key == "llama.norm_eps") f32_field = &config.rms_eps;

    if (u32_field) {
      double v;
      if (!read_number(c, vt, v)) return set_err(err, "GGUF: non-numeric value for " + key), false;
      *u32_field = (uint32_t)(int64_t)v;
      if (u32_field == &config.num_heads && config.num_heads_kv == 0) config.num_heads_kv = config.num_heads;
      if ((u32_field == &config.dim || u32_field == &config.num_heads) && config.num_heads > 0)
        config.head_dim = config.dim / config.num_heads;
      return true;
    }
    if (f32_field) {
      double v;
      if (!is_float_type(vt) || !read_number(c, vt, v))
        return set_err(err, "GGUF: non-float value for " + key), false;
      *f32_field = (float)v;
      return true;
    }
    if (key == "tokenizer.ggml.tokens" && vt == 9) {
      uint32_t at;
      uint64_t len;
      if (!c.get(at) || !c.get(len) || at != 8 || len > kMaxLen)
        return set_err(err, "GGUF: bad tokenizer.ggml.tokens"), false;
      config.vocabulary.clear();
      config.vocabulary.reserve(len);
      for (uint64_t i = 0; i < len; ++i) {
        uint64_t sl;
        if (!c.get(sl)) return set_err(err, "GGUF: truncated token"), false;
        if (sl > 1024) {
          if (!c.skip(sl)) return set_err(err, "GGUF: truncated token"), false;
          config.vocabulary.push_back("<too_long>");
          continue;
        }
        std::string s(sl, '\0');
        if (!c.take(sl ? &s[0] : nullptr, sl)) return set_err(err, "GGUF: truncated token"), false;
        config.vocabulary.push_back(std::move(s));
      }
      config.vocab_size = (uint32_t)len;
      return true;
    }
    if (!skip_value(c, vt, 0)) return set_err(err, "GGUF: cannot skip value of " + key), false;
    return true;
  }

  // Tensor info (weight_loader.cpp:429-465).
  bool parse_tensor(Cursor &c, TensorInfo &info, uint32_t &type, std::string *err) {
    uint64_t nl;
    if (!c.get(nl) || nl > 512) return set_err(err, "GGUF: bad tensor name length"), false;
    info.name.assign(nl, '\0');
    if (!c.take(nl ? &info.name[0] : nullptr, nl)) return set_err(err, "GGUF: truncated tensor name"), false;
    uint32_t nd;
    if (!c.get(nd) || nd > 8) return set_err(err, "GGUF: bad n_dims for " + info.name), false;
    info.shape.resize(nd);
    size_t n = 1;
    for (uint32_t i = 0; i < nd; ++i) {
      uint64_t d;
      if (!c.get(d)) return set_err(err, "GGUF: truncated shape"), false;
      info.shape[i] = (size_t)d;
      n *= (size_t)d;
    }
    uint64_t off;
    if (!c.get(type) || !c.get(off)) return set_err(err, "GGUF: truncated tensor info"), false;
    info.dtype = type_name(type);
    info.offset = (size_t)off;
    size_t bs = type_block_elems(type), ts = type_block_bytes(type);
    info.size_bytes = type <= T_F16 ? n * ts : ((n + bs - 1) / bs) * ts;
    return true;
  }

  bool open(const std::string &p, std::string *err) {
    close();
    path = p;
    fd = ::open(p.c_str(), O_RDONLY);
    if (fd < 0) return set_err(err, "cannot open " + p), false;
    struct stat st;
    if (fstat(fd, &st) != 0) return set_err(err, "cannot stat " + p), false;
    map_size = (size_t)st.st_size;
    if (map_size > 0) {
      void *m = mmap(nullptr, map_size, PROT_READ, MAP_PRIVATE, fd, 0);
      if (m == MAP_FAILED) return set_err(err, "mmap failed for " + p), false;
      map = (const uint8_t *)m;
    }
    Cursor c{map, map_size};
    char magic[4];
    if (!c.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return set_err(err, "Not GGUF"), false;
    uint32_t version;
    if (!c.get(version) || version < 2) return set_err(err, "Old GGUF"), false;
    uint64_t n_tensors, n_kv;
    if (!c.get(n_tensors) || !c.get(n_kv)) return set_err(err, "GGUF: truncated header"), false;
    if (n_kv > 2000) return set_err(err, "GGUF: too many key/value pairs"), false;
    config = ModelConfig::llama2_7b();
    for (uint64_t i = 0; i < n_kv; ++i)
      if (!parse_kv(c, err)) return false;
    // every tensor info takes at least 24 bytes
    if (n_tensors > (map_size - c.pos) / 24) return set_err(err, "GGUF: bad tensor count"), false;
    tensors.reserve(n_tensors);
    types.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; ++i) {
      TensorInfo info;
      uint32_t t;
      if (!parse_tensor(c, info, t, err)) return false;
      tensors.push_back(std::move(info));
      types.push_back(t);
    }
    // data section: next 32-byte boundary (alignment fixed at 32, :497-501)
    data_offset = (c.pos + 31) & ~(size_t)31;
    for (auto &t : tensors) t.offset += data_offset;
    if (const char *e = std::getenv("GQ_Q4K_LAYOUT")) q4k_ggml = std::strcmp(e, "ggml") == 0;
    loaded = true;
    return true;
  }

  int find(const std::string &name) const {
    for (size_t i = 0; i < tensors.size(); ++i)
      if (tensors[i].name == name) return (int)i;
    return -1;
  }

  // Locates a tensor's bytes inside the mapping.
  bool locate(const std::string &name, int &idx, const uint8_t *&data, std::string *err) const {
    if (!loaded) return set_err(err, "GGUF loader not open"), false;
    idx = find(name);
    if (idx < 0) return set_err(err, "tensor not found: " + name), false;
    const TensorInfo &t = tensors[idx];
    if (t.offset > map_size || t.size_bytes > map_size - t.offset)
      return set_err(err, "tensor data outside the file: " + name), false;
    data = map + t.offset;
    return true;
  }

  int q4k_fmt() const { return q4k_ggml ? GQ_FMT_Q4_K_GGML : GQ_FMT_Q4_K; }
  // the k-quant layout flag covers Q6_K too (a file uses one family of layouts)
  int q6k_fmt() const { return q4k_ggml ? GQ_FMT_Q6_K_GGML : GQ_FMT_Q6_K; }

  // Device dequant of a tensor to fp32 (weight_loader.cpp:517-560 conversions).
  bool to_f32(int idx, const uint8_t *data, size_t n_elem, float *out, std::string *err) {
    const uint32_t t = types[idx];
    const TensorInfo &info = tensors[idx];
    if (t == T_F32) return upload(out, data, n_elem * 4, err);
    int fmt;
    size_t be;
    switch (t) {
    case T_F16: fmt = GQ_FMT_F16; be = 1; break;
    case T_Q4_0: fmt = GQ_FMT_Q4_0; be = 32; break;
    case T_Q8_0: fmt = GQ_FMT_Q8_0; be = 32; break;
    case T_Q4_K: fmt = q4k_fmt(); be = 256; break;
    case T_Q6_K: fmt = q6k_fmt(); be = 256; break;
    default: return set_err(err, "unsupported tensor type " + info.dtype + " for " + info.name), false;
    }
    if (n_elem % be) return set_err(err, "element count not a whole number of blocks: " + info.name), false;
    DevMem raw;
    if (!raw.alloc(info.size_bytes, err)) return false;
    if (!upload(raw.p, data, info.size_bytes, err)) return false;
    if (!gq_ok(gq_dequant_gguf(fmt, raw.p, n_elem / be, out, nullptr), "dequant", err)) return false;
    return hip_ok(hipStreamSynchronize(nullptr), "dequant", err);
  }
};

GGUFLoader::GGUFLoader() : impl_(std::make_unique<Impl>()) {}
GGUFLoader::~GGUFLoader() = default;

bool GGUFLoader::open(const std::string &path, std::string *err) { return impl_->open(path, err); }
std::vector<TensorInfo> GGUFLoader::list_tensors() const { return impl_->tensors; }
ModelConfig GGUFLoader::get_config() const { return impl_->config; }
void GGUFLoader::set_q4k_layout_ggml(bool ggml) { impl_->q4k_ggml = ggml; }

int GGUFLoader::ggml_type(const std::string &name) const {
  int i = impl_->find(name);
  return i < 0 ? -1 : (int)impl_->types[i];
}

bool GGUFLoader::read_raw(const std::string &name, std::vector<uint8_t> &out, std::string *err) const {
  int idx;
  const uint8_t *data;
  if (!impl_->locate(name, idx, data, err)) return false;
  out.assign(data, data + impl_->tensors[idx].size_bytes);
  return true;
}

bool GGUFLoader::plan(const std::string &name, LoadKind kind, LoadPlan *p, std::string *err) const {
  int idx;
  const uint8_t *data;
  if (!impl_->locate(name, idx, data, err)) return false;
  const TensorInfo &t = impl_->tensors[idx];
  const uint32_t type = impl_->types[idx];
  const ModelConfig &cfg = impl_->config;
  LoadPlan r;
  r.n_elem = 1;
  for (size_t d : t.shape) r.n_elem *= d;
  using DT = gcore::rt::GretaDataType;

  // GQA K/V handling (weight_loader.cpp:597-658): tensors named attn_k/attn_v
  // in a [D, KV] shape are read as [D][KV] and transposed to [KV][D].
  auto gqa = [&](const char *what) -> bool {
    if (!(is_kv_name(name) && cfg.num_heads_kv > 0 && cfg.head_dim > 0)) return true;
    const size_t kv = (size_t)cfg.num_heads_kv * cfg.head_dim, dm = cfg.dim;
    if (t.shape.size() != 2 || kv == 0 || dm == 0)
      return set_err(err, std::string("GQA KV ") + what + "load failed for " + name +
                              ": unexpected shape dims or config mismatch"),
             false;
    if (t.shape[0] == dm && t.shape[1] == kv) r.transpose = true;
    else if (t.shape[0] == kv && t.shape[1] == dm) {
    } else
      return set_err(err, std::string("GQA KV ") + what + "load failed for " + name + ": shape " +
                              std::to_string(t.shape[0]) + " x " + std::to_string(t.shape[1]) +
                              " matches neither dim x kv nor kv x dim"),
             false;
    return true;
  };
  auto dequantizable = [&]() {
    return type == T_F32 || type == T_F16 || type == T_Q4_0 || type == T_Q8_0 || type == T_Q4_K ||
           type == T_Q6_K;
  };

  switch (kind) {
  case LoadKind::F32:
    if (!dequantizable()) return set_err(err, "unsupported tensor type " + t.dtype + " for " + name), false;
    r.bytes = r.n_elem * 4;
    r.type = DT::FP32;
    break;
  case LoadKind::F16:
    if (!dequantizable()) return set_err(err, "unsupported tensor type " + t.dtype + " for " + name), false;
    if (!gqa("")) return false;
    r.bytes = r.n_elem * 2;
    r.type = DT::FP16;
    break;
  case LoadKind::INT8:
    if (!dequantizable())
      return set_err(err, "no INT8 requantization from tensor type " + t.dtype), false;
    // Q8_0 blocks are split as stored (no transpose), other types requantized
    if (type != T_Q8_0 && !gqa("INT8 ")) return false;
    r.bytes = r.n_elem;
    r.scale_bytes = ((r.n_elem + 31) / 32) * 4;
    r.type = DT::INT8;
    break;
  case LoadKind::INT4: {
    if (!dequantizable())
      return set_err(err, "no INT4 requantization from tensor type " + t.dtype), false;
    if (!gqa("INT4 ")) return false;
    r.bytes = (r.n_elem + 1) / 2;
    r.scale_bytes = ((r.n_elem + 31) / 32) * 4;
    r.type = DT::INT4;
    uint32_t nh = cfg.num_heads;
    if (is_kv_name(name) && cfg.num_heads_kv > 0) nh = cfg.num_heads_kv;
    r.is_qkv = is_qkv_name(name);
    r.has_head_scales = r.is_qkv && nh > 0 && cfg.head_dim > 0;
    r.num_heads = nh;
    if (r.has_head_scales && (size_t)nh * cfg.head_dim * cfg.dim > r.n_elem)
      return set_err(err, "head scales of " + name + " need " + std::to_string(nh) + " x " +
                              std::to_string(cfg.head_dim) + " x " + std::to_string(cfg.dim) +
                              " values; the tensor has " + std::to_string(r.n_elem)),
             false;
    break;
  }
  case LoadKind::QUANT: {
    if (type == T_Q4_0) r.fmt = GQ_FMT_Q4_0, r.type = DT::Q4_0;
    else if (type == T_Q8_0) r.fmt = GQ_FMT_Q8_0, r.type = DT::Q8_0;
    else if (type == T_Q4_K) {
      r.fmt = impl_->q4k_fmt();
      r.type = impl_->q4k_ggml ? DT::Q4_K_GGML : DT::Q4_K;
    } else if (type == T_Q6_K) {
      r.fmt = impl_->q6k_fmt();
      r.type = impl_->q4k_ggml ? DT::Q6_K_GGML : DT::Q6_K;
    } else
      return set_err(err, "load_tensor_quant: " + name + " is " + t.dtype +
                              " (Q4_0, Q8_0, Q4_K or Q6_K expected)"),
             false;
    if (t.shape.empty()) return set_err(err, "load_tensor_quant: scalar tensor " + name), false;
    r.K = t.shape[0];
    r.N = r.K ? r.n_elem / r.K : 0;
    if (!gq_ok(gq_packed_size(r.fmt, r.N, r.K, &r.bytes), "load_tensor_quant", err)) return false;
    break;
  }
  }
  *p = r;
  return true;
}

bool GGUFLoader::load_into(const std::string &name, LoadKind kind, const LoadPlan &p, void *out, void *scales,
                           void *head_scales, std::string *err) const {
  int idx;
  const uint8_t *data;
  if (!impl_->locate(name, idx, data, err)) return false;
  if (!out || ((kind == LoadKind::INT8 || kind == LoadKind::INT4) && !scales) ||
      (kind == LoadKind::INT4 && p.has_head_scales && !head_scales))
    return set_err(err, "load_into: missing destination"), false;
  const ModelConfig &cfg = impl_->config;
  const size_t n = p.n_elem;
  const size_t kv = (size_t)cfg.num_heads_kv * cfg.head_dim, dm = cfg.dim;
  auto note_transpose = [&]() {
    std::cout << "[gq-load] " << name << ": K/V rows reordered, dim x kv -> kv x dim" << std::endl;
  };

  if (kind == LoadKind::QUANT) {
    // sliced upload, each slice repacked into `out` while the next is copied
    const size_t rb = impl_->tensors[idx].size_bytes;
    if (p.N == 0 || rb % p.N) return set_err(err, "load_tensor_quant: ragged rows in " + name), false;
    return impl_->uploader().repack(p.fmt, data, p.N, p.K, rb / p.N, out, err);
  }
  if (kind == LoadKind::F32) return impl_->to_f32(idx, data, n, (float *)out, err);

  if (kind == LoadKind::INT8 && impl_->types[idx] == T_Q8_0) {
    DevMem raw;
    const size_t rb = impl_->tensors[idx].size_bytes;
    if (n % 32) return set_err(err, "element count not a whole number of blocks: " + name), false;
    if (!raw.alloc(rb, err)) return false;
    if (!impl_->upload(raw.p, data, rb, err)) return false;
    if (!gq_ok(gq_split_q8_0(raw.p, n / 32, (int8_t *)out, (float *)scales, nullptr), "Q8_0 split", err))
      return false;
    return hip_ok(hipStreamSynchronize(nullptr), "Q8_0 split", err);
  }

  if (kind == LoadKind::F16 && impl_->types[idx] == T_F16) {
    // stored fp16 is uploaded as is (weight_loader.cpp:596-597): fp16
    // subnormals survive, unlike the fp32 -> fp16 truncation of other types
    const size_t rb = n * 2;
    if (!p.transpose) return impl_->upload(out, data, rb, err);
    DevMem h;
    if (!h.alloc(rb, err)) return false;
    if (!impl_->upload(h.p, data, rb, err)) return false;
    if (!gq_ok(gq_transpose_kv(2, h.p, dm, kv, out, nullptr), "GQA transpose", err)) return false;
    if (!hip_ok(hipStreamSynchronize(nullptr), "GQA transpose", err)) return false;
    note_transpose();
    return true;
  }

  DevMem f32, f32t;
  if (!f32.alloc(n * 4, err)) return false;
  if (!impl_->to_f32(idx, data, n, (float *)f32.p, err)) return false;
  const float *w = (const float *)f32.p;

  if (kind == LoadKind::F16) {
    if (!p.transpose) {
      if (!gq_ok(gq_convert_f32_to_f16(w, n, (uint16_t *)out, nullptr), "fp16 convert", err)) return false;
    } else {
      DevMem h;
      if (!h.alloc(n * 2, err)) return false;
      if (!gq_ok(gq_convert_f32_to_f16(w, n, (uint16_t *)h.p, nullptr), "fp16 convert", err)) return false;
      if (!gq_ok(gq_transpose_kv(2, h.p, dm, kv, out, nullptr), "GQA transpose", err)) return false;
      if (!hip_ok(hipStreamSynchronize(nullptr), "GQA transpose", err)) return false;
      note_transpose();
    }
    return hip_ok(hipStreamSynchronize(nullptr), "fp16 convert", err);
  }

  if (p.transpose) {
    if (!f32t.alloc(n * 4, err)) return false;
    if (!gq_ok(gq_transpose_kv(4, w, dm, kv, f32t.p, nullptr), "GQA transpose", err)) return false;
    w = (const float *)f32t.p;
    note_transpose();
  }
  if (kind == LoadKind::INT8) {
    if (!gq_ok(gq_requant_int8(w, n, (int8_t *)out, (float *)scales, nullptr), "INT8 requant", err)) return false;
  } else {
    if (!gq_ok(gq_requant_int4(w, n, (uint8_t *)out, (float *)scales, nullptr), "INT4 requant", err)) return false;
    if (p.has_head_scales &&
        !gq_ok(gq_head_scales(w, n, p.num_heads, cfg.head_dim, cfg.dim, (float *)head_scales, nullptr),
               "head scales", err))
      return false;
  }
  return hip_ok(hipStreamSynchronize(nullptr), "requant", err);
}

// ---- Buffer-based interface (weight_loader.cpp:517-1008) -------------------
namespace {
bool alloc_buffer(gcore::rt::hip::Buffer &b, size_t bytes, gcore::rt::GretaDataType type, std::string *err) {
  return b.allocate(bytes, gcore::rt::hip::BufferUsage::DeviceOnly, type, err);
}
}  // namespace

bool GGUFLoader::load_tensor(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) {
  LoadPlan p;
  if (!plan(name, LoadKind::F32, &p, err) || !alloc_buffer(buffer, p.bytes, p.type, err)) return false;
  return load_into(name, LoadKind::F32, p, buffer.data(), nullptr, nullptr, err);
}

bool GGUFLoader::load_tensor_fp16(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) {
  LoadPlan p;
  if (!plan(name, LoadKind::F16, &p, err) || !alloc_buffer(buffer, p.bytes, p.type, err)) return false;
  return load_into(name, LoadKind::F16, p, buffer.data(), nullptr, nullptr, err);
}

bool GGUFLoader::load_tensor_int8(const std::string &name, gcore::rt::hip::Buffer &buffer,
                                  gcore::rt::hip::Buffer &scales, std::string *err) {
  LoadPlan p;
  if (!plan(name, LoadKind::INT8, &p, err) || !alloc_buffer(buffer, p.bytes, p.type, err) ||
      !alloc_buffer(scales, p.scale_bytes, gcore::rt::GretaDataType::FP32, err))
    return false;
  if (!load_into(name, LoadKind::INT8, p, buffer.data(), scales.data(), nullptr, err)) return false;
  gcore::rt::GretaQuantInfo q;
  q.group_size = 32;
  q.scales = scales.data();
  buffer.set_quant_info(q);
  return true;
}

bool GGUFLoader::load_tensor_int4(const std::string &name, gcore::rt::hip::Buffer &buffer,
                                  gcore::rt::hip::Buffer &scales, gcore::rt::hip::Buffer &head_scales,
                                  std::string *err) {
  LoadPlan p;
  if (!plan(name, LoadKind::INT4, &p, err) || !alloc_buffer(buffer, p.bytes, p.type, err) ||
      !alloc_buffer(scales, p.scale_bytes, gcore::rt::GretaDataType::FP32, err))
    return false;
  if (p.has_head_scales && !alloc_buffer(head_scales, (size_t)p.num_heads * 4, gcore::rt::GretaDataType::FP32, err))
    return false;
  if (!load_into(name, LoadKind::INT4, p, buffer.data(), scales.data(),
                 p.has_head_scales ? head_scales.data() : nullptr, err))
    return false;
  gcore::rt::GretaQuantInfo q;
  q.group_size = 32;
  q.scales = scales.data();
  q.head_scales = p.is_qkv ? head_scales.data() : nullptr;
  q.num_heads = p.is_qkv ? p.num_heads : 0;
  buffer.set_quant_info(q);
  return true;
}

bool GGUFLoader::load_quant_many(const std::string *names, void *const *outs, const size_t *out_bytes, size_t n,
                                 std::string *err) const {
  if (n == 0) return true;
  if (!names || !outs || !out_bytes) return set_err(err, "load_quant_many: null argument"), false;
  std::vector<Uploader::RepackJob> jobs(n);
  for (size_t i = 0; i < n; ++i) {
    LoadPlan p;
    if (!plan(names[i], LoadKind::QUANT, &p, err)) return false;
    if (!outs[i] || out_bytes[i] < p.bytes)
      return set_err(err, "load_quant_many: destination missing or smaller than planned: " + names[i]), false;
    int idx = -1;
    const uint8_t *data = nullptr;
    if (!impl_->locate(names[i], idx, data, err)) return false;
    const size_t rb = impl_->tensors[idx].size_bytes;
    if (p.N == 0 || rb % p.N) return set_err(err, "load_quant_many: ragged rows in " + names[i]), false;
    jobs[i] = Uploader::RepackJob{p.fmt, data, p.N, p.K, rb / p.N, outs[i]};
  }
  return impl_->uploader().repack_many(jobs.data(), n, err);
}

bool GGUFLoader::load_tensor_quant(const std::string &name, gcore::rt::hip::Buffer &packed, std::string *err) {
  LoadPlan p;
  if (!plan(name, LoadKind::QUANT, &p, err) || !alloc_buffer(packed, p.bytes, p.type, err)) return false;
  if (!load_into(name, LoadKind::QUANT, p, packed.data(), nullptr, nullptr, err)) return false;
  gcore::rt::GretaQuantInfo q;
  q.group_size = (p.fmt == GQ_FMT_Q4_K || p.fmt == GQ_FMT_Q4_K_GGML || p.fmt == GQ_FMT_Q6_K ||
                  p.fmt == GQ_FMT_Q6_K_GGML)
                     ? 256
                     : 32;
  q.format = (uint32_t)p.fmt;
  packed.set_quant_info(q);
  return true;
}

std::unique_ptr<WeightLoader> create_weight_loader(const std::string &path, std::string *err) {
  if (path.find(".gguf") != std::string::npos) {
    auto l = std::make_unique<GGUFLoader>();
    if (!l->open(path, err)) return nullptr;
    return l;
  }
  // the reference's factory knows only .gguf (:1043-1053); .greta files are
  // read by GretaLoader
  if (path.find(".greta") != std::string::npos) {
    auto l = std::make_unique<GretaLoader>();
    if (!l->open(path, err)) return nullptr;
    return l;
  }
  set_err(err, "not a .gguf or .greta path: " + path);
  return nullptr;
}

}  // namespace gcore::inference
