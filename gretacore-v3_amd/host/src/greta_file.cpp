// .greta writer and reader (container of tools/quantize/greta_quantize_gguf.cpp:
// 40-124; the reference has no reader).
#include "gcore/inference/greta_file.hpp"

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iostream>

#include "gq.h"
#include "upload.hpp"

namespace gcore::inference {

using gcore::rt::GretaDataType;

namespace {

bool fail(std::string *err, const std::string &m) {
  if (err) *err = m;
  return false;
}

const char kMagic[8] = {'G', 'R', 'E', 'T', 'A', '_', 'W', '\0'};

// name of a record's dtype in TensorInfo::dtype
const char *dtype_name(uint32_t d) {
  switch ((GretaDataType)d) {
  case GretaDataType::FP32: return "F32";
  case GretaDataType::FP16: return "F16";
  case GretaDataType::INT8: return "INT8";
  case GretaDataType::INT4: return "INT4";
  case GretaDataType::Q4_0: return "Q4_0";
  case GretaDataType::Q8_0: return "Q8_0";
  case GretaDataType::Q4_K: return "Q4_K";
  case GretaDataType::Q4_K_GGML: return "Q4_K_GGML";
  case GretaDataType::Q6_K: return "Q6_K";
  case GretaDataType::Q6_K_GGML: return "Q6_K_GGML";
  default: return "UNKNOWN";
  }
}

// Value of a top-level numeric key in a flat JSON object, if present.
bool json_number(const std::string &js, const char *key, double *v) {
  const std::string k = std::string("\"") + key + "\"";
  size_t p = js.find(k);
  if (p == std::string::npos) return false;
  p = js.find(':', p + k.size());
  if (p == std::string::npos) return false;
  const char *s = js.c_str() + p + 1;
  char *end = nullptr;
  double d = std::strtod(s, &end);
  if (end == s) return false;
  *v = d;
  return true;
}

// Buffered little-endian writer over FILE*, errors sticky.
struct Out {
  FILE *f = nullptr;
  bool ok = true;
  void bytes(const void *p, size_t n) {
    if (ok && n && std::fwrite(p, 1, n, f) != n) ok = false;
  }
  void u32(uint32_t v) { bytes(&v, 4); }
  void u64(uint64_t v) { bytes(&v, 8); }
  void str(const std::string &s) {
    u32((uint32_t)s.size());
    bytes(s.data(), s.size());
  }
};

struct DevMem {
  void *p = nullptr;
  ~DevMem() {
    if (p) (void)hipFree(p);
  }
  bool alloc(size_t n, std::string *err) {
    hipError_t e = hipMalloc(&p, n ? n : 1);
    if (e == hipSuccess) return true;
    p = nullptr;
    return fail(err, std::string("hipMalloc failed: ") + hipGetErrorString(e));
  }
};

bool hip_ok(hipError_t e, const char *what, std::string *err) {
  return e == hipSuccess || fail(err, std::string(what) + ": " + hipGetErrorString(e));
}

std::string config_json(const ModelConfig &c) {
  char buf[512];
  std::snprintf(buf, sizeof(buf),
                "{\"layout\": \"t16\", \"t16_version\": %u, \"dim\": %u, \"num_heads\": %u, \"num_heads_kv\": %u, "
                "\"num_layers\": %u, \"vocab_size\": %u, \"hidden_dim\": %u, \"head_dim\": %u, "
                "\"max_seq_len\": %u, \"rope_base\": %.9g, \"rms_eps\": %.9g}",
                kGretaT16Version, c.dim, c.num_heads, c.num_heads_kv, c.num_layers, c.vocab_size, c.hidden_dim,
                c.head_dim, c.max_seq_len, (double)c.rope_base, (double)c.rms_eps);
  return buf;
}

}  // namespace

int greta_dtype_of_fmt(int fmt) {
  switch (fmt) {
  case GQ_FMT_Q4_0: return (int)GretaDataType::Q4_0;
  case GQ_FMT_Q8_0: return (int)GretaDataType::Q8_0;
  case GQ_FMT_Q4_K: return (int)GretaDataType::Q4_K;
  case GQ_FMT_Q4_K_GGML: return (int)GretaDataType::Q4_K_GGML;
  case GQ_FMT_Q6_K: return (int)GretaDataType::Q6_K;
  case GQ_FMT_Q6_K_GGML: return (int)GretaDataType::Q6_K_GGML;
  default: return -1;
  }
}

int greta_fmt_of_dtype(uint32_t d) {
  switch ((GretaDataType)d) {
  case GretaDataType::Q4_0: return GQ_FMT_Q4_0;
  case GretaDataType::Q8_0: return GQ_FMT_Q8_0;
  case GretaDataType::Q4_K: return GQ_FMT_Q4_K;
  case GretaDataType::Q4_K_GGML: return GQ_FMT_Q4_K_GGML;
  case GretaDataType::Q6_K: return GQ_FMT_Q6_K;
  case GretaDataType::Q6_K_GGML: return GQ_FMT_Q6_K_GGML;
  default: return -1;
  }
}

// ---- writer ------------------------------------------------------------------

bool write_greta(GGUFLoader &gguf, const std::string &path, GretaWriteKind kind, size_t *written,
                 std::string *err) {
  if (written) *written = 0;
  const std::string tmp = path + ".tmp";
  Out o;
  o.f = std::fopen(tmp.c_str(), "wb");
  if (!o.f) return fail(err, "cannot create " + tmp);
  auto abort_write = [&](const std::string &m) {
    std::fclose(o.f);
    std::remove(tmp.c_str());
    return fail(err, m);
  };

  o.bytes(kMagic, 8);
  // the reference tool writes an empty config; T16 files carry theirs
  o.str(kind == GretaWriteKind::INT4 ? std::string("{}") : config_json(gguf.get_config()));
  const long count_pos = std::ftell(o.f);
  o.u32(0);  // patched below

  uint32_t n = 0;
  std::vector<uint8_t> raw, packed, w, s, h;
  for (const TensorInfo &t : gguf.list_tensors()) {
    // the reference converts every tensor whose name holds ".weight"
    if (t.name.find(".weight") == std::string::npos) continue;
    std::string e;
    GGUFLoader::LoadPlan p;
    uint32_t dtype = 0, group = 0, heads = 0;
    if (kind == GretaWriteKind::T16) {
      if (!gguf.plan(t.name, GGUFLoader::LoadKind::QUANT, &p, &e)) {
        std::cerr << "  - " << t.name << ": skipped (" << e << ")\n";
        continue;
      }
      if (!gguf.read_raw(t.name, raw, &e)) return abort_write(e);
      packed.resize(p.bytes);
      const int st = gq_repack_host(p.fmt, raw.data(), p.N, p.K, packed.data());
      if (st != GQ_OK) return abort_write(t.name + ": repack: " + gq_status_string(st));
      dtype = (uint32_t)p.type;
      group = (p.fmt == GQ_FMT_Q4_0 || p.fmt == GQ_FMT_Q8_0) ? 32 : 256;
      w.swap(packed);
      s.clear();
      h.clear();
    } else {
      if (!gguf.plan(t.name, GGUFLoader::LoadKind::INT4, &p, &e)) {
        std::cerr << "  - " << t.name << ": Failed: " << e << "\n";
        continue;
      }
      DevMem dw, ds, dh;
      if (!dw.alloc(p.bytes, &e) || !ds.alloc(p.scale_bytes, &e) ||
          (p.has_head_scales && !dh.alloc((size_t)p.num_heads * 4, &e)))
        return abort_write(e);
      if (!gguf.load_into(t.name, GGUFLoader::LoadKind::INT4, p, dw.p, ds.p, p.has_head_scales ? dh.p : nullptr,
                          &e)) {
        std::cerr << "  - " << t.name << ": Failed: " << e << "\n";
        continue;
      }
      w.resize(p.bytes);
      s.resize(p.scale_bytes);
      h.resize(p.has_head_scales ? (size_t)p.num_heads * 4 : 0);
      if (!hip_ok(hipMemcpy(w.data(), dw.p, w.size(), hipMemcpyDeviceToHost), "hipMemcpy", &e) ||
          !hip_ok(hipMemcpy(s.data(), ds.p, s.size(), hipMemcpyDeviceToHost), "hipMemcpy", &e) ||
          (h.size() && !hip_ok(hipMemcpy(h.data(), dh.p, h.size(), hipMemcpyDeviceToHost), "hipMemcpy", &e)))
        return abort_write(e);
      dtype = (uint32_t)GretaDataType::INT4;
      group = 32;
      heads = p.is_qkv ? p.num_heads : 0;
    }
    o.str(t.name);
    o.u32(dtype);
    o.u32((uint32_t)t.shape.size());
    for (size_t d : t.shape) o.u64((uint64_t)d);
    o.u32(group);
    o.u32(heads);
    o.u64(w.size());
    o.u64(s.size());
    o.u64(h.size());
    o.bytes(w.data(), w.size());
    o.bytes(s.data(), s.size());
    o.bytes(h.data(), h.size());
    if (!o.ok) return abort_write("write failed: " + tmp);
    ++n;
  }
  if (std::fseek(o.f, count_pos, SEEK_SET) != 0) return abort_write("seek failed: " + tmp);
  o.u32(n);
  if (!o.ok || std::fclose(o.f) != 0) {
    std::remove(tmp.c_str());
    return fail(err, "write failed: " + tmp);
  }
  if (std::rename(tmp.c_str(), path.c_str()) != 0) {
    std::remove(tmp.c_str());
    return fail(err, "cannot rename " + tmp + " to " + path);
  }
  if (written) *written = n;
  return true;
}

// ---- reader ------------------------------------------------------------------

struct GretaLoader::Impl {
  int fd = -1;
  const uint8_t *map = nullptr;
  size_t size = 0;
  std::string json;
  std::vector<GretaRecord> recs;
  ModelConfig config;
  std::unique_ptr<Uploader> up;

  ~Impl() { close(); }
  void close() {
    if (map) munmap(const_cast<uint8_t *>(map), size);
    if (fd >= 0) ::close(fd);
    map = nullptr;
    fd = -1;
    size = 0;
    recs.clear();
  }
  Uploader &uploader() {
    if (!up) up = std::make_unique<Uploader>();
    up->bind_file(fd, map, size);  // slices of the mapping are read with pread
    return *up;
  }
  const GretaRecord *find(const std::string &name) const {
    for (const auto &r : recs)
      if (r.name == name) return &r;
    return nullptr;
  }

  bool parse(std::string *err) {
    size_t pos = 0;
    auto take = [&](void *dst, size_t n) {
      if (n > size - pos) return false;
      std::memcpy(dst, map + pos, n);
      pos += n;
      return true;
    };
    auto skip = [&](uint64_t n, uint64_t *at) {
      if (n > size - pos) return false;
      *at = pos;
      pos += (size_t)n;
      return true;
    };
    char magic[8];
    if (!take(magic, 8) || std::memcmp(magic, kMagic, 8) != 0) return fail(err, "not a .greta file");
    uint32_t jl;
    if (!take(&jl, 4) || jl > size - pos) return fail(err, ".greta: truncated config");
    json.assign((const char *)map + pos, jl);
    pos += jl;
    uint32_t n;
    if (!take(&n, 4)) return fail(err, ".greta: truncated header");
    // every record takes at least 4 + 4 + 4 + 8 + 24 bytes
    if (n > (size - pos) / 44) return fail(err, ".greta: bad tensor count");
    recs.reserve(n);
    for (uint32_t i = 0; i < n; ++i) {
      GretaRecord r;
      uint32_t nl, rank;
      if (!take(&nl, 4) || nl > 65536 || nl > size - pos) return fail(err, ".greta: bad tensor name");
      r.name.assign((const char *)map + pos, nl);
      pos += nl;
      if (!take(&r.dtype, 4) || !take(&rank, 4) || rank > 8) return fail(err, ".greta: bad record " + r.name);
      r.shape.resize(rank);
      for (uint32_t d = 0; d < rank; ++d)
        if (!take(&r.shape[d], 8)) return fail(err, ".greta: truncated shape of " + r.name);
      if (!take(&r.group_size, 4) || !take(&r.num_heads, 4) || !take(&r.w_size, 8) || !take(&r.s_size, 8) ||
          !take(&r.h_size, 8))
        return fail(err, ".greta: truncated record " + r.name);
      if (!skip(r.w_size, &r.w_off) || !skip(r.s_size, &r.s_off) || !skip(r.h_size, &r.h_off))
        return fail(err, ".greta: data of " + r.name + " outside the file");
      recs.push_back(std::move(r));
    }
    return true;
  }

  bool check_t16(std::string *err) const {
    bool any = false;
    for (const auto &r : recs) any |= greta_fmt_of_dtype(r.dtype) >= 0;
    if (!any) return true;
    double v = 0;
    if (!json_number(json, "t16_version", &v) || v != (double)kGretaT16Version)
      return fail(err, ".greta: T16 records of another layout version (this build reads version " +
                           std::to_string(kGretaT16Version) + ")");
    // each T16 record must hold exactly the tiles of its shape
    for (const auto &r : recs) {
      const int fmt = greta_fmt_of_dtype(r.dtype);
      if (fmt < 0) continue;
      if (r.shape.empty() || r.shape[0] == 0) return fail(err, ".greta: bad shape of " + r.name);
      uint64_t n = 1;
      for (uint64_t d : r.shape) n *= d;
      size_t bytes = 0;
      if (gq_packed_size(fmt, n / r.shape[0], r.shape[0], &bytes) != GQ_OK || bytes != r.w_size)
        return fail(err, ".greta: size of " + r.name + " does not match its shape");
    }
    return true;
  }
};

GretaLoader::GretaLoader() : impl_(std::make_unique<Impl>()) {}
GretaLoader::~GretaLoader() = default;

bool GretaLoader::open(const std::string &path, std::string *err) {
  Impl &m = *impl_;
  m.close();
  m.fd = ::open(path.c_str(), O_RDONLY);
  if (m.fd < 0) return fail(err, "cannot open " + path);
  struct stat st;
  if (fstat(m.fd, &st) != 0) return fail(err, "cannot stat " + path);
  m.size = (size_t)st.st_size;
  if (m.size == 0) return fail(err, "not a .greta file");
  void *p = mmap(nullptr, m.size, PROT_READ, MAP_PRIVATE, m.fd, 0);
  if (p == MAP_FAILED) return fail(err, "mmap failed for " + path);
  m.map = (const uint8_t *)p;
  if (!m.parse(err) || !m.check_t16(err)) {
    m.close();
    return false;
  }
  m.config = ModelConfig::llama2_7b();
  double v;
  ModelConfig &c = m.config;
  if (json_number(m.json, "dim", &v)) c.dim = (uint32_t)v;
  if (json_number(m.json, "num_heads", &v)) c.num_heads = (uint32_t)v;
  if (json_number(m.json, "num_heads_kv", &v)) c.num_heads_kv = (uint32_t)v;
  if (json_number(m.json, "num_layers", &v)) c.num_layers = (uint32_t)v;
  if (json_number(m.json, "vocab_size", &v)) c.vocab_size = (uint32_t)v;
  if (json_number(m.json, "hidden_dim", &v)) c.hidden_dim = (uint32_t)v;
  if (json_number(m.json, "head_dim", &v)) c.head_dim = (uint32_t)v;
  if (json_number(m.json, "max_seq_len", &v)) c.max_seq_len = (uint32_t)v;
  if (json_number(m.json, "rope_base", &v)) c.rope_base = (float)v;
  if (json_number(m.json, "rms_eps", &v)) c.rms_eps = (float)v;
  return true;
}

const std::vector<GretaRecord> &GretaLoader::records() const { return impl_->recs; }

std::vector<TensorInfo> GretaLoader::list_tensors() const {
  std::vector<TensorInfo> out;
  for (const auto &r : impl_->recs) {
    TensorInfo t;
    t.name = r.name;
    for (uint64_t d : r.shape) t.shape.push_back((size_t)d);
    t.offset = (size_t)r.w_off;
    t.size_bytes = (size_t)r.w_size;
    t.dtype = dtype_name(r.dtype);
    out.push_back(std::move(t));
  }
  return out;
}

ModelConfig GretaLoader::get_config() const { return impl_->config; }

bool GretaLoader::load_into(const std::string &name, void *w, size_t w_cap, void *s, size_t s_cap, void *h,
                            size_t h_cap, std::string *err) const {
  const GretaRecord *r = impl_->find(name);
  if (!r) return fail(err, "tensor not found: " + name);
  if (!w || w_cap < r->w_size || (r->s_size && (!s || s_cap < r->s_size)) ||
      (r->h_size && (!h || h_cap < r->h_size)))
    return fail(err, "load_into: destination missing or too small for " + name);
  Uploader &u = impl_->uploader();
  const uint8_t *base = impl_->map;
  return u.copy(w, base + r->w_off, r->w_size, err) && (!r->s_size || u.copy(s, base + r->s_off, r->s_size, err)) &&
         (!r->h_size || u.copy(h, base + r->h_off, r->h_size, err));
}

bool GretaLoader::load_tensor_quant(const std::string &name, gcore::rt::hip::Buffer &packed, std::string *err) {
  const GretaRecord *r = impl_->find(name);
  if (!r) return fail(err, "tensor not found: " + name);
  const int fmt = greta_fmt_of_dtype(r->dtype);
  if (fmt < 0)
    return fail(err, "load_tensor_quant: " + name + " is " + dtype_name(r->dtype) + " (a T16 record expected)");
  if (!packed.allocate(r->w_size, gcore::rt::hip::BufferUsage::DeviceOnly, (GretaDataType)r->dtype, err))
    return false;
  if (!load_into(name, packed.data(), r->w_size, nullptr, 0, nullptr, 0, err)) return false;
  gcore::rt::GretaQuantInfo q;
  q.group_size = r->group_size;
  q.format = (uint32_t)fmt;
  packed.set_quant_info(q);
  return true;
}

bool GretaLoader::load_tensor_int4(const std::string &name, gcore::rt::hip::Buffer &buffer,
                                   gcore::rt::hip::Buffer &scales, gcore::rt::hip::Buffer &head_scales,
                                   std::string *err) {
  const GretaRecord *r = impl_->find(name);
  if (!r) return fail(err, "tensor not found: " + name);
  if (r->dtype != (uint32_t)GretaDataType::INT4)
    return fail(err, "load_tensor_int4: " + name + " is " + dtype_name(r->dtype) + " (an INT4 record expected)");
  using gcore::rt::hip::BufferUsage;
  if (!buffer.allocate(r->w_size, BufferUsage::DeviceOnly, GretaDataType::INT4, err) ||
      !scales.allocate(r->s_size, BufferUsage::DeviceOnly, GretaDataType::FP32, err) ||
      (r->h_size && !head_scales.allocate(r->h_size, BufferUsage::DeviceOnly, GretaDataType::FP32, err)))
    return false;
  if (!load_into(name, buffer.data(), r->w_size, scales.data(), r->s_size, r->h_size ? head_scales.data() : nullptr,
                 r->h_size, err))
    return false;
  gcore::rt::GretaQuantInfo q;
  q.group_size = r->group_size;
  q.scales = scales.data();
  q.head_scales = r->num_heads && r->h_size ? head_scales.data() : nullptr;
  q.num_heads = r->num_heads;
  buffer.set_quant_info(q);
  return true;
}

bool GretaLoader::load_tensor(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) {
  const GretaRecord *r = impl_->find(name);
  if (!r) return fail(err, "tensor not found: " + name);
  const int fmt = greta_fmt_of_dtype(r->dtype);
  if (fmt < 0) return fail(err, "load_tensor: " + name + " is an " + dtype_name(r->dtype) + " record (no fp32 form)");
  uint64_t n = 1;
  for (uint64_t d : r->shape) n *= d;
  const size_t K = (size_t)r->shape[0], N = (size_t)(n / K);
  DevMem t16;
  if (!t16.alloc(r->w_size, err) || !load_into(name, t16.p, r->w_size, nullptr, 0, nullptr, 0, err)) return false;
  if (!buffer.allocate(n * 4, gcore::rt::hip::BufferUsage::DeviceOnly, GretaDataType::FP32, err)) return false;
  const int st = gq_dequant_packed(fmt, t16.p, N, K, (float *)buffer.data(), nullptr);
  if (st != GQ_OK) return fail(err, std::string("dequant: ") + gq_status_string(st));
  return hip_ok(hipStreamSynchronize(nullptr), "dequant", err);
}

bool GretaLoader::load_tensor_fp16(const std::string &name, gcore::rt::hip::Buffer &, std::string *err) {
  return fail(err, "load_tensor_fp16: a .greta file holds T16 and INT4 records only (" + name + ")");
}

bool GretaLoader::load_tensor_int8(const std::string &name, gcore::rt::hip::Buffer &, gcore::rt::hip::Buffer &,
                                   std::string *err) {
  return fail(err, "load_tensor_int8: a .greta file holds T16 and INT4 records only (" + name + ")");
}

}  // namespace gcore::inference
