#pragma once
// .greta weight files: the container of the reference's pre-quantization tool
// (tools/quantize/greta_quantize_gguf.cpp:40-124), written here and, unlike the
// reference (which has no reader), read back.
//
// Container (little-endian, no padding; the reference's layout):
//   "GRETA_W\0"                                    8 bytes
//   u32 json_len, json                             model config ("{}" in INT4 files)
//   u32 n_tensors
//   per tensor:
//     u32 name_len, name
//     u32 dtype                                    GretaDataType value
//     u32 rank, u64 dims[rank]                     GGUF order (dims[0] contiguous)
//     u32 group_size, u32 num_heads
//     u64 w_size, u64 s_size, u64 h_size
//     w_size bytes, s_size bytes, h_size bytes
//
// Two kinds of records:
//  * INT4 (dtype 4): load_tensor_int4's packed codes, fp32 scales and head
//    scales -- what the reference tool writes, byte for byte;
//  * T16 (dtype Q4_0 / Q8_0 / Q4_K / Q4_K_GGML / Q6_K / Q6_K_GGML): the tiled
//    layout the GEMV / GEMM kernels stream, so a load is one upload with no
//    repack.  A file of T16 records carries {"layout": "t16", "t16_version": 1,
//    ...config} as its json, and a reader refuses any other t16_version.
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "gcore/inference/weight_loader.hpp"

namespace gcore::inference {

constexpr uint32_t kGretaT16Version = 1;

struct GretaRecord {
  std::string name;
  uint32_t dtype = 0;  // GretaDataType
  std::vector<uint64_t> shape;
  uint32_t group_size = 0, num_heads = 0;
  uint64_t w_off = 0, w_size = 0, s_off = 0, s_size = 0, h_off = 0, h_size = 0;  // absolute file offsets
};

// Reads .greta files (memory-mapped, every length bounds-checked).
class GretaLoader : public WeightLoader {
public:
  GretaLoader();
  ~GretaLoader() override;

  bool open(const std::string &path, std::string *err) override;
  std::vector<TensorInfo> list_tensors() const override;
  // T16 records: dequantized to fp32 on the GPU (the GGUF values, bit-exact).
  bool load_tensor(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) override;
  // Not held by a .greta file (error).
  bool load_tensor_fp16(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) override;
  bool load_tensor_int8(const std::string &name, gcore::rt::hip::Buffer &buffer, gcore::rt::hip::Buffer &scales,
                        std::string *err) override;
  // INT4 records: the three stored arrays, quant_info as GGUFLoader sets it.
  bool load_tensor_int4(const std::string &name, gcore::rt::hip::Buffer &buffer, gcore::rt::hip::Buffer &scales,
                        gcore::rt::hip::Buffer &head_scales, std::string *err) override;
  // json config of a T16 file; the reference defaults (llama2_7b) otherwise.
  ModelConfig get_config() const override;

  // T16 records: one upload of the stored tiles (no repack); data_type() and
  // quant_info() as GGUFLoader::load_tensor_quant sets them.
  bool load_tensor_quant(const std::string &name, gcore::rt::hip::Buffer &packed, std::string *err);

  const std::vector<GretaRecord> &records() const;
  // Uploads a record's arrays into caller-owned device memory (each at least
  // the stored size; s / h may be null when the record has none).
  bool load_into(const std::string &name, void *w, size_t w_cap, void *s, size_t s_cap, void *h, size_t h_cap,
                 std::string *err) const;

private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

// GretaDataType of a T16 format id (GQ_FMT_*), -1 if none; and back.
int greta_dtype_of_fmt(int fmt);
int greta_fmt_of_dtype(uint32_t dtype);

enum class GretaWriteKind {
  INT4,  // the reference tool: every ".weight" tensor through load_tensor_int4 (needs the GPU)
  T16,   // every ".weight" tensor stored as Q4_0 / Q8_0 / Q4_K / Q6_K, repacked on the host (no GPU)
};

// Writes a .greta file from an open GGUF loader.  Tensors that cannot be
// converted are skipped with a note on stderr (as the reference tool does) and
// n_tensors counts the records actually written.  The file is written under a
// temporary name and renamed into place.
bool write_greta(GGUFLoader &gguf, const std::string &path, GretaWriteKind kind, size_t *written,
                 std::string *err);

}  // namespace gcore::inference
