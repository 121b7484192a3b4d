#pragma once
// GGUF weight loader with the reference's WeightLoader interface
// (src/inference/include/gcore/inference/weight_loader.hpp:24-86), plus
// load_tensor_quant: upload of GGUF-native blocks repacked on the GPU into the
// T16 layout the quantized GEMV/GEMM kernels stream.
//
// Differences from the reference, on purpose:
//  * the file is memory-mapped; every conversion (dequant, requant, GQA
//    transpose, head scales, repack) runs on the GPU and is bit-exact with the
//    reference's CPU loops;
//  * Q8_0 is named "Q8_0" (the reference reports "UNKNOWN" and then reads it as
//    F32, weight_loader.cpp:179-208, 719-720), and load_tensor_int8 uses the
//    intended Q8_0 semantics (:703-712);
//  * u64 / i64 integer values are accepted for the llama.* keys.
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "gcore/inference/model_config.hpp"
#include "gcore/rt/hip/buffer.hpp"

namespace gcore::inference {

struct TensorInfo {
  std::string name;
  std::vector<size_t> shape;  // GGUF order: shape[0] = ne0 (contiguous)
  size_t offset = 0;          // absolute file offset
  size_t size_bytes = 0;
  std::string dtype;          // "F32", "F16", "Q4_0", "Q8_0", "Q4_K", "Q6_K", "UNKNOWN"
};

class WeightLoader {
public:
  virtual ~WeightLoader() = default;
  virtual bool open(const std::string &path, std::string *err) = 0;
  virtual std::vector<TensorInfo> list_tensors() const = 0;
  virtual bool load_tensor(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) = 0;
  virtual bool load_tensor_fp16(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) = 0;
  virtual bool load_tensor_int8(const std::string &name, gcore::rt::hip::Buffer &buffer,
                                gcore::rt::hip::Buffer &scales, std::string *err) = 0;
  virtual bool load_tensor_int4(const std::string &name, gcore::rt::hip::Buffer &buffer,
                                gcore::rt::hip::Buffer &scales, gcore::rt::hip::Buffer &head_scales,
                                std::string *err) = 0;
  virtual ModelConfig get_config() const = 0;
};

class GGUFLoader : public WeightLoader {
public:
  GGUFLoader();
  ~GGUFLoader() override;

  bool open(const std::string &path, std::string *err) override;
  std::vector<TensorInfo> list_tensors() const override;
  bool load_tensor(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) override;
  bool load_tensor_fp16(const std::string &name, gcore::rt::hip::Buffer &buffer, std::string *err) override;
  bool load_tensor_int8(const std::string &name, gcore::rt::hip::Buffer &buffer, gcore::rt::hip::Buffer &scales,
                        std::string *err) override;
  bool load_tensor_int4(const std::string &name, gcore::rt::hip::Buffer &buffer, gcore::rt::hip::Buffer &scales,
                        gcore::rt::hip::Buffer &head_scales, std::string *err) override;
  ModelConfig get_config() const override;

  // GGUF-native upload: raw Q4_0 / Q8_0 / Q4_K blocks repacked on the GPU into
  // the T16 layout.  data_type() of the buffer becomes Q4_0 / Q8_0 / Q4_K (or
  // Q4_K_GGML), quant_info().format the GGML type id.  N = shape[1] rows,
  // K = shape[0].
  bool load_tensor_quant(const std::string &name, gcore::rt::hip::Buffer &packed, std::string *err);
  // k-quant code layouts of this file (Q4_K and Q6_K): false (default) = the
  // reference's layouts (weight_loader.cpp:125-177), true = llama.cpp's.
  // GQ_Q4K_LAYOUT=ggml in the environment sets true at open().
  void set_q4k_layout_ggml(bool ggml);
  // Raw tensor bytes (no GPU).
  bool read_raw(const std::string &name, std::vector<uint8_t> &out, std::string *err) const;
  // GGML type id of a tensor (-1 if absent).
  int ggml_type(const std::string &name) const;

  // Loads into caller-owned device memory (used by the Buffer methods above and
  // by the C ABI).  plan() gives the sizes; load_into() needs `out` of
  // plan.bytes, `scales` of plan.scale_bytes (INT8/INT4) and `head_scales` of
  // plan.num_heads floats when plan.has_head_scales.  Synchronous.
  enum class LoadKind { F32, F16, INT8, INT4, QUANT };
  struct LoadPlan {
    size_t n_elem = 0;
    size_t bytes = 0;
    size_t scale_bytes = 0;
    bool is_qkv = false;          // INT4: name holds attn_q / attn_k / attn_v
    bool has_head_scales = false; // INT4: is_qkv and num_heads, head_dim > 0
    uint32_t num_heads = 0;
    bool transpose = false;       // GQA K/V [D][KV] -> [KV][D]
    int fmt = 0;                  // QUANT: GQ_FMT_* of the T16 data
    size_t N = 0, K = 0;          // QUANT: rows, row length
    gcore::rt::GretaDataType type = gcore::rt::GretaDataType::FP32;
  };
  bool plan(const std::string &name, LoadKind kind, LoadPlan *plan, std::string *err) const;
  bool load_into(const std::string &name, LoadKind kind, const LoadPlan &plan, void *out, void *scales,
                 void *head_scales, std::string *err) const;
  // LoadKind::QUANT of several tensors in one pipelined pass (no counterpart
  // in the reference, which loads tensor by tensor): outs[i] holds at least
  // out_bytes[i] >= plan(names[i], QUANT).bytes.  Every name is planned and
  // checked before any data moves; returns when all tensors are on the
  // device.  After a failure during the transfer, tensors before the failing
  // one may be loaded and the rest not.
  bool load_quant_many(const std::string *names, void *const *outs, const size_t *out_bytes, size_t n,
                       std::string *err) const;

private:
  struct Impl;
  std::unique_ptr<Impl> impl_;
};

std::unique_ptr<WeightLoader> create_weight_loader(const std::string &path, std::string *err);

}  // namespace gcore::inference
