#pragma once
// Runtime boundary types of the quantized-weight matrix path, with the names
// and meaning of the reference's L0 interface
// (src/rt/include/gcore/rt/greta_runtime.hpp:16-97).  Additions are appended
// only: enum values Q4_0 / Q8_0 / Q4_K_GGML / Q6_K / Q6_K_GGML for GGUF-native T16 weights and the
// `format` field of GretaQuantInfo (the GGML type id of such weights).
#include <cstddef>
#include <cstdint>

namespace gcore::rt {

#define GRETA_API_VERSION_MAJOR 0
#define GRETA_API_VERSION_MINOR 1

enum class GretaResult {
  SUCCESS = 0,
  ERROR_OUT_OF_MEM = 1,
  ERROR_GRAPH_CAPTURE = 2,
  ERROR_KERNEL_LAUNCH = 3,
  ERROR_INVALID_ARGS = 4,
  ERROR_NOT_IMPLEMENTED = 5
};

enum class GretaDataType {
  FP32 = 0,
  FP16 = 1,
  BF16 = 2,
  INT8 = 3,
  INT4 = 4,
  Q4_K = 5,  // GGUF-native Q4_K in the T16 layout (reference layout codes)
  FP8_E4M3 = 6,
  FP8_E5M2 = 7,
  // appended: GGUF-native blocks in the T16 layout
  Q4_0 = 8,
  Q8_0 = 9,
  Q4_K_GGML = 10,
  Q6_K = 11,
  Q6_K_GGML = 12,
};

struct GretaQuantInfo {
  const void *scales = nullptr;
  const void *head_scales = nullptr;
  float zero_point = 0.0f;
  uint32_t group_size = 0;  // 0 means per-tensor
  uint32_t num_heads = 0;
  uint32_t format = 0;  // appended: GGML type id of GGUF-native (T16) data, 0 otherwise
};

class GretaStream;

class GretaEvent {
public:
  virtual ~GretaEvent() = default;
  virtual void record(GretaStream *stream) = 0;
  virtual float elapsed_time_since(GretaEvent *start) = 0;
};

class GretaMemory {
public:
  virtual ~GretaMemory() = default;
  virtual void *data() = 0;
  virtual const void *data() const = 0;
  virtual size_t size() const = 0;  // total size in bytes
  virtual GretaDataType data_type() const = 0;
  virtual GretaQuantInfo quant_info() const = 0;
  virtual bool copy_from_host(const void *src, size_t size) = 0;
  virtual bool copy_to_host(void *dst, size_t size) const = 0;
};

class GretaStream {
public:
  virtual ~GretaStream() = default;
  virtual void synchronize() = 0;
  virtual void wait_event(GretaEvent *event) = 0;
  virtual void record_event(GretaEvent *event) = 0;
};

}  // namespace gcore::rt
