#pragma once
// Model configuration read from GGUF llama.* keys, with the reference's fields
// and Llama-2-7B defaults (src/inference/include/gcore/inference/model_config.hpp:11-36).
#include <cstdint>
#include <string>
#include <vector>

namespace gcore::inference {

struct ModelConfig {
  uint32_t dim = 4096;
  uint32_t num_heads = 32;
  uint32_t num_heads_kv = 32;
  uint32_t num_layers = 32;
  uint32_t vocab_size = 32000;
  uint32_t hidden_dim = 11008;
  uint32_t head_dim = 128;
  uint32_t max_seq_len = 2048;
  float rope_base = 10000.0f;
  float rms_eps = 1e-5f;
  std::vector<std::string> vocabulary;

  static ModelConfig llama2_7b() { return ModelConfig{}; }
};

}  // namespace gcore::inference
