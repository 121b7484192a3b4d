#pragma once
// L1 op entry for the quantized-weight matrix path, with the reference's
// interface (src/compute/include/gcore/compute/greta_compute.hpp:49-72):
//   GretaCompute::gemm(stream, A, B, C, M, N, K, ...) dispatches on B's data
//   type: INT8 / INT4 (reference requantized formats) and, added here, the
//   GGUF-native T16 types Q4_0 / Q8_0 / Q4_K / Q4_K_GGML.
#include <cstdint>
#include <string>

#include "gcore/rt/greta_runtime.hpp"

namespace gcore::compute {

using namespace gcore::rt;

// Route record of the last gemm call (reference: greta_compute.hpp:14-40,
// kept to the fields this path fills).
struct GemmAuditInfo {
  std::string op_label;
  std::string route;  // "GEMV" or "GEMM"
  std::string quant_mode;
  int type_a = 0;
  int type_b = 0;
  uint32_t m = 0, n = 0, k = 0;
  bool perhead_enabled = false;
  bool force_gemv = false;
};

class GretaCompute {
public:
  // C[M][N] = A[M][K] * B^T with B stored as N rows of K (GGUF order).
  // A: FP32 (any B), or FP16 / BF16 for GGUF-native B with M > 16.  C: FP32.
  // Returns ERROR_INVALID_ARGS for null / mismatched operands,
  // ERROR_NOT_IMPLEMENTED for B types outside this path (FP16/FP32 weights),
  // ERROR_KERNEL_LAUNCH when a launch fails.
  static GretaResult gemm(GretaStream *stream, GretaMemory *A, GretaMemory *B, GretaMemory *C, uint32_t M,
                          uint32_t N, uint32_t K, bool transpose_A = false, bool transpose_B = false,
                          GretaDataType accum_type = GretaDataType::FP32);

  // Process-global label of the next gemm call (not thread-safe, as in the
  // reference: greta_compute_hip.cpp:421-427).
  static void set_op_label(const char *label);
  static GemmAuditInfo get_last_gemm_audit();
};

}  // namespace gcore::compute
