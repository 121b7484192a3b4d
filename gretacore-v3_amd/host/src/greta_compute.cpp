// GretaCompute::gemm for the quantized-weight matrix path.
//
// Routing restated from src/compute/src/greta_compute_hip.cpp:148-374:
//   * lda = K, ldb = N, ldc = N are implied; transpose_A / transpose_B /
//     accum_type are accepted and ignored, as in the reference.
//   * B INT8 -> the INT8 weight-only launcher (:305-311).
//   * B INT4 -> the INT4 launcher (:312-360) with head_dim = N / num_heads, the
//     per-head scales unless GRETA_PERHEAD_QKV is set to something other than
//     "1" (:161-163), and force_gemv from the op label and the GRETA_PREFILL_* /
//     GRETA_WO_LAYOUT_FORCE flags (:316-352).
//   * B GGUF-native (Q4_0 / Q8_0 / Q4_K / Q4_K_GGML / Q6_K / Q6_K_GGML, T16 layout) -> gq_matmul:
//     GEMV kernels for M <= 16, gq_gemm above (added by this library).
// Unlike the reference (which always returns SUCCESS), launch failures and
// unsupported operands are reported.
#include "gcore/compute/greta_compute.hpp"

#include <cstdlib>
#include <cstring>
#include <string>

#include "gq.h"
#include "gcore/rt/hip/greta_runtime_hip.hpp"

namespace {

std::string &current_op_label() {
  static std::string label;
  return label;
}
gcore::compute::GemmAuditInfo &last_audit() {
  static gcore::compute::GemmAuditInfo info;
  return info;
}

bool env_flag(const char *k) {
  const char *v = std::getenv(k);
  return v && (v[0] == '1' || v[0] == 'y' || v[0] == 'Y');
}
bool env_is(const char *k, const char *a, const char *b) {
  const char *v = std::getenv(k);
  return v && *v && (std::strcmp(v, a) == 0 || std::strcmp(v, b) == 0);
}

// force_gemv of the INT4 route (greta_compute_hip.cpp:316-352)
bool int4_force_gemv(const std::string &label) {
  const bool qkv_row = env_is("GRETA_PREFILL_QKV_LAYOUT", "row", "ROW");
  bool force = false;
  if (label == "attn_q_prefill" && (env_flag("GRETA_PREFILL_FORCE_WQ_ROW") || qkv_row)) force = true;
  if (label == "attn_k_prefill" && (env_flag("GRETA_PREFILL_FORCE_WK_ROW") || qkv_row)) force = true;
  if (label == "attn_v_prefill") {
    if (env_is("GRETA_PREFILL_FORCE_WV_LAYOUT", "row", "ROW")) force = true;
    else if (!env_is("GRETA_PREFILL_FORCE_WV_LAYOUT", "col", "COL") &&
             !env_is("GRETA_PREFILL_FORCE_WV_LAYOUT", "auto", "AUTO") && env_flag("GRETA_PREFILL_FORCE_WV_ROW"))
      force = true;
  }
  if (label == "attn_o_prefill" && qkv_row) force = true;
  if (label == "attn_o_prefill" || label == "attn_o_decode") {
    if (env_is("GRETA_WO_LAYOUT_FORCE", "row", "ROW")) force = true;
    else if (env_is("GRETA_WO_LAYOUT_FORCE", "col", "COL")) force = false;
  }
  return force;
}

int gguf_format(const gcore::rt::GretaMemory *B) {
  using gcore::rt::GretaDataType;
  const uint32_t f = B->quant_info().format;
  if (f) return (int)f;
  switch (B->data_type()) {
  case GretaDataType::Q4_0: return GQ_FMT_Q4_0;
  case GretaDataType::Q8_0: return GQ_FMT_Q8_0;
  case GretaDataType::Q4_K: return GQ_FMT_Q4_K;
  case GretaDataType::Q4_K_GGML: return GQ_FMT_Q4_K_GGML;
  case GretaDataType::Q6_K: return GQ_FMT_Q6_K;
  case GretaDataType::Q6_K_GGML: return GQ_FMT_Q6_K_GGML;
  default: return 0;
  }
}

}  // namespace

namespace gcore::compute {

GretaResult GretaCompute::gemm(GretaStream *stream, GretaMemory *A, GretaMemory *B, GretaMemory *C, uint32_t M,
                               uint32_t N, uint32_t K, bool transpose_A, bool transpose_B,
                               GretaDataType accum_type) {
  (void)transpose_A;
  (void)transpose_B;
  (void)accum_type;
  if (!A || !B || !C) return GretaResult::ERROR_INVALID_ARGS;
  if (M == 0 || N == 0 || K == 0) return GretaResult::SUCCESS;
  hipStream_t s = stream ? static_cast<gcore::rt::hip::GretaStreamHip *>(stream)->handle() : nullptr;
  const std::string label = current_op_label();
  GemmAuditInfo &audit = last_audit();
  audit = GemmAuditInfo{};
  audit.op_label = label;
  audit.type_a = (int)A->data_type();
  audit.type_b = (int)B->data_type();
  audit.m = M;
  audit.n = N;
  audit.k = K;
  const GretaQuantInfo q = B->quant_info();
  int st = GQ_OK;

  switch (B->data_type()) {
  case GretaDataType::INT8: {
    if (A->data_type() != GretaDataType::FP32) return GretaResult::ERROR_INVALID_ARGS;
    audit.quant_mode = "INT8";
    audit.route = M <= 32 ? "GEMV" : "GEMM";
    st = gq_launch_gemm_mfma_int8_wt_fp32_acc32(s, static_cast<const float *>(A->data()),
                                                static_cast<const int8_t *>(B->data()),
                                                static_cast<float *>(C->data()),
                                                static_cast<const float *>(q.scales), M, N, K, K, N, N,
                                                q.group_size);
    break;
  }
  case GretaDataType::INT4: {
    const bool fp16_a = A->data_type() == GretaDataType::FP16;
    if (!fp16_a && A->data_type() != GretaDataType::FP32) return GretaResult::ERROR_INVALID_ARGS;
    const char *ph = std::getenv("GRETA_PERHEAD_QKV");
    const bool perhead = ph == nullptr || std::string(ph) == "1";
    const uint32_t head_dim = q.num_heads > 0 ? N / q.num_heads : 0;
    const bool force_gemv = int4_force_gemv(label);
    audit.quant_mode = "INT4";
    audit.perhead_enabled = perhead;
    audit.force_gemv = force_gemv;
    audit.route = (force_gemv || M <= 32) ? "GEMV" : "GEMM";
    st = gq_launch_gemm_mfma_int4_wt_fp32_acc32(
        s, A->data(), static_cast<const int8_t *>(B->data()), static_cast<float *>(C->data()),
        static_cast<const float *>(q.scales), perhead ? static_cast<const float *>(q.head_scales) : nullptr, M, N,
        K, K, N, N, q.group_size, head_dim, fp16_a ? 1 : 0, force_gemv ? 1 : 0);
    break;
  }
  case GretaDataType::Q4_0:
  case GretaDataType::Q8_0:
  case GretaDataType::Q4_K:
  case GretaDataType::Q4_K_GGML:
  case GretaDataType::Q6_K:
  case GretaDataType::Q6_K_GGML: {
    const int fmt = gguf_format(B);
    size_t need = 0;
    if (gq_packed_size(fmt, N, K, &need) != GQ_OK || B->size() < need) return GretaResult::ERROR_INVALID_ARGS;
    audit.quant_mode = "GGUF";
    if (M <= GQ_MAX_BATCH) {
      if (A->data_type() != GretaDataType::FP32) return GretaResult::ERROR_INVALID_ARGS;
      audit.route = "GEMV";
      st = gq_gemv(fmt, B->data(), static_cast<const float *>(A->data()), static_cast<float *>(C->data()), N, K,
                   (int)M, nullptr, 0, s);
    } else {
      int adt;
      switch (A->data_type()) {
      case GretaDataType::FP32: adt = GQ_DT_F32; break;
      case GretaDataType::FP16: adt = GQ_DT_F16; break;
      case GretaDataType::BF16: adt = GQ_DT_BF16; break;
      default: return GretaResult::ERROR_INVALID_ARGS;
      }
      if (fmt == GQ_FMT_Q6_K || fmt == GQ_FMT_Q6_K_GGML) {
        // gq_matmul: the skinny GEMM (K <= 4096), else GEMVs over 16-row
        // batches (fp32 A)
        if (adt != GQ_DT_F32) return GretaResult::ERROR_INVALID_ARGS;
        audit.route = K <= 4096 ? "GEMM" : "GEMV";
        st = gq_matmul(fmt, B->data(), static_cast<const float *>(A->data()), static_cast<float *>(C->data()), M, N,
                       K, s);
        break;
      }
      audit.route = "GEMM";
      st = gq_gemm(fmt, B->data(), A->data(), adt, C->data(), GQ_DT_F32, M, N, K, nullptr, 0, s);
    }
    break;
  }
  case GretaDataType::FP16: {
    // the reference's FP16 route (greta_compute_hip.cpp:361-371): W is N x K
    // fp16, A fp32 (the reference reads A as float whatever its type); VALU
    // launcher for M <= 32 or an lm_head label, MFMA launcher above -- both
    // run gq_gemm_f16w here
    if (A->data_type() != GretaDataType::FP32) return GretaResult::ERROR_INVALID_ARGS;
    if (B->size() < (size_t)N * K * 2) return GretaResult::ERROR_INVALID_ARGS;
    // (the lm_head labels of greta_compute_hip.cpp:73-76 take the VALU route
    // unless GRETA_LMHEAD_FORCE_ROUTE asks otherwise; GRETA_GEMM_FORCE=MFMA|VALU
    // forces either, :174-184)
    bool valu = M <= 32;
    const bool lm = label == "lm_head" || label == "lm_head_prefill" || label == "lm_head_decode";
    const char *ff = std::getenv("GRETA_GEMM_FORCE");
    if (ff && std::string(ff) == "MFMA") valu = false;
    if (ff && std::string(ff) == "VALU") valu = true;
    const char *lf = std::getenv("GRETA_LMHEAD_FORCE_ROUTE");
    if (lm) valu = !(lf && (std::string(lf) == "mfma" || std::string(lf) == "MFMA"));
    audit.quant_mode = "FP16";
    audit.route = valu ? "VALU" : "MFMA";
    st = valu ? gq_launch_gemm_mixed_f16f32(s, static_cast<const float *>(A->data()), B->data(),
                                            static_cast<float *>(C->data()), M, N, K, K, N, N)
              : gq_launch_gemm_mfma_mixed_f16f32(s, static_cast<const float *>(A->data()), B->data(),
                                                 static_cast<float *>(C->data()), M, N, K, K, N, N);
    break;
  }
  default:
    return GretaResult::ERROR_NOT_IMPLEMENTED;  // FP32 weights: the reference reads them as fp16 (a bug)
  }
  if (st == GQ_ERR_INVALID_ARGS || st == GQ_ERR_UNSUPPORTED) return GretaResult::ERROR_INVALID_ARGS;
  return st == GQ_OK ? GretaResult::SUCCESS : GretaResult::ERROR_KERNEL_LAUNCH;
}

void GretaCompute::set_op_label(const char *label) {
  if (label) current_op_label() = label;
  else current_op_label().clear();
}

GemmAuditInfo GretaCompute::get_last_gemm_audit() { return last_audit(); }

}  // namespace gcore::compute
