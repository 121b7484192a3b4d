#pragma once
// HIP stream / event wrappers with the reference's names
// (src/rt/backend/hip/include/gcore/rt/hip/greta_runtime_hip.hpp:37-70):
// GretaCompute::gemm takes the hipStream_t from GretaStreamHip::handle().
#include <hip/hip_runtime.h>

#include "gcore/rt/greta_runtime.hpp"

namespace gcore::rt::hip {

class GretaEventHip : public GretaEvent {
public:
  GretaEventHip();
  ~GretaEventHip() override;
  void record(GretaStream *stream) override;
  float elapsed_time_since(GretaEvent *start) override;
  hipEvent_t handle() const { return event_; }

private:
  hipEvent_t event_ = nullptr;
};

class GretaStreamHip : public GretaStream {
public:
  GretaStreamHip();                     // creates (and owns) a stream
  explicit GretaStreamHip(hipStream_t existing);  // wraps a caller's stream
  ~GretaStreamHip() override;
  void synchronize() override;
  void wait_event(GretaEvent *event) override;
  void record_event(GretaEvent *event) override;
  hipStream_t handle() const { return stream_; }

private:
  hipStream_t stream_ = nullptr;
  bool owned_ = false;
};

}  // namespace gcore::rt::hip
