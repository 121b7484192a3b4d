// HIP stream / event wrappers and Buffer (see the headers for the reference
// interfaces they mirror).
#include "gcore/rt/hip/greta_runtime_hip.hpp"

#include <hip/hip_runtime.h>

#include "gcore/rt/hip/buffer.hpp"

namespace gcore::rt::hip {

GretaEventHip::GretaEventHip() { (void)hipEventCreate(&event_); }
GretaEventHip::~GretaEventHip() {
  if (event_) (void)hipEventDestroy(event_);
}
void GretaEventHip::record(GretaStream *stream) {
  auto *s = static_cast<GretaStreamHip *>(stream);
  (void)hipEventRecord(event_, s ? s->handle() : nullptr);
}
float GretaEventHip::elapsed_time_since(GretaEvent *start) {
  float ms = 0.0f;
  (void)hipEventSynchronize(event_);
  (void)hipEventElapsedTime(&ms, static_cast<GretaEventHip *>(start)->handle(), event_);
  return ms;
}

GretaStreamHip::GretaStreamHip() : owned_(true) { (void)hipStreamCreate(&stream_); }
GretaStreamHip::GretaStreamHip(hipStream_t existing) : stream_(existing), owned_(false) {}
GretaStreamHip::~GretaStreamHip() {
  if (owned_ && stream_) (void)hipStreamDestroy(stream_);
}
void GretaStreamHip::synchronize() { (void)hipStreamSynchronize(stream_); }
void GretaStreamHip::wait_event(GretaEvent *event) {
  (void)hipStreamWaitEvent(stream_, static_cast<GretaEventHip *>(event)->handle(), 0);
}
void GretaStreamHip::record_event(GretaEvent *event) { event->record(this); }

// ---- Buffer (reference: src/rt/backend/hip/src/buffer.cpp:9-84) ----------
Buffer::~Buffer() { free(); }

bool Buffer::allocate(size_t size, BufferUsage usage, GretaDataType type, std::string *err) {
  free();
  usage_ = usage;
  type_ = type;
  qinfo_ = GretaQuantInfo{};
  hipError_t res = usage == BufferUsage::HostVisible ? hipHostMalloc(&ptr_, size) : hipMalloc(&ptr_, size);
  if (res != hipSuccess) {
    if (err) *err = "HIP allocation failed: " + std::string(hipGetErrorString(res));
    ptr_ = nullptr;
    size_ = 0;
    return false;
  }
  size_ = size;
  return true;
}

void Buffer::free() {
  if (ptr_) {
    if (usage_ == BufferUsage::HostVisible) (void)hipHostFree(ptr_);
    else (void)hipFree(ptr_);
  }
  ptr_ = nullptr;
  size_ = 0;
}

bool Buffer::copy_to_device(const void *host_ptr, size_t size, std::string *err) {
  if (size > size_) {
    if (err) *err = "copy_to_device: " + std::to_string(size) + " bytes into a " + std::to_string(size_) + "-byte buffer";
    return false;
  }
  hipError_t res = hipMemcpy(ptr_, host_ptr, size, hipMemcpyHostToDevice);
  if (res != hipSuccess) {
    if (err) *err = "hipMemcpy H2D failed: " + std::string(hipGetErrorString(res));
    return false;
  }
  return true;
}

bool Buffer::copy_to_host(void *host_ptr, size_t size, std::string *err) const {
  return copy_to_host_offset(host_ptr, 0, size, err);
}

bool Buffer::copy_to_host_offset(void *host_ptr, size_t offset, size_t size, std::string *err) const {
  if (offset + size > size_) {
    if (err)
      *err = "Buffer copy out of bounds: offset=" + std::to_string(offset) + ", size=" + std::to_string(size) +
             ", total_size=" + std::to_string(size_);
    return false;
  }
  hipError_t res = hipMemcpy(host_ptr, static_cast<char *>(ptr_) + offset, size, hipMemcpyDeviceToHost);
  if (res != hipSuccess) {
    if (err) *err = "hipMemcpy D2H failed: " + std::string(hipGetErrorString(res));
    return false;
  }
  return true;
}

}  // namespace gcore::rt::hip
