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

// ---- Buffer ------------------------------------------------------------------
// Same contract as the reference's Buffer (src/rt/backend/hip/src/buffer.cpp):
// owns one allocation (device memory, or pinned host memory for HostVisible),
// re-allocation releases the old one first, copies are synchronous and
// bounds-checked.  Every copy goes through one checked helper; the status
// text names the operation, the byte range and the HIP error.
namespace {

// [offset, offset + bytes) inside a buffer of `capacity` bytes, without
// overflow in the sum.
bool range_inside(size_t offset, size_t bytes, size_t capacity) {
  return offset <= capacity && bytes <= capacity - offset;
}

bool report(std::string *err, const std::string &what) {
  if (err) *err = what;
  return false;
}

bool checked_copy(void *dst, const void *src, size_t bytes, hipMemcpyKind kind, const char *op, std::string *err) {
  if (bytes == 0) return true;
  const hipError_t e = hipMemcpy(dst, src, bytes, kind);
  if (e == hipSuccess) return true;
  return report(err, std::string("Buffer::") + op + ": " + std::to_string(bytes) + "-byte copy: " +
                         hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

}  // namespace

Buffer::~Buffer() { free(); }

bool Buffer::allocate(size_t size, BufferUsage usage, GretaDataType type, std::string *err) {
  free();
  void *p = nullptr;
  const hipError_t e = usage == BufferUsage::HostVisible ? hipHostMalloc(&p, size) : hipMalloc(&p, size);
  if (e != hipSuccess)
    return report(err, std::string("Buffer::allocate: ") + std::to_string(size) + " bytes of " +
                           (usage == BufferUsage::HostVisible ? "pinned host" : "device") + " memory: " +
                           hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
  ptr_ = p;
  size_ = size;
  usage_ = usage;
  type_ = type;
  qinfo_ = GretaQuantInfo{};
  return true;
}

void Buffer::free() {
  void *p = ptr_;
  ptr_ = nullptr;
  size_ = 0;
  if (!p) return;
  if (usage_ == BufferUsage::HostVisible) (void)hipHostFree(p);
  else (void)hipFree(p);
}

bool Buffer::copy_to_device(const void *host_ptr, size_t size, std::string *err) {
  if (!range_inside(0, size, size_))
    return report(err, "Buffer::copy_to_device: " + std::to_string(size) + " bytes do not fit the " +
                           std::to_string(size_) + "-byte buffer");
  return checked_copy(ptr_, host_ptr, size, hipMemcpyHostToDevice, "copy_to_device", err);
}

bool Buffer::copy_to_host(void *host_ptr, size_t size, std::string *err) const {
  return copy_to_host_offset(host_ptr, 0, size, err);
}

bool Buffer::copy_to_host_offset(void *host_ptr, size_t offset, size_t size, std::string *err) const {
  if (!range_inside(offset, size, size_))
    return report(err, "Buffer::copy_to_host: bytes [" + std::to_string(offset) + ", " +
                           std::to_string(offset) + " + " + std::to_string(size) + ") outside the " +
                           std::to_string(size_) + "-byte buffer");
  return checked_copy(host_ptr, static_cast<const char *>(ptr_) + offset, size, hipMemcpyDeviceToHost,
                      "copy_to_host", err);
}

}  // namespace gcore::rt::hip
