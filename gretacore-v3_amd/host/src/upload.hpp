#pragma once
// Host -> device upload pipeline of the weight loaders.
//
// The reference reads each tensor with ifstream into a std::vector and copies it
// with a synchronous pageable hipMemcpy (src/inference/src/weight_loader.cpp:
// 532-534, src/rt/backend/hip/src/buffer.cpp:45-53), so disk / page-cache
// reads, the driver's bounce copy and the DMA run one after another.  Here a
// tensor moves in slices through a ring of pinned staging buffers:
//
//   host threads: mmap slice j -> pinned slot j % S      (parallel memcpy)
//   stream:       pinned slot -> device (async DMA) -> optional repack kernel
//
// so the host copy of slice j + 1 overlaps the DMA (and repack) of slice j.
// A slot is reused only after the event recorded behind its last use has
// completed.  For GGUF-native tensors the DMA lands in a device slot and
// gq_repack_rows writes the slice's T16 tiles straight into the destination,
// so no whole-tensor raw copy is ever allocated on the device.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

namespace gcore::inference {

class Uploader {
public:
  Uploader();
  ~Uploader();
  Uploader(const Uploader &) = delete;
  Uploader &operator=(const Uploader &) = delete;

  // Copies `bytes` from host memory `src` (typically a file mapping) to device
  // memory `dst`.  Returns when the data is on the device.
  bool copy(void *dst, const void *src, size_t bytes, std::string *err);

  // Uploads the GGUF rows of an N x K tensor of format `fmt` (row_bytes each)
  // and repacks them into `packed` (gq_packed_size bytes), slice by slice.
  // Returns when the repack has finished.
  bool repack(int fmt, const uint8_t *src, size_t N, size_t K, size_t row_bytes, void *packed, std::string *err);

  // Slice size (bytes) and ring depth; GQ_LOAD_SLICE_MB, GQ_LOAD_SLOTS and
  // GQ_LOAD_THREADS override the defaults (32 MiB, 3, min(8, cores)).
  size_t slice_bytes() const { return slice_; }
  int slots() const { return nslots_; }
  int threads() const { return nthreads_; }

private:
  static constexpr int kMaxSlots = 8;
  struct Slot {
    void *host = nullptr;  // pinned (hipHostMalloc)
    void *dev = nullptr;   // device staging for repack slices
    size_t host_cap = 0, dev_cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
  };
  bool init(std::string *err);
  bool acquire(Slot &s, size_t bytes, bool need_dev, std::string *err);
  void host_copy(void *dst, const void *src, size_t bytes) const;
  bool copy_slices(void *dst, const void *src, size_t bytes, std::string *err);
  bool repack_slices(int fmt, const uint8_t *src, size_t N, size_t K, size_t row_bytes, void *packed,
                     std::string *err);
  bool drain_after_error();

  Slot slot_[kMaxSlots];
  hipStream_t stream_ = nullptr;
  size_t slice_ = 32u << 20;
  int nslots_ = 3;
  int nthreads_ = 1;
  bool ready_ = false;
};

}  // namespace gcore::inference
