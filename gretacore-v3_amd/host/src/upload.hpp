#pragma once
// Host -> device upload pipeline of the weight loaders.
//
// The reference reads each tensor with ifstream into a std::vector and copies it
// with a synchronous pageable hipMemcpy (src/inference/src/weight_loader.cpp:
// 532-534, src/rt/backend/hip/src/buffer.cpp:45-53), so disk / page-cache
// reads, the driver's bounce copy and the DMA run one after another.  Here a
// tensor moves in slices through a ring of pinned staging buffers:
//
//   host threads: file slice j -> pinned slot j % S      (parallel pread)
//   stream:       pinned slot -> device (async DMA) -> optional repack kernel
//
// so the host copy of slice j + 1 overlaps the DMA (and repack) of slice j.
// The host copy reads the file with pread() when the source lies in the
// loader's file mapping: copying out of the mapping instead would fault in
// every page of it once (a page-table fault per 4 KiB, ~27 GB/s on 8 threads
// on the MI355X boxes' hosts), where pread copies from the page cache with no
// user-space faults (58-80 GB/s on 4-16 threads, above the ~57 GB/s of the
// pinned H2D link).  Other sources are copied with memcpy.  The copy threads
// are a pool owned by the uploader.  One uploader serves one host thread at a
// time (its ring, stream and copy job are shared state), as the loaders that
// own one are used.
// A slot is reused only after the event recorded behind its last use has
// completed.  For GGUF-native tensors the DMA lands in a device slot and
// gq_repack_rows writes the slice's T16 tiles straight into the destination,
// so no whole-tensor raw copy is ever allocated on the device.
#include <hip/hip_runtime.h>

#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace gcore::inference {

class Uploader {
public:
  Uploader();
  ~Uploader();
  Uploader(const Uploader &) = delete;
  Uploader &operator=(const Uploader &) = delete;

  // The loader's file: its descriptor and its read-only mapping [base, base +
  // len).  Sources inside the mapping are then read with pread(fd) at their
  // offset.  fd < 0 unbinds (memcpy for every source).  The descriptor must
  // stay open while copies run.
  void bind_file(int fd, const void *base, size_t len);

  // Copies `bytes` from host memory `src` (typically a file mapping) to device
  // memory `dst`.  Returns when the data is on the device.
  bool copy(void *dst, const void *src, size_t bytes, std::string *err);

  // Uploads the GGUF rows of an N x K tensor of format `fmt` (row_bytes each)
  // and repacks them into `packed` (gq_packed_size bytes), slice by slice.
  // Returns when the repack has finished.
  bool repack(int fmt, const uint8_t *src, size_t N, size_t K, size_t row_bytes, void *packed, std::string *err);

  // Several tensors through the ring without waiting in between: the slices
  // of tensor i + 1 are read while those of tensor i are still in flight, so
  // the ring stays full across tensors.  Returns when every tensor has been
  // repacked; after a failure, when the work already queued has finished.
  struct RepackJob {
    int fmt;
    const uint8_t *src;
    size_t N, K, row_bytes;
    void *packed;
  };
  bool repack_many(const RepackJob *jobs, size_t n, std::string *err);

  // Slice size (bytes) and ring depth; GQ_LOAD_SLICE_MB, GQ_LOAD_SLOTS and
  // GQ_LOAD_THREADS override the defaults (16 MiB, 4, min(16, cores)).
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
  void host_copy(void *dst, const void *src, size_t bytes);
  void copy_part(int part);
  void worker();
  bool copy_slices(void *dst, const void *src, size_t bytes, std::string *err);
  bool repack_slices(int fmt, const uint8_t *src, size_t N, size_t K, size_t row_bytes, void *packed,
                     std::string *err);
  bool drain_after_error();

  Slot slot_[kMaxSlots];
  // bound file
  int fd_ = -1;
  const uint8_t *fbase_ = nullptr;
  size_t flen_ = 0;
  // copy pool: one job (dst, src, bytes cut into nparts_ parts of part_
  // bytes) at a time; the calling thread takes parts too
  std::vector<std::thread> pool_;
  std::mutex mu_;
  std::condition_variable cv_job_, cv_done_;
  int next_ = 0;        // next part to take (workers wait while next_ >= nparts_)
  int left_ = 0;        // parts not finished
  int nparts_ = 0;
  size_t part_ = 0, jbytes_ = 0;
  char *jdst_ = nullptr;
  const char *jsrc_ = nullptr;
  bool stop_ = false;
  hipStream_t stream_ = nullptr;
  size_t slice_ = 32u << 20;
  int nslots_ = 3;
  int nthreads_ = 1;
  bool ready_ = false;
};

}  // namespace gcore::inference
