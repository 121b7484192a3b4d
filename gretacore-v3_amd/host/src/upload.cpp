// Pinned, sliced, overlapped host -> device uploads for the weight loaders.
#include "upload.hpp"

#include <errno.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "gq.h"

namespace gcore::inference {

namespace {
bool fail(std::string *err, const std::string &m) {
  if (err) *err = m;
  return false;
}
bool hip_ok(hipError_t e, const char *what, std::string *err) {
  return e == hipSuccess || fail(err, std::string(what) + ": " + hipGetErrorString(e));
}
long env_long(const char *name, long def, long lo, long hi) {
  const char *e = std::getenv(name);
  if (!e || !*e) return def;
  char *end = nullptr;
  long v = std::strtol(e, &end, 10);
  if (end == e) return def;
  return std::min(hi, std::max(lo, v));
}
// Asks the kernel to read a mapped range ahead (no-op for non-mapped memory).
void advise_willneed(const void *p, size_t bytes) {
  const long pg = sysconf(_SC_PAGESIZE);
  if (pg <= 0 || bytes == 0) return;
  uintptr_t a = (uintptr_t)p & ~(uintptr_t)(pg - 1);
  (void)madvise((void *)a, (uintptr_t)p + bytes - a, MADV_WILLNEED);
}
}  // namespace

Uploader::Uploader() {
  // defaults measured on a Llama-3-8B-shaped Q4_K file (page-cache warm,
  // tensors of 2.4-33 MB): 16 MiB x 4 slots x 16 threads 33 GB/s against
  // 30 GB/s at 32 MiB x 3 x 8; smaller slices lose to the per-slice costs
  // (4 MiB: 25 GB/s)
  slice_ = (size_t)env_long("GQ_LOAD_SLICE_MB", 16, 1, 1024) << 20;
  nslots_ = (int)env_long("GQ_LOAD_SLOTS", 4, 2, kMaxSlots);
  const long hw = (long)std::max(1u, std::thread::hardware_concurrency());
  nthreads_ = (int)env_long("GQ_LOAD_THREADS", std::min(16L, hw), 1, 64);
}

Uploader::~Uploader() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  cv_job_.notify_all();
  for (auto &t : pool_) t.join();
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto &s : slot_) {
    if (s.host) (void)hipHostFree(s.host);
    if (s.dev) (void)hipFree(s.dev);
    if (s.done) (void)hipEventDestroy(s.done);
  }
  if (stream_) (void)hipStreamDestroy(stream_);
}

bool Uploader::init(std::string *err) {
  if (ready_) return true;
  // default priority: the loader's stream never competes with compute streams
  if (!hip_ok(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "upload stream", err)) return false;
  for (int i = 0; i < nslots_; ++i)
    if (!hip_ok(hipEventCreateWithFlags(&slot_[i].done, hipEventDisableTiming), "upload event", err)) return false;
  ready_ = true;
  return true;
}

// Waits until the slot's previous slice has left it, then makes sure its
// buffers hold `bytes`.
bool Uploader::acquire(Slot &s, size_t bytes, bool need_dev, std::string *err) {
  if (s.pending) {
    if (!hip_ok(hipEventSynchronize(s.done), "upload wait", err)) return false;
    s.pending = false;
  }
  if (s.host_cap < bytes) {
    if (s.host) (void)hipHostFree(s.host);
    s.host = nullptr;
    s.host_cap = 0;
    if (!hip_ok(hipHostMalloc(&s.host, bytes, hipHostMallocDefault), "hipHostMalloc (staging)", err)) return false;
    s.host_cap = bytes;
  }
  if (need_dev && s.dev_cap < bytes) {
    if (s.dev) (void)hipFree(s.dev);
    s.dev = nullptr;
    s.dev_cap = 0;
    if (!hip_ok(hipMalloc(&s.dev, bytes), "hipMalloc (staging)", err)) return false;
    s.dev_cap = bytes;
  }
  return true;
}

void Uploader::bind_file(int fd, const void *base, size_t len) {
  fd_ = (fd >= 0 && base && len) ? fd : -1;
  fbase_ = fd_ >= 0 ? (const uint8_t *)base : nullptr;
  flen_ = fd_ >= 0 ? len : 0;
}

// Part `part` of the current job: pread from the bound file when the source
// lies in its mapping (short reads continued; on a read error the rest of
// the part is copied from the mapping), memcpy otherwise.
void Uploader::copy_part(int part) {
  const size_t o = (size_t)part * part_;
  if (o >= jbytes_) return;
  const size_t n = std::min(part_, jbytes_ - o);
  char *dst = jdst_ + o;
  const char *src = jsrc_ + o;
  if (fd_ >= 0 && (const uint8_t *)src >= fbase_ && (const uint8_t *)src + n <= fbase_ + flen_) {
    const off_t fo = (off_t)((const uint8_t *)src - fbase_);
    size_t done = 0;
    while (done < n) {
      const ssize_t r = pread(fd_, dst + done, n - done, fo + (off_t)done);
      if (r > 0) {
        done += (size_t)r;
      } else if (r < 0 && errno == EINTR) {
        continue;
      } else {
        break;
      }
    }
    if (done < n) std::memcpy(dst + done, src + done, n - done);
    return;
  }
  std::memcpy(dst, src, n);
}

void Uploader::worker() {
  for (;;) {
    int part;
    {
      std::unique_lock<std::mutex> lk(mu_);
      cv_job_.wait(lk, [&] { return stop_ || next_ < nparts_; });
      if (stop_) return;
      part = next_++;
    }
    copy_part(part);
    std::lock_guard<std::mutex> lk(mu_);
    if (--left_ == 0) cv_done_.notify_all();
  }
}

// The copy cut into parts of at least 1 MiB over the pool and the calling
// thread; returns when every part is done.
void Uploader::host_copy(void *dst, const void *src, size_t bytes) {
  const size_t min_part = 1u << 20;
  const int nt = (int)std::min<size_t>((size_t)nthreads_, std::max<size_t>(1, bytes / min_part));
  const size_t part = ((bytes + nt - 1) / nt + 4095) & ~(size_t)4095;
  {
    std::lock_guard<std::mutex> lk(mu_);
    jdst_ = (char *)dst;
    jsrc_ = (const char *)src;
    jbytes_ = bytes;
    part_ = part;
    nparts_ = (int)((bytes + part - 1) / part);
    next_ = 0;
    left_ = nparts_;
  }
  if (nparts_ > 1) {
    while ((int)pool_.size() < nthreads_ - 1) pool_.emplace_back([this] { worker(); });
    cv_job_.notify_all();
  }
  for (;;) {
    int p;
    {
      std::lock_guard<std::mutex> lk(mu_);
      if (next_ >= nparts_) break;
      p = next_++;
    }
    copy_part(p);
    std::lock_guard<std::mutex> lk(mu_);
    --left_;
  }
  std::unique_lock<std::mutex> lk(mu_);
  cv_done_.wait(lk, [&] { return left_ == 0; });
}

// After a failure, waits for the slices already queued, so none of them still
// writes to the destination once the caller sees the error.
bool Uploader::drain_after_error() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto &s : slot_) s.pending = false;
  return false;
}

bool Uploader::copy(void *dst, const void *src, size_t bytes, std::string *err) {
  if (bytes == 0) return true;
  if (!dst || !src) return fail(err, "upload: null pointer");
  if (!init(err)) return false;
  if (!copy_slices(dst, src, bytes, err)) return drain_after_error();
  return hip_ok(hipStreamSynchronize(stream_), "upload", err);
}

bool Uploader::copy_slices(void *dst, const void *src, size_t bytes, std::string *err) {
  advise_willneed(src, bytes);
  size_t j = 0;
  for (size_t off = 0; off < bytes; off += slice_, ++j) {
    const size_t n = std::min(slice_, bytes - off);
    Slot &s = slot_[j % nslots_];
    if (!acquire(s, n, false, err)) return false;
    host_copy(s.host, (const char *)src + off, n);
    if (!hip_ok(hipMemcpyAsync((char *)dst + off, s.host, n, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync",
                err))
      return false;
    if (!hip_ok(hipEventRecord(s.done, stream_), "upload event", err)) return false;
    s.pending = true;
  }
  return true;
}

bool Uploader::repack(int fmt, const uint8_t *src, size_t N, size_t K, size_t row_bytes, void *packed,
                      std::string *err) {
  if (N == 0 || K == 0) return true;
  if (!src || !packed) return fail(err, "upload: null pointer");
  if (!init(err)) return false;
  if (!repack_slices(fmt, src, N, K, row_bytes, packed, err)) return drain_after_error();
  return hip_ok(hipStreamSynchronize(stream_), "repack", err);
}

bool Uploader::repack_many(const RepackJob *jobs, size_t n, std::string *err) {
  if (n == 0) return true;
  if (!jobs) return fail(err, "upload: null pointer");
  for (size_t i = 0; i < n; ++i)
    if (jobs[i].N && jobs[i].K && (!jobs[i].src || !jobs[i].packed)) return fail(err, "upload: null pointer");
  if (!init(err)) return false;
  for (size_t i = 0; i < n; ++i) {
    const RepackJob &j = jobs[i];
    if (j.N == 0 || j.K == 0) continue;
    if (!repack_slices(j.fmt, j.src, j.N, j.K, j.row_bytes, j.packed, err)) return drain_after_error();
  }
  return hip_ok(hipStreamSynchronize(stream_), "repack", err);
}

bool Uploader::repack_slices(int fmt, const uint8_t *src, size_t N, size_t K, size_t row_bytes, void *packed,
                             std::string *err) {
  advise_willneed(src, N * row_bytes);
  // whole 16-row tiles per slice; at least one tile even if it exceeds slice_
  size_t rows_per = std::max<size_t>(16, (slice_ / std::max<size_t>(1, row_bytes)) & ~(size_t)15);
  size_t j = 0;
  for (size_t r0 = 0; r0 < N; r0 += rows_per, ++j) {
    const size_t rows = std::min(rows_per, N - r0), n = rows * row_bytes;
    Slot &s = slot_[j % nslots_];
    if (!acquire(s, rows_per * row_bytes, true, err)) return false;
    host_copy(s.host, src + r0 * row_bytes, n);
    if (!hip_ok(hipMemcpyAsync(s.dev, s.host, n, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync", err))
      return false;
    const int st = gq_repack_rows(fmt, s.dev, N, K, r0, rows, packed, stream_);
    if (st != GQ_OK) return fail(err, std::string("repack: ") + gq_status_string(st));
    if (!hip_ok(hipEventRecord(s.done, stream_), "upload event", err)) return false;
    s.pending = true;
  }
  return true;
}

}  // namespace gcore::inference
