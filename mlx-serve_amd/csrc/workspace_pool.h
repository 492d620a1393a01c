// Grow-only device buffer. A HIP graph captured while a generation was current keeps that
// generation's address in its kernel arguments, so an outgrown generation that was handed
// out during a capture is retired (kept allocated) until an explicit release: replays of
// such a graph would otherwise read and write freed memory. A generation never handed out
// during a capture is freed as soon as it is outgrown, so eager callers whose sizes keep
// rising do not accumulate dead generations. Host-only logic, templated on the allocator so
// it is testable without a GPU.
#pragma once
#include <cstddef>
#include <vector>

namespace mi {

class GrowOnlyBuffer {
 public:
  void* data() const { return data_; }
  size_t size() const { return size_; }
  size_t retired_count() const { return retired_.size(); }
  bool captured() const { return captured_; }

  // The current generation was handed out while a stream was capturing.
  void mark_captured() { captured_ = data_ != nullptr; }

  // Make the buffer at least `bytes` long. alloc(void** p, size_t n) returns 0 on success;
  // free_now(void*) frees an outgrown generation no capture holds (the caller makes sure
  // no queued work still uses it). A captured generation is retired instead. Returns
  // alloc's non-zero code on failure (the current generation is then unchanged).
  template <class Alloc, class Free>
  int grow(size_t bytes, Alloc alloc, Free free_now) {
    if (size_ >= bytes && data_) return 0;
    const size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes + bytes / 4;
    void* p = nullptr;
    const int rc = alloc(&p, want);
    if (rc) return rc;
    if (data_) {
      if (captured_)
        retired_.push_back(data_);
      else
        free_now(data_);
    }
    data_ = p;
    size_ = want;
    captured_ = false;
    return 0;
  }

  // Free every retired generation (free_fn(void*)). The caller guarantees no queued work or
  // graph that will still run refers to them.
  template <class Free>
  void release_retired(Free free_fn) {
    for (void* p : retired_) free_fn(p);
    retired_.clear();
  }

 private:
  void* data_ = nullptr;
  size_t size_ = 0;
  bool captured_ = false;
  std::vector<void*> retired_;
};

}  // namespace mi
