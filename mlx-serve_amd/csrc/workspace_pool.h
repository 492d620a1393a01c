// Grow-only device buffer whose outgrown generations stay allocated until an explicit
// release. A HIP graph captured while an older generation was current keeps that
// generation's address in its kernel arguments, so growing must not free it: replays of
// such a graph would read and write freed memory. Host-only logic, templated on the
// allocator so it is testable without a GPU.
#pragma once
#include <cstddef>
#include <vector>

namespace mi {

class GrowOnlyBuffer {
 public:
  void* data() const { return data_; }
  size_t size() const { return size_; }
  size_t retired_count() const { return retired_.size(); }

  // Make the buffer at least `bytes` long. alloc(void** p, size_t n) returns 0 on success.
  // The previous generation is retired, not freed. Returns alloc's non-zero code on failure
  // (the current generation is then unchanged).
  template <class Alloc>
  int grow(size_t bytes, Alloc alloc) {
    if (size_ >= bytes && data_) return 0;
    const size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes + bytes / 4;
    void* p = nullptr;
    const int rc = alloc(&p, want);
    if (rc) return rc;
    if (data_) retired_.push_back(data_);
    data_ = p;
    size_ = want;
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
  std::vector<void*> retired_;
};

}  // namespace mi
