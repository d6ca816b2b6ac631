// Host-side bookkeeping of the device memory the library hands out: the
// caching block allocator behind tt_malloc / tt_free, and the per-stream
// scratch buffers of the attention launchers.
//
// The reference allocates with cudaMalloc and frees with cudaFree on every
// TinyTensor construction, copy and resize (src/Tinytensor.cu:21,39,60,77,
// 90,108,116,239,252,375-378) and checks none of the results.  Here device
// memory comes from one cache per process, every failure is reported, and the
// code has no HIP dependency of its own: it runs over a Backend
//
//   struct Backend {
//     int  alloc(size_t bytes, void** p);  // TT_OK or an error code; *p set on success
//     void release(void* p);               // return a block to the device
//     int  sync(void* stream);             // wait for all work queued on `stream`
//     int  order_after_library(void* stream);  // work queued on `stream` from now on
//                                              // waits for the library stream's queued work
//   };
//
// so that the same code is compiled into the HIP runtime and, with a fake
// backend, into CPU tests (including sanitizer builds).
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <utility>

namespace tt {

// Allocation-failure injection for tests of the out-of-memory paths:
// with TT_FAIL_ALLOC_AFTER=n in the environment, device allocations number
// n, n + 1, ... (counting from 0 in this process) fail as if the device were
// out of memory.  Unset or negative: no injection.
class AllocFailureInjector {
 public:
  AllocFailureInjector() {
    const char* e = std::getenv("TT_FAIL_ALLOC_AFTER");
    limit_ = e && *e ? std::strtoll(e, nullptr, 10) : -1;
  }
  // Whether the next device allocation must fail; counts it either way.
  bool next_fails() {
    std::lock_guard<std::mutex> lk(mu_);
    const long long n = count_++;
    return limit_ >= 0 && n >= limit_;
  }
  void set_limit(long long limit) {
    std::lock_guard<std::mutex> lk(mu_);
    limit_ = limit;
    count_ = 0;
  }

 private:
  std::mutex mu_;
  long long limit_ = -1, count_ = 0;
};

// Size class of a request: 512-byte granules below 1 MiB, 2 MiB granules
// above.  Requests of 0 bytes take one granule.
inline size_t block_size_class(size_t bytes) {
  if (bytes == 0) bytes = 1;
  const size_t small = 512, big = size_t(2) << 20;
  if (bytes < (size_t(1) << 20)) return (bytes + small - 1) / small * small;
  return (bytes + big - 1) / big * big;
}

// Caching allocator.  Freed blocks stay in a free list keyed by size class
// and are handed out again first-fit (the smallest cached class >= the
// request, if it is at most twice the request).  When the device refuses an
// allocation, every cached block is returned to it and the allocation is
// tried once more.  Blocks are reused in the order the host frees and
// allocates them: callers order their device work on one stream (a freed
// block's last reader runs before the next owner's first writer).
template <class Backend>
class BlockCache {
 public:
  explicit BlockCache(Backend& be) : be_(be) {}

  // TT_OK and *ptr, or the backend's error code (ptr untouched).
  int alloc(size_t bytes, void** ptr) {
    const size_t cls = block_size_class(bytes);
    {
      std::lock_guard<std::mutex> lk(mu_);
      auto it = free_.lower_bound(cls);
      if (it != free_.end() && it->first <= 2 * cls) {
        void* p = it->second;
        const size_t c = it->first;
        free_.erase(it);
        live_[p] = c;
        cached_ -= c;
        in_use_ += c;
        *ptr = p;
        return 0;
      }
    }
    void* p = nullptr;
    int rc = be_.alloc(cls, &p);
    if (rc != 0) {
      trim();
      rc = be_.alloc(cls, &p);
      if (rc != 0) return rc;
    }
    std::lock_guard<std::mutex> lk(mu_);
    live_[p] = cls;
    in_use_ += cls;
    *ptr = p;
    return 0;
  }

  // false if `p` is not a live block of this cache (nullptr is fine).
  bool release(void* p) {
    if (!p) return true;
    std::lock_guard<std::mutex> lk(mu_);
    auto it = live_.find(p);
    if (it == live_.end()) return false;
    const size_t c = it->second;
    live_.erase(it);
    in_use_ -= c;
    free_.emplace(c, p);
    cached_ += c;
    return true;
  }

  // Return every cached (free) block to the device.
  void trim() {
    std::multimap<size_t, void*> blocks;
    {
      std::lock_guard<std::mutex> lk(mu_);
      blocks.swap(free_);
      cached_ = 0;
    }
    for (auto& kv : blocks) be_.release(kv.second);
  }

  void stats(size_t* in_use, size_t* cached) {
    std::lock_guard<std::mutex> lk(mu_);
    if (in_use) *in_use = in_use_;
    if (cached) *cached = cached_;
  }

 private:
  Backend& be_;
  std::mutex mu_;
  std::multimap<size_t, void*> free_;
  std::unordered_map<void*, size_t> live_;  // block -> class size
  size_t in_use_ = 0, cached_ = 0;
};

// Scratch buffers of the attention launchers, one per (stream, user): two
// calls on different streams never share a buffer, so their kernels may
// overlap.  A Lease holds the cache's lock from the moment the buffer is
// handed out until the caller has queued every kernel that reads it, so
// calls on one stream from several host threads cannot interleave their
// launches; the stream then orders the kernels of consecutive calls.  A
// buffer that must grow is replaced only after the stream that used it has
// drained (its last kernels may still read it).  A buffer handed to a stream
// for the first time is a block of the BlockCache, which tt_free may have
// returned while work on the library stream still used it: that stream is
// first ordered after the library stream's queued work.
template <class Backend>
class WorkspaceCache {
 public:
  struct Slot {
    void* ptr = nullptr;
    size_t bytes = 0;
    uint64_t uses = 0;  // earlier get() calls that returned this buffer
  };

  WorkspaceCache(Backend& be, BlockCache<Backend>& blocks) : be_(be), blocks_(blocks) {}

  class Lease {
   public:
    explicit Lease(WorkspaceCache& c) : c_(c), lk_(c.mu_) {}
    // A buffer of at least `bytes` for `user` on `stream`, valid while the
    // lease lives (and for the device work queued on `stream` meanwhile).
    // *uses (optional): how many earlier get() calls returned this same
    // buffer; 0 for a new buffer, whose contents are undefined.
    int get(void* stream, int user, size_t bytes, void** ptr, uint64_t* uses = nullptr) {
      return c_.get_locked(stream, user, bytes, ptr, uses);
    }

   private:
    WorkspaceCache& c_;
    std::unique_lock<std::mutex> lk_;
  };

  // Wait for each buffer's stream, then give every buffer back to the block
  // cache.  Returns the first backend error, if any.
  int release_all() {
    std::lock_guard<std::mutex> lk(mu_);
    int first = 0;
    for (auto& kv : slots_) {
      const int rc = be_.sync(kv.first.first);
      if (rc && !first) first = rc;
      blocks_.release(kv.second.ptr);
    }
    slots_.clear();
    return first;
  }

  // Wait for `stream`, then give its buffers back (before the stream is
  // destroyed: a later stream may reuse the handle).
  int release_stream(void* stream) {
    std::lock_guard<std::mutex> lk(mu_);
    int rc = 0;
    for (auto it = slots_.begin(); it != slots_.end();) {
      if (it->first.first != stream) {
        ++it;
        continue;
      }
      if (!rc) rc = be_.sync(stream);
      blocks_.release(it->second.ptr);
      it = slots_.erase(it);
    }
    return rc;
  }

  size_t count() {
    std::lock_guard<std::mutex> lk(mu_);
    return slots_.size();
  }
  size_t bytes_held() {
    std::lock_guard<std::mutex> lk(mu_);
    size_t n = 0;
    for (auto& kv : slots_) n += kv.second.bytes;
    return n;
  }

 private:
  int get_locked(void* stream, int user, size_t bytes, void** ptr, uint64_t* uses) {
    Slot& s = slots_[{stream, user}];
    if (s.ptr && bytes <= s.bytes) {
      *ptr = s.ptr;
      if (uses) *uses = s.uses;
      ++s.uses;
      return 0;
    }
    if (s.ptr) {
      const int rc = be_.sync(stream);  // kernels queued earlier on this stream may still read it
      if (rc) return rc;
      blocks_.release(s.ptr);
      s = Slot{};
    }
    void* p = nullptr;
    int rc = blocks_.alloc(bytes, &p);
    if (!rc) {
      rc = be_.order_after_library(stream);
      if (rc) blocks_.release(p);
    }
    if (rc) {
      slots_.erase({stream, user});
      return rc;
    }
    s.ptr = p;
    s.bytes = bytes;
    s.uses = 1;
    *ptr = p;
    if (uses) *uses = 0;
    return 0;
  }

  Backend& be_;
  BlockCache<Backend>& blocks_;
  std::mutex mu_;
  std::map<std::pair<void*, int>, Slot> slots_;
};

}  // namespace tt
