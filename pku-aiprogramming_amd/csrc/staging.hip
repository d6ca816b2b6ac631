// Host <-> device transfers of TinyTensor data (the reference's synchronous
// cudaMemcpy at src/Tinytensor.cu:40,61,213,238,251 and the element loops
// around them), through pinned staging buffers.
//
// hipMemcpy from pageable memory moves data through the runtime's own bounce
// buffer with one CPU thread; DMA from pinned (page-locked) memory runs at
// the link's rate.  Large copies here are cut into chunks: a small pool of
// host threads copies, or converts, one chunk between the caller's memory and
// one of three pinned buffers while the DMA engine moves the others.  Converting
// copies (float32 host values <-> bf16 device storage) do the conversion in
// that same pass, so no intermediate host array is made.  Plain copies below
// kDirectMax, and copies whose host side is already pinned, go straight to
// hipMemcpyAsync.
#include <hip/hip_runtime.h>
#include <sched.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "host_copy.h"
#include "tt_internal.h"

namespace tt {
namespace {

constexpr int kBufs = 3;                     // pinned buffers in the ring
constexpr size_t kChunk = size_t(16) << 20;  // bytes of one pinned buffer
constexpr size_t kRamp = size_t(1) << 20;        // first and last chunk bytes
constexpr size_t kPiece = size_t(256) << 10;     // least device bytes per thread
constexpr size_t kDirectMax = size_t(4) << 20;   // plain copies below this skip staging

// Persistent worker threads.  run(n, fn) calls fn(0..n-1) on the workers and
// the calling thread and returns when all calls returned.  One caller at a
// time (the staging lock is held around every use).  Between jobs a worker
// spins for up to kSpinUs before it sleeps, so that the jobs of one staged
// copy, a few hundred microseconds apart, find it awake.
class HostPool {
 public:
  explicit HostPool(int workers) : nworkers_(workers) {
    for (int i = 0; i < workers; ++i) std::thread([this] { loop(); }).detach();
  }
  void run(size_t n, const std::function<void(size_t)>& fn) {
    if (nworkers_ == 0 || n <= 1) {
      for (size_t i = 0; i < n; ++i) fn(i);
      return;
    }
    {
      std::lock_guard<std::mutex> lk(mu_);
      fn_ = &fn;
      njobs_ = n;
      next_.store(0, std::memory_order_relaxed);
      busy_.store(nworkers_, std::memory_order_relaxed);
      gen_.fetch_add(1, std::memory_order_release);
    }
    start_.notify_all();
    drain(fn, n);
    if (spin_until([this] { return busy_.load(std::memory_order_acquire) == 0; })) return;
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [this] { return busy_.load(std::memory_order_acquire) == 0; });
  }

 private:
  static constexpr int kSpinUs = 200;

  template <typename F>
  static bool spin_until(F&& ready) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0;; ++i) {
      if (ready()) return true;
      __builtin_ia32_pause();
      if ((i & 63) == 63 && std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(kSpinUs)) return false;
    }
  }
  void drain(const std::function<void(size_t)>& fn, size_t n) {
    for (size_t i; (i = next_.fetch_add(1, std::memory_order_relaxed)) < n;) fn(i);
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      if (!spin_until([&] { return gen_.load(std::memory_order_acquire) != seen; })) {
        std::unique_lock<std::mutex> lk(mu_);
        start_.wait(lk, [&] { return gen_.load(std::memory_order_acquire) != seen; });
      }
      const std::function<void(size_t)>* fn;
      size_t n;
      {
        std::lock_guard<std::mutex> lk(mu_);
        seen = gen_.load(std::memory_order_relaxed);
        fn = fn_;
        n = njobs_;
      }
      drain(*fn, n);
      std::lock_guard<std::mutex> lk(mu_);
      if (busy_.fetch_sub(1, std::memory_order_acq_rel) == 1) done_.notify_one();
    }
  }

  std::mutex mu_;
  std::condition_variable start_, done_;
  const std::function<void(size_t)>* fn_ = nullptr;
  size_t njobs_ = 0;
  std::atomic<size_t> next_{0};
  std::atomic<uint64_t> gen_{0};
  std::atomic<int> busy_{0};
  const int nworkers_;
};

// Host threads used per copy (the caller included): TT_HOST_THREADS, else
// min(16, CPUs this process may run on).
int host_threads() {
  static const int n = [] {
    if (const char* e = std::getenv("TT_HOST_THREADS")) {
      int v = std::atoi(e);
      if (v >= 1) return std::min(v, 64);
    }
    cpu_set_t set;
    int cpus = sched_getaffinity(0, sizeof(set), &set) == 0 ? CPU_COUNT(&set) : 0;
    if (cpus <= 0) cpus = (int)std::thread::hardware_concurrency();
    return std::max(1, std::min(16, cpus));
  }();
  return n;
}

enum class Cvt { kCopy, kF32ToBf16, kBf16ToF32 };

// Bytes per element on the device and on the host for a conversion.
size_t dev_size(Cvt c) { return c == Cvt::kCopy ? 1 : 2; }
size_t host_size(Cvt c) { return c == Cvt::kCopy ? 1 : 4; }

// Moves n elements host->pinned (h2d) or pinned->host (d2h), converting.
void move(Cvt c, void* dst, const void* src, size_t n) {
  switch (c) {
    case Cvt::kCopy: copy_stream(dst, src, n); break;
    case Cvt::kF32ToBf16: f32_to_bf16_stream((uint16_t*)dst, (const float*)src, n); break;
    case Cvt::kBf16ToF32: bf16_to_f32_stream((float*)dst, (const uint16_t*)src, n); break;
  }
}

struct Stage {
  void* buf[kBufs] = {};
  hipEvent_t ev[kBufs] = {};
  HostPool* pool = nullptr;
  pid_t owner = 0;
};
std::mutex g_stage_mu;
Stage g_stage;

// Pinned buffers, their events and the thread pool, made on first use and
// kept for the life of the process.  A forked child (which has neither the
// parent's threads nor its HIP context) starts over.
int stage_ready() {
  if (g_stage.owner == getpid() && g_stage.buf[kBufs - 1]) return TT_OK;
  g_stage = Stage();
  for (int b = 0; b < kBufs; ++b) {
    hipError_t e = hipHostMalloc(&g_stage.buf[b], kChunk, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&g_stage.ev[b], hipEventDisableTiming);
    if (e != hipSuccess) {
      for (int j = 0; j <= b; ++j) {
        if (g_stage.buf[j]) (void)hipHostFree(g_stage.buf[j]);
        if (g_stage.ev[j]) (void)hipEventDestroy(g_stage.ev[j]);
      }
      g_stage = Stage();
      return hip_fail(e, "staging buffer (hipHostMalloc)");
    }
  }
  g_stage.pool = new HostPool(host_threads() - 1);  // never destroyed: workers are detached
  g_stage.owner = getpid();
  return TT_OK;
}

// Runs move() over n elements split into pieces of at least kPiece device
// bytes, on the pool.
void move_parallel(Cvt c, char* dst, const char* src, size_t n, bool to_device) {
  const size_t dsz = dev_size(c), hsz = host_size(c);
  const size_t per = std::max<size_t>(kPiece / dsz, 64);
  const size_t pieces = std::min<size_t>((n + per - 1) / per, (size_t)host_threads());
  const size_t step = ((n + pieces - 1) / pieces + 63) / 64 * 64;
  g_stage.pool->run(pieces, [&](size_t p) {
    const size_t i0 = p * step;
    if (i0 >= n) return;
    const size_t m = std::min(step, n - i0);
    if (to_device)
      move(c, dst + i0 * dsz, src + i0 * hsz, m);
    else
      move(c, dst + i0 * hsz, src + i0 * dsz, m);
  });
}

// Chunk boundaries (element offsets) for n elements of dsz device bytes.
// Only the first chunk's host pass (h2d) or DMA (d2h) and the last chunk's
// DMA (h2d) or host pass (d2h) are not overlapped, so the chunks grow from
// kRamp to kChunk bytes and each of the last ones takes half of what is left.
std::vector<size_t> chunk_bounds(size_t n, size_t dsz) {
  const size_t full = kChunk / dsz, lo = kRamp / dsz;
  std::vector<size_t> b{0};
  size_t cur = lo;
  for (size_t i = 0; i < n;) {
    const size_t left = n - i;
    size_t m = std::min(cur, full);
    if (left <= lo) m = left;
    else if (m > left / 2) m = std::max(lo, (left / 2 + 63) / 64 * 64);
    if (left - std::min(m, left) < lo) m = left;  // no crumb after the last halving
    m = std::min(m, left);
    i += m;
    b.push_back(i);
    cur = std::min(full, 2 * cur);
  }
  return b;
}

// n elements from host src to device dst.
int staged_h2d(char* dst, const char* src, size_t n, Cvt c, hipStream_t s) {
  int rc = stage_ready();
  if (rc) return rc;
  const size_t dsz = dev_size(c), hsz = host_size(c);
  const std::vector<size_t> cb = chunk_bounds(n, dsz);
  bool pending[kBufs] = {};
  for (size_t k = 0; k + 1 < cb.size(); ++k) {
    const int b = (int)(k % kBufs);
    const size_t i0 = cb[k], m = cb[k + 1] - cb[k];
    if (pending[b]) TT_HIP(hipEventSynchronize(g_stage.ev[b]));  // the DMA that read buf[b] is done
    move_parallel(c, (char*)g_stage.buf[b], src + i0 * hsz, m, true);
    TT_HIP(hipMemcpyAsync(dst + i0 * dsz, g_stage.buf[b], m * dsz, hipMemcpyHostToDevice, s));
    TT_HIP(hipEventRecord(g_stage.ev[b], s));
    pending[b] = true;
  }
  TT_HIP(hipStreamSynchronize(s));
  return ok();
}

// n elements from device src to host dst.
int staged_d2h(char* dst, const char* src, size_t n, Cvt c, hipStream_t s) {
  int rc = stage_ready();
  if (rc) return rc;
  const size_t dsz = dev_size(c), hsz = host_size(c);
  const std::vector<size_t> cb = chunk_bounds(n, dsz);
  const size_t nk = cb.size() - 1;
  auto issue = [&](size_t k) -> int {
    const int b = (int)(k % kBufs);
    TT_HIP(hipMemcpyAsync(g_stage.buf[b], src + cb[k] * dsz, (cb[k + 1] - cb[k]) * dsz, hipMemcpyDeviceToHost, s));
    TT_HIP(hipEventRecord(g_stage.ev[b], s));
    return TT_OK;
  };
  for (size_t k = 0; k + 1 < (size_t)kBufs && k < nk; ++k)
    if ((rc = issue(k))) return rc;
  for (size_t k = 0; k < nk; ++k) {
    const int b = (int)(k % kBufs);
    // chunk k + kBufs - 1 goes to the buffer the host drained in the previous iteration
    if (k + kBufs - 1 < nk && (rc = issue(k + kBufs - 1))) return rc;
    TT_HIP(hipEventSynchronize(g_stage.ev[b]));
    move_parallel(c, dst + cb[k] * hsz, (const char*)g_stage.buf[b], cb[k + 1] - cb[k], false);
  }
  return ok();
}

// What HIP knows of the host-side pointer of a copy: pinned host memory
// (copied directly), device memory (an argument error: the host threads of
// the staged path cannot touch it), or ordinary pageable memory.
enum class HostMem { kPageable, kPinned, kDevice };
HostMem host_mem(const void* p) {
  hipPointerAttribute_t a;
  HostMem m = HostMem::kPageable;
  if (hipPointerGetAttributes(&a, p) == hipSuccess) {
    if (a.type == hipMemoryTypeHost) m = HostMem::kPinned;
    else if (a.type == hipMemoryTypeDevice) m = HostMem::kDevice;
  }
  (void)hipGetLastError();
  return m;
}

// A failed staged copy may leave a DMA in flight on a pinned buffer: wait for
// it before the buffers are reused, and report the first error.
int settle(int rc, hipStream_t s) {
  if (rc != TT_OK) (void)hipStreamSynchronize(s);
  return rc;
}

}  // namespace
}  // namespace tt

using namespace tt;

int tt_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return TT_OK;
  if (!dst || !src) return fail(TT_ERR_ARG, "tt_memcpy_h2d: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(nullptr);
  const HostMem hm = host_mem(src);
  if (hm == HostMem::kDevice) return fail(TT_ERR_ARG, "tt_memcpy_h2d: source is device memory (use tt_memcpy_d2d)");
  if (bytes < kDirectMax || hm == HostMem::kPinned) {
    TT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
    TT_HIP(hipStreamSynchronize(s));
    return ok();
  }
  std::lock_guard<std::mutex> lk(g_stage_mu);
  return settle(staged_h2d((char*)dst, (const char*)src, bytes, Cvt::kCopy, s), s);
}

int tt_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return TT_OK;
  if (!dst || !src) return fail(TT_ERR_ARG, "tt_memcpy_d2h: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(nullptr);
  const HostMem hm = host_mem(dst);
  if (hm == HostMem::kDevice)
    return fail(TT_ERR_ARG, "tt_memcpy_d2h: destination is device memory (use tt_memcpy_d2d)");
  if (bytes < kDirectMax || hm == HostMem::kPinned) {
    TT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    TT_HIP(hipStreamSynchronize(s));
    return ok();
  }
  std::lock_guard<std::mutex> lk(g_stage_mu);
  return settle(staged_d2h((char*)dst, (const char*)src, bytes, Cvt::kCopy, s), s);
}

int tt_upload_bf16_from_f32(void* dst, const float* src, size_t n) {
  if (n == 0) return TT_OK;
  if (!dst || !src) return fail(TT_ERR_ARG, "tt_upload_bf16_from_f32: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  if (host_mem(src) == HostMem::kDevice) return fail(TT_ERR_ARG, "tt_upload_bf16_from_f32: source is device memory");
  hipStream_t s = stream_or_default(nullptr);
  std::lock_guard<std::mutex> lk(g_stage_mu);
  return settle(staged_h2d((char*)dst, (const char*)src, n, Cvt::kF32ToBf16, s), s);
}

int tt_download_bf16_to_f32(float* dst, const void* src, size_t n) {
  if (n == 0) return TT_OK;
  if (!dst || !src) return fail(TT_ERR_ARG, "tt_download_bf16_to_f32: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  if (host_mem(dst) == HostMem::kDevice)
    return fail(TT_ERR_ARG, "tt_download_bf16_to_f32: destination is device memory");
  hipStream_t s = stream_or_default(nullptr);
  std::lock_guard<std::mutex> lk(g_stage_mu);
  return settle(staged_d2h((char*)dst, (const char*)src, n, Cvt::kBf16ToF32, s), s);
}

int tt_host_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(TT_ERR_ARG, "tt_host_malloc: null pointer");
  *ptr = nullptr;
  int rc = ensure_init();
  if (rc) return rc;
  TT_HIP(hipHostMalloc(ptr, std::max<size_t>(bytes, 1), hipHostMallocDefault));
  return ok();
}

int tt_host_free(void* ptr) {
  if (!ptr) return TT_OK;
  TT_HIP(hipHostFree(ptr));
  return ok();
}
