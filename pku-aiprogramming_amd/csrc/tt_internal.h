// Internal helpers shared by the runtime and the attention kernels.
// Host-side error reporting, the library stream and the workspace cache.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/tt_attn.h"

namespace tt {

// Records a message for tt_last_error() and returns `code`.
int fail(int code, const std::string& msg);
// Clears the last error and returns TT_OK.
int ok();
// Maps a HIP status to TT_ERR_HIP with the call site.
int hip_fail(hipError_t e, const char* what);

// The library stream (created by tt_init on first use).
hipStream_t stream_or_default(void* s);
int ensure_init();
// Compute units of the bound device (after ensure_init).
int device_cu_count();

// Records the next instrumentation event (tt_set_launch_events) after a
// kernel launch on `s`; a no-op unless instrumentation is enabled.
void after_launch(hipStream_t s);

// The allocation-free backward's scratch: a static device array of
// kNoAllocScratchBytes whose device address tt_init looks up once per
// device.  Returns nullptr before tt_init; *bytes gets the array's size.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
void* noalloc_scratch(size_t* bytes);

// Device scratch of the attention launchers: one buffer per (stream, user),
// grown on demand and kept for reuse.  A lease holds the workspace lock from
// get() until it is destroyed: keep it alive until every kernel that reads
// the buffer has been launched on that stream.
enum { kWsBackwardRows = 0, kWsDecodePartials = 1, kWsForwardSplits = 2, kWsSoftmaxPartials = 3 };
class WorkspaceLease {
 public:
  WorkspaceLease();
  ~WorkspaceLease();
  WorkspaceLease(const WorkspaceLease&) = delete;
  WorkspaceLease& operator=(const WorkspaceLease&) = delete;
  // *uses (optional): earlier get() calls that returned the same buffer (0:
  // a new buffer with undefined contents).
  int get(hipStream_t stream, int user, size_t bytes, void** ptr, uint64_t* uses = nullptr);

 private:
  struct Impl;
  Impl* impl_;
};

}  // namespace tt

#define TT_HIP(call)                                   \
  do {                                                 \
    hipError_t e_ = (call);                            \
    if (e_ != hipSuccess) return tt::hip_fail(e_, #call); \
  } while (0)

#define TT_LAUNCH_CHECK(what)                                  \
  do {                                                         \
    hipError_t e_ = hipGetLastError();                         \
    if (e_ != hipSuccess) return tt::hip_fail(e_, what);       \
  } while (0)

namespace tt {
// A one-dimensional launch holds at most 2^32 - 1 work-items (the dispatch
// packet counts the grid in work-items, not workgroups).
inline bool grid_fits(int64_t workgroups, int64_t threads) {
  return workgroups >= 0 && workgroups <= int64_t(0xffffffffu) / threads;
}
}  // namespace tt

// Launch-error check plus the instrumentation hook, for kernels on stream s.
#define TT_LAUNCHED(what, s)    \
  do {                          \
    TT_LAUNCH_CHECK(what);      \
    tt::after_launch(s);        \
  } while (0)
