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

// Records the next instrumentation event (tt_set_launch_events) after a
// kernel launch on `s`; a no-op unless instrumentation is enabled.
void after_launch(hipStream_t s);

// Device scratch owned by the library, grown on demand and kept for reuse.
// `slot` separates independent users (0: attention bwd row sums,
// 1: decode partials).  Stream-ordered on the library stream; callers that
// pass another stream must not overlap two calls that share a slot.
int workspace(int slot, size_t bytes, void** ptr);

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

// Launch-error check plus the instrumentation hook, for kernels on stream s.
#define TT_LAUNCHED(what, s)    \
  do {                          \
    TT_LAUNCH_CHECK(what);      \
    tt::after_launch(s);        \
  } while (0)
