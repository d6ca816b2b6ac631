// TinyTensor device runtime for MI355X: errors, stream, caching allocator,
// copies, events and the elementwise kernels behind TinyTensor's methods.
//
// The reference allocates with cudaMalloc/cudaFree on every construction and
// synchronises after every launch (src/Tinytensor.cu:21,90,146).  Here all
// work is ordered on one library stream; host-visible copies wait for it.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "device_cache.h"
#include "tt_internal.h"

namespace tt {

static thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}
int ok() {
  g_err.clear();
  return TT_OK;
}
int hip_fail(hipError_t e, const char* what) {
  std::string m = std::string("HIP error in ") + what + ": " + hipGetErrorName(e) + " (" +
                  hipGetErrorString(e) + ")";
  int code = (e == hipErrorOutOfMemory) ? TT_ERR_NOMEM : TT_ERR_HIP;
  return fail(code, m);
}

static std::mutex g_mu;
// Set (release) by tt_init after the device, stream and scratch address are
// in place; read (acquire) without the lock on every call.
static std::atomic<bool> g_inited{false};
static int g_device = 0;
static int g_cus = 1;  // compute units of the bound device (set by tt_init)
static hipStream_t g_stream = nullptr;

int device_cu_count() { return g_cus; }

int ensure_init() {
  if (g_inited.load(std::memory_order_acquire)) return TT_OK;
  return tt_init(g_device);
}

hipStream_t stream_or_default(void* s) {
  return s ? static_cast<hipStream_t>(s) : g_stream;
}

// ---------------------------------------------------------------- allocator
// hipMalloc / hipFree / hipStreamSynchronize as the backend of the caching
// allocator and the workspace cache (device_cache.h).  Allocation failures,
// real or injected by TT_FAIL_ALLOC_AFTER, are TT_ERR_NOMEM with a message.
struct HipBackend {
  AllocFailureInjector inject;
  int alloc(size_t bytes, void** p) {
    if (inject.next_fails())
      return fail(TT_ERR_NOMEM, "tt_malloc: allocation of " + std::to_string(bytes) +
                                    " bytes refused (TT_FAIL_ALLOC_AFTER failure injection)");
    const hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(TT_ERR_NOMEM,
                  "tt_malloc: hipMalloc of " + std::to_string(bytes) + " bytes failed: " + hipGetErrorString(e));
    }
    return TT_OK;
  }
  // hipFree waits for the device work that may still use the block
  void release(void* p) { (void)hipFree(p); }
  int sync(void* stream) {
    const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
    return e == hipSuccess ? TT_OK : hip_fail(e, "hipStreamSynchronize (workspace)");
  }
  // A block tt_free returned while library-stream work still used it may
  // become another stream's workspace: that stream waits for the library
  // stream's queued work (an event, no host wait).  Called under the
  // workspace lock, which also guards `order_ev`.
  hipEvent_t order_ev = nullptr;
  int order_after_library(void* stream) {
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (!s || s == g_stream) return TT_OK;
    hipError_t e = hipSuccess;
    if (!order_ev) e = hipEventCreateWithFlags(&order_ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(order_ev, g_stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(s, order_ev, 0);
    return e == hipSuccess ? TT_OK : hip_fail(e, "ordering a new workspace after the library stream");
  }
};
static HipBackend g_backend;
static BlockCache<HipBackend> g_blocks(g_backend);
static WorkspaceCache<HipBackend> g_ws(g_backend, g_blocks);

// ---------------------------------------------------------------- instrumentation
// Events to record after the next launches (tt_set_launch_events).  The
// count is read without the lock, so launches pay nothing while none is set.
static std::mutex g_ev_mu;
static std::vector<void*> g_launch_events;
static size_t g_launch_next = 0;
static std::atomic<size_t> g_launch_left{0};

void after_launch(hipStream_t s) {
  if (g_launch_left.load(std::memory_order_acquire) == 0) return;
  std::lock_guard<std::mutex> lk(g_ev_mu);
  if (g_launch_next >= g_launch_events.size()) return;
  (void)hipEventRecord((hipEvent_t)g_launch_events[g_launch_next++], s);
  g_launch_left.store(g_launch_events.size() - g_launch_next, std::memory_order_release);
}

// ---------------------------------------------------------------- allocation-free scratch
// Row scratch of tt_attn_bwd_bf16_noalloc (-D and LSE * log2(e) of up to
// 2 Mi query rows).  Every GPU holds its own copy until the process ends;
// host code uses the device address tt_init looked up, never the array's
// name (which on the host is only a stand-in for the symbol).
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];
constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices] = {};

void* noalloc_scratch(size_t* bytes) {
  if (bytes) *bytes = kNoAllocScratchBytes;
  if (!g_inited.load(std::memory_order_acquire)) return nullptr;
  return g_scratch_ptr[g_device];
}

// ---------------------------------------------------------------- workspace
struct WorkspaceLease::Impl {
  WorkspaceCache<HipBackend>::Lease lease{g_ws};
};
WorkspaceLease::WorkspaceLease() : impl_(new Impl) {}
WorkspaceLease::~WorkspaceLease() { delete impl_; }
int WorkspaceLease::get(hipStream_t s, int user, size_t bytes, void** ptr, uint64_t* uses) {
  return impl_->lease.get(static_cast<void*>(s), user, bytes, ptr, uses);
}

// ---------------------------------------------------------------- elementwise
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Uniform in [0, 1) with 24 bits from a 64-bit hash.
__device__ __forceinline__ float u01(uint64_t h) { return (float)(h >> 40) * (1.0f / 16777216.0f); }

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);                                          // RNE
  return uint16_t(u >> 16);
}

template <typename T> struct Num {
  __device__ static float ld(const T* p, int64_t i) { return (float)p[i]; }
  __device__ static void st(T* p, int64_t i, double v) { p[i] = (T)v; }
  __device__ static float from(T x) { return (float)x; }
  __device__ static T to(double v) { return (T)v; }
};
template <> struct Num<uint16_t> {  // bf16 storage
  __device__ static float ld(const uint16_t* p, int64_t i) { return bf2f(p[i]); }
  __device__ static void st(uint16_t* p, int64_t i, double v) { p[i] = f2bf((float)v); }
  __device__ static float from(uint16_t x) { return bf2f(x); }
  __device__ static uint16_t to(double v) { return f2bf((float)v); }
};
template <> struct Num<double> {
  __device__ static double ld(const double* p, int64_t i) { return p[i]; }
  __device__ static void st(double* p, int64_t i, double v) { p[i] = v; }
  __device__ static double from(double x) { return x; }
  __device__ static double to(double v) { return v; }
};

// One element of tt_elementwise: element i of c from the stored values x = a[i]
// and y = b[i] (zero where the op reads no such operand).  Floating storage
// computes in double and rounds once on the store (for add, sub and scale of
// floats this is the correctly rounded float result); int32 keeps integer
// arithmetic where the reference has it (add / sub / neg / scale).
template <int OP, typename T>
__device__ __forceinline__ T ew_one(T xs, T ys, int64_t i, double alpha, double beta, uint64_t seed) {
  const double x = Num<T>::from(xs), y = Num<T>::from(ys);
  double r = 0.0;
  if constexpr (OP == TT_EW_ADD) r = x + y;
  else if constexpr (OP == TT_EW_SUB) r = x - y;
  else if constexpr (OP == TT_EW_FILL) r = alpha;
  else if constexpr (OP == TT_EW_NEG) r = -x;
  else if constexpr (OP == TT_EW_SCALE) r = x * alpha;
  else if constexpr (OP == TT_EW_RELU) r = x > 0 ? x : 0;
  else if constexpr (OP == TT_EW_RELU_BWD) r = x > 0 ? y : 0.0;
  else if constexpr (OP == TT_EW_SIGMOID) r = 1.0 / (1.0 + exp(-x));
  else if constexpr (OP == TT_EW_SIGMOID_BWD) {
    const double s = 1.0 / (1.0 + exp(-x));
    r = s * (1.0 - s) * y;
  } else if constexpr (OP == TT_EW_UNIFORM) {
    r = alpha + (beta - alpha) * u01(splitmix64(seed ^ splitmix64((uint64_t)i)));
  }
  return Num<T>::to(r);
}
template <int OP>
__device__ __forceinline__ int32_t ew_one_i32(int32_t x, int32_t y, int64_t i, double alpha, double beta,
                                              uint64_t seed) {
  if constexpr (OP == TT_EW_ADD) return x + y;
  else if constexpr (OP == TT_EW_SUB) return x - y;
  else if constexpr (OP == TT_EW_FILL) return (int32_t)alpha;
  else if constexpr (OP == TT_EW_NEG) return -x;
  else if constexpr (OP == TT_EW_SCALE) return (int32_t)(x * (int32_t)alpha);
  else if constexpr (OP == TT_EW_RELU) return x > 0 ? x : 0;
  else if constexpr (OP == TT_EW_RELU_BWD) return x > 0 ? y : 0;
  else if constexpr (OP == TT_EW_SIGMOID) return (int32_t)(1.0 / (1.0 + exp(-(double)x)));
  else if constexpr (OP == TT_EW_SIGMOID_BWD) {
    const double s = 1.0 / (1.0 + exp(-(double)x));
    return (int32_t)(s * (1.0 - s) * y);
  } else {
    // inclusive integer range [alpha, beta] like std::uniform_int_distribution
    const int64_t lo = (int64_t)alpha, hi = (int64_t)beta;
    const uint64_t span = (uint64_t)(hi - lo + 1);
    return (int32_t)(lo + (int64_t)(splitmix64(seed ^ splitmix64((uint64_t)i)) % span));
  }
}
template <int OP, typename T>
__device__ __forceinline__ T ew_elem(T x, T y, int64_t i, double alpha, double beta, uint64_t seed) {
  if constexpr (std::is_same<T, int32_t>::value)
    return ew_one_i32<OP>(x, y, i, alpha, beta, seed);
  else
    return ew_one<OP, T>(x, y, i, alpha, beta, seed);
}

constexpr bool ew_reads_a(int op) { return !(op == TT_EW_FILL || op == TT_EW_UNIFORM); }
constexpr bool ew_reads_b(int op) {
  return op == TT_EW_ADD || op == TT_EW_SUB || op == TT_EW_RELU_BWD || op == TT_EW_SIGMOID_BWD;
}

// Any alignment: one element per thread and step of a grid-stride loop.
template <int OP, typename T>
__device__ void ew_scalar_loop(T* c, const T* a, const T* b, int64_t n, double alpha, double beta,
                               uint64_t seed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    c[i] = ew_elem<OP, T>(ew_reads_a(OP) ? a[i] : T(0), ew_reads_b(OP) ? b[i] : T(0), i, alpha, beta, seed);
}

// 16-byte aligned operands: 16 bytes of each operand per thread, a grid of
// one thread per 16-byte word up to 2^24 workgroups (a grid-stride loop
// beyond), and the n % V tail elements done one by one by the first threads.
// One word per thread over the full grid measured fastest for a 1 GiB f32
// scale (6.5 TB/s, against 5.3-5.7 with four words per thread or the grid
// capped at 65536 workgroups).  NT: non-temporal loads and stores, for
// operands too large to stay in the 256 MB Infinity Cache (1 GiB: 6.5 against
// 6.2 TB/s); smaller ones keep ordinary accesses (64 MiB, repeated: 6.8
// against 6.0 TB/s).
typedef unsigned int ew_u32x4 __attribute__((ext_vector_type(4)));
constexpr int64_t kEwMaxBlocks = int64_t(1) << 24;
constexpr int64_t kEwNtBytes = int64_t(256) << 20;
template <bool NT>
__device__ __forceinline__ ew_u32x4 ew_ld16(const void* p, int64_t v) {
  const ew_u32x4* q = reinterpret_cast<const ew_u32x4*>(p) + v;
  if constexpr (NT) return __builtin_nontemporal_load(q);
  return *q;
}
template <bool NT>
__device__ __forceinline__ void ew_st16(void* p, int64_t v, ew_u32x4 x) {
  ew_u32x4* q = reinterpret_cast<ew_u32x4*>(p) + v;
  if constexpr (NT)
    __builtin_nontemporal_store(x, q);
  else
    *q = x;
}
template <int OP, typename T, bool NT>
__device__ void ew_vec_loop(T* c, const T* a, const T* b, int64_t n, double alpha, double beta, uint64_t seed) {
  constexpr int V = 16 / sizeof(T);
  union Pack {
    ew_u32x4 u;
    T e[V];
  };
  const int64_t nv = n / V;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t v = t0; v < nv; v += stride) {
    Pack pa, pb, pc;
    pa.u = ew_u32x4{0, 0, 0, 0};
    pb.u = ew_u32x4{0, 0, 0, 0};
    if constexpr (ew_reads_a(OP)) pa.u = ew_ld16<NT>(a, v);
    if constexpr (ew_reads_b(OP)) pb.u = ew_ld16<NT>(b, v);
#pragma unroll
    for (int e = 0; e < V; ++e) pc.e[e] = ew_elem<OP, T>(pa.e[e], pb.e[e], v * V + e, alpha, beta, seed);
    ew_st16<NT>(c, v, pc.u);
  }
  const int64_t i = nv * V + t0;
  if (i < n)
    c[i] = ew_elem<OP, T>(ew_reads_a(OP) ? a[i] : T(0), ew_reads_b(OP) ? b[i] : T(0), i, alpha, beta, seed);
}

// MODE 0: one element per thread (any alignment); 1: 16-byte words; 2: 16-byte
// words, non-temporal.
template <int MODE, int OP, typename T>
__device__ __forceinline__ void ew_run(T* c, const T* a, const T* b, int64_t n, double alpha, double beta,
                                       uint64_t seed) {
  if constexpr (MODE == 0)
    ew_scalar_loop<OP, T>(c, a, b, n, alpha, beta, seed);
  else
    ew_vec_loop<OP, T, MODE == 2>(c, a, b, n, alpha, beta, seed);
}

// The op is uniform over the launch: one switch outside the loop, each case a
// loop specialised for its op.
template <int MODE, typename T>
__device__ void ew_dispatch(int op, T* c, const T* a, const T* b, int64_t n, double alpha, double beta,
                            uint64_t seed) {
  switch (op) {
    case TT_EW_ADD: ew_run<MODE, TT_EW_ADD, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_SUB: ew_run<MODE, TT_EW_SUB, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_FILL: ew_run<MODE, TT_EW_FILL, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_NEG: ew_run<MODE, TT_EW_NEG, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_SCALE: ew_run<MODE, TT_EW_SCALE, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_RELU: ew_run<MODE, TT_EW_RELU, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_RELU_BWD: ew_run<MODE, TT_EW_RELU_BWD, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_SIGMOID: ew_run<MODE, TT_EW_SIGMOID, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_SIGMOID_BWD: ew_run<MODE, TT_EW_SIGMOID_BWD, T>(c, a, b, n, alpha, beta, seed); break;
    case TT_EW_UNIFORM: ew_run<MODE, TT_EW_UNIFORM, T>(c, a, b, n, alpha, beta, seed); break;
    default: break;
  }
}

template <typename T, bool NT>
__global__ __launch_bounds__(256) void k_elementwise(int op, T* c, const T* a, const T* b, int64_t n,
                                                     double alpha, double beta, uint64_t seed) {
  ew_dispatch<NT ? 2 : 1, T>(op, c, a, b, n, alpha, beta, seed);
}
template <typename T>
__global__ __launch_bounds__(256) void k_elementwise_scalar(int op, T* c, const T* a, const T* b, int64_t n,
                                                            double alpha, double beta, uint64_t seed) {
  ew_dispatch<0, T>(op, c, a, b, n, alpha, beta, seed);
}

// scale * N(0,1) by Box-Muller on two 24-bit uniforms of splitmix64(seed, i).
template <typename T>
__global__ void k_fill_normal(T* dst, int64_t n, uint64_t seed, float scale) {
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint64_t h = splitmix64(seed * 0x100000001B3ull ^ splitmix64((uint64_t)i));
    float u1 = ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
    float u2 = (float)((h >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    Num<T>::st(dst, i, (double)(z * scale));
  }
}

static int grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

}  // namespace tt

using namespace tt;

extern "C" {

const char* tt_last_error(void) { return g_err.c_str(); }
const char* tt_version(void) { return "tinytensor-mi355x 0.1 (gfx950)"; }

int tt_device_count(int* n) {
  if (!n) return fail(TT_ERR_ARG, "tt_device_count: null pointer");
  int c = 0;
  if (hipGetDeviceCount(&c) != hipSuccess) {
    (void)hipGetLastError();
    c = 0;
  }
  *n = c;
  return ok();
}

int tt_init(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_inited) {
    if (device != g_device) return fail(TT_ERR_ARG, "tt_init: library already bound to another device");
    return TT_OK;
  }
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return fail(TT_ERR_HIP, "tt_init: no HIP device available");
  }
  if (device < 0 || device >= n) return fail(TT_ERR_ARG, "tt_init: device index out of range");
  if (device >= kMaxDevices) return fail(TT_ERR_ARG, "tt_init: device index above the supported 64");
  TT_HIP(hipSetDevice(device));
  // once per device, with that device current: its copy of the static scratch
  void* sp = nullptr;
  TT_HIP(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
  g_scratch_ptr[device] = sp;
  int cus = 0;
  TT_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  g_cus = cus > 0 ? cus : 1;
  // Default priority on purpose: one stream, ordinary priority.
  TT_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  g_device = device;
  g_inited.store(true, std::memory_order_release);
  return ok();
}

void* tt_stream(void) {
  if (ensure_init() != TT_OK) return nullptr;
  return (void*)g_stream;
}

int tt_stream_create(void** stream) {
  if (!stream) return fail(TT_ERR_ARG, "tt_stream_create: null pointer");
  *stream = nullptr;
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s;
  // Default priority on purpose, like the library stream.
  TT_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = (void*)s;
  return ok();
}

int tt_stream_sync(void* stream) {
  int rc = ensure_init();
  if (rc) return rc;
  TT_HIP(hipStreamSynchronize(stream_or_default(stream)));
  return ok();
}

int tt_stream_destroy(void* stream) {
  if (!stream) return TT_OK;
  if (stream == (void*)g_stream) return fail(TT_ERR_ARG, "tt_stream_destroy: the library stream is not the caller's");
  const int rc = g_ws.release_stream(stream);  // waits for the stream
  if (rc) return rc;
  TT_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return ok();
}

int tt_malloc(void** ptr, size_t bytes) {
  if (!ptr) return fail(TT_ERR_ARG, "tt_malloc: null pointer");
  *ptr = nullptr;
  int rc = ensure_init();
  if (rc) return rc;
  rc = g_blocks.alloc(bytes, ptr);
  if (rc) return rc;
  return ok();
}

int tt_free(void* ptr) {
  if (!ptr) return TT_OK;
  // Work queued on the library stream that still reads this block runs
  // before any later user of the block on the same stream.
  if (!g_blocks.release(ptr)) return fail(TT_ERR_ARG, "tt_free: pointer not from tt_malloc");
  return TT_OK;
}

int tt_empty_cache(void) {
  if (!g_inited.load(std::memory_order_acquire)) return TT_OK;
  TT_HIP(hipStreamSynchronize(g_stream));
  const int rc = g_ws.release_all();
  g_blocks.trim();
  return rc ? rc : ok();
}

int tt_mem_stats(size_t* in_use, size_t* cached) {
  g_blocks.stats(in_use, cached);
  return TT_OK;
}

// tt_memcpy_h2d / tt_memcpy_d2h: staging.hip

int tt_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return TT_OK;
  if (!dst || !src) return fail(TT_ERR_ARG, "tt_memcpy_d2d: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  TT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  return ok();
}

int tt_memset(void* ptr, int value, size_t bytes) {
  if (bytes == 0) return TT_OK;
  if (!ptr) return fail(TT_ERR_ARG, "tt_memset: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  TT_HIP(hipMemsetAsync(ptr, value, bytes, g_stream));
  return ok();
}

int tt_sync(void) {
  int rc = ensure_init();
  if (rc) return rc;
  TT_HIP(hipStreamSynchronize(g_stream));
  return ok();
}

int tt_event_create(void** ev) {
  if (!ev) return fail(TT_ERR_ARG, "tt_event_create: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  hipEvent_t e;
  TT_HIP(hipEventCreate(&e));
  *ev = (void*)e;
  return ok();
}
int tt_event_record(void* ev, void* stream) {
  if (!ev) return fail(TT_ERR_ARG, "tt_event_record: null event");
  TT_HIP(hipEventRecord((hipEvent_t)ev, stream_or_default(stream)));
  return ok();
}
int tt_event_elapsed_ms(float* ms, void* start, void* stop) {
  if (!ms || !start || !stop) return fail(TT_ERR_ARG, "tt_event_elapsed_ms: null pointer");
  TT_HIP(hipEventSynchronize((hipEvent_t)stop));
  TT_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return ok();
}
int tt_event_destroy(void* ev) {
  if (!ev) return TT_OK;
  TT_HIP(hipEventDestroy((hipEvent_t)ev));
  return ok();
}

int tt_set_launch_events(void** evs, int n) {
  std::lock_guard<std::mutex> lk(g_ev_mu);
  g_launch_events.clear();
  g_launch_next = 0;
  if (evs && n > 0) g_launch_events.assign(evs, evs + n);
  g_launch_left.store(g_launch_events.size(), std::memory_order_release);
  return TT_OK;
}

int tt_launch_events_recorded(int* n) {
  if (!n) return fail(TT_ERR_ARG, "tt_launch_events_recorded: null pointer");
  std::lock_guard<std::mutex> lk(g_ev_mu);
  *n = (int)g_launch_next;
  return TT_OK;
}

// Streams chunk16 16-byte words per workgroup (workgroup b: words
// [b * chunk16, min((b + 1) * chunk16, n16))), 16 non-temporal loads in
// flight per thread (the fastest streaming-read pattern measured on the
// MI355X: 7.1-7.2 TB/s over 8 GiB, against 6.2-6.4 TB/s with ordinary loads).
typedef unsigned int probe_u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_read_probe(const probe_u32x4* __restrict__ p, int64_t n16,
                                                     int64_t chunk16, float* out) {
  const int64_t lo = (int64_t)blockIdx.x * chunk16;
  const int64_t hi = lo + chunk16 < n16 ? lo + chunk16 : n16;
  float acc = 0.f;
  for (int64_t i = lo + threadIdx.x; i < hi; i += 256 * 16) {
    probe_u32x4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u)
      v[u] = i + 256 * u < hi ? __builtin_nontemporal_load(p + i + 256 * u) : probe_u32x4{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < 16; ++u)
      acc += (__uint_as_float(v[u].x) + __uint_as_float(v[u].y)) + (__uint_as_float(v[u].z) + __uint_as_float(v[u].w));
  }
  if (acc == 1234.5f) out[0] = acc;  // keeps the loads; practically never taken
}

int tt_read_probe(const void* buf, int64_t bytes, float* out, void* stream) {
  if (bytes < 0 || bytes % 16 != 0) return fail(TT_ERR_ARG, "tt_read_probe: bytes must be a multiple of 16");
  if (bytes == 0) return TT_OK;
  if (!buf || !out || ((uintptr_t)buf & 15)) return fail(TT_ERR_ARG, "tt_read_probe: null or unaligned pointer");
  int rc = ensure_init();
  if (rc) return rc;
  const int64_t n16 = bytes / 16, chunk16 = (int64_t(256) << 10) / 16;
  const int64_t nb = (n16 + chunk16 - 1) / chunk16;
  if (!grid_fits(nb, 256)) return fail(TT_ERR_ARG, "tt_read_probe: too large");
  hipStream_t s = stream_or_default(stream);
  hipLaunchKernelGGL(k_read_probe, dim3((unsigned)nb), dim3(256), 0, s, (const probe_u32x4*)buf, n16, chunk16, out);
  TT_LAUNCHED("read probe launch", s);
  return ok();
}

int tt_elementwise(int op, int dtype, void* c, const void* a, const void* b, int64_t n,
                   double alpha, double beta, uint64_t seed, void* stream) {
  if (n < 0) return fail(TT_ERR_ARG, "tt_elementwise: negative size");
  if (n == 0) return TT_OK;
  if (op < TT_EW_ADD || op > TT_EW_UNIFORM) return fail(TT_ERR_ARG, "tt_elementwise: bad op");
  bool need_a = !(op == TT_EW_FILL || op == TT_EW_UNIFORM);
  bool need_b = (op == TT_EW_ADD || op == TT_EW_SUB || op == TT_EW_RELU_BWD || op == TT_EW_SIGMOID_BWD);
  if (!c || (need_a && !a) || (need_b && !b)) return fail(TT_ERR_ARG, "tt_elementwise: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  auto aligned = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  const bool vec = aligned(c) && (!need_a || aligned(a)) && (!need_b || aligned(b));
  auto launch = [&](auto tag) {
    using T = decltype(tag);
    if (vec) {
      const int64_t nv = n / (int64_t)(16 / sizeof(T));
      int64_t g = (nv + 255) / 256;
      g = g < 1 ? 1 : (g > kEwMaxBlocks ? kEwMaxBlocks : g);
      const int64_t bytes = n * (int64_t)sizeof(T) * (1 + (need_a ? 1 : 0) + (need_b ? 1 : 0));
      if (bytes >= kEwNtBytes)
        hipLaunchKernelGGL((k_elementwise<T, true>), dim3((unsigned)g), dim3(256), 0, s, op, (T*)c,
                           (const T*)a, (const T*)b, n, alpha, beta, seed);
      else
        hipLaunchKernelGGL((k_elementwise<T, false>), dim3((unsigned)g), dim3(256), 0, s, op, (T*)c,
                           (const T*)a, (const T*)b, n, alpha, beta, seed);
    } else {
      hipLaunchKernelGGL(k_elementwise_scalar<T>, dim3(grid_for(n)), dim3(256), 0, s, op, (T*)c, (const T*)a,
                         (const T*)b, n, alpha, beta, seed);
    }
  };
  switch (dtype) {
    case TT_F32: launch(float{}); break;
    case TT_F64: launch(double{}); break;
    case TT_I32: launch(int32_t{}); break;
    case TT_BF16: launch(uint16_t{}); break;
    default:
      return fail(TT_ERR_ARG, "tt_elementwise: bad dtype");
  }
  TT_LAUNCH_CHECK("tt_elementwise");
  return ok();
}

int tt_fill_normal(int dtype, void* dst, int64_t n, uint64_t seed, float scale, void* stream) {
  if (n < 0) return fail(TT_ERR_ARG, "tt_fill_normal: negative size");
  if (n == 0) return TT_OK;
  if (!dst) return fail(TT_ERR_ARG, "tt_fill_normal: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  int g = grid_for(n);
  if (dtype == TT_F32)
    hipLaunchKernelGGL(k_fill_normal<float>, dim3(g), dim3(256), 0, s, (float*)dst, n, seed, scale);
  else if (dtype == TT_BF16)
    hipLaunchKernelGGL(k_fill_normal<uint16_t>, dim3(g), dim3(256), 0, s, (uint16_t*)dst, n, seed, scale);
  else
    return fail(TT_ERR_ARG, "tt_fill_normal: dtype must be f32 or bf16");
  TT_LAUNCH_CHECK("tt_fill_normal");
  return ok();
}

}  // extern "C"
