// Row softmax over the last axis of a row-major [rows, cols] fp32 matrix.
//
// Replaces SoftmaxForward (Task3/Tinytensor/src/Layers.cu:324-349), which
// runs five passes -- cudaChannelMax / Sub / Exp / Sum / Div of
// src/Layers_kernels.cu:189-257, the max and the sum each a host loop of
// thrust calls, one per row -- with one kernel that keeps the row in
// registers (one HBM read and one write per element) or, for long rows,
// streams it twice.  Same arithmetic per row as the reference:
//   m = max_c x[c];  e[c] = exp(x[c] - m);  s = sum_c e[c];  y[c] = e[c] / s
// (the sum's association order differs: lanes, then a butterfly).
//
// Shapes of work, all coalesced (lane t of a row group reads columns
// t, t + G, t + 2G, ... for group width G):
//   cols <= 64:   G = the next power of two >= cols lanes per row, 64 / G
//                 rows per wave, one element per lane;
//   cols <= 2048: one wave per row, up to 32 elements per lane in registers;
//   cols <= 8192 (and longer rows that are not 16-byte aligned, up to 65536):
//                 one workgroup of 4 or 16 waves per row, up to 64 elements
//                 per lane in registers, partials through LDS;
//   longer aligned rows, up to 2 M columns: the row is split over up to 64
//                 workgroups that each hold their chunk in registers and
//                 exchange (max, sum) partials through device memory (one
//                 HBM read and one write per element);
//   the rest:     one workgroup of 16 waves per row; pass 1 keeps a running
//                 (max, sum) per lane, pass 2 rereads the row and writes it.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "tt_internal.h"

namespace tt {

namespace {

constexpr int kBlock = 256;  // four waves

// e^x as 2^(x log2 e) on v_exp_f32 (relative error a few 1e-7 for |x| < 10,
// growing with |x|; the softmax outputs those terms feed are e^x / s small).
__device__ __forceinline__ float ex(float x) { return __expf(x); }

// Every element is read and written once (twice read for the longest rows),
// so the loads and stores are marked non-temporal: 5-14 % faster on the
// MI355X than ordinary ones for 1024, 65536 and 262144-column rows.
__device__ __forceinline__ float ld(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st(float* p, float v) { __builtin_nontemporal_store(v, p); }

// max / sum over the G lanes of a row group (G a power of two <= 64)
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// cols <= G: one element per lane, 64 / G rows per wave.
template <int G>
__global__ __launch_bounds__(kBlock) void k_softmax_small(const float* __restrict__ x, float* y, int64_t rows,
                                                         int cols) {
  constexpr int RPB = kBlock / G;  // rows per block
  const int t = threadIdx.x % G;
  for (int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / G; r < rows; r += (int64_t)gridDim.x * RPB) {
    const bool in = t < cols;
    const float v = in ? ld(&x[r * cols + t]) : -INFINITY;
    const float m = group_max<G>(v);
    const float e = in ? ex(v - m) : 0.f;
    const float s = group_sum<G>(e);
    if (in) st(&y[r * cols + t], e / s);
  }
}

// cols <= 64 * NE: one wave per row, NE elements per lane in registers.
template <int NE>
__global__ __launch_bounds__(kBlock) void k_softmax_reg(const float* __restrict__ x, float* y, int64_t rows,
                                                       int cols) {
  constexpr int WPB = kBlock / 64;
  const int t = threadIdx.x & 63;
  for (int64_t r = (int64_t)blockIdx.x * WPB + threadIdx.x / 64; r < rows; r += (int64_t)gridDim.x * WPB) {
    const float* xr = x + r * cols;
    float v[NE];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int c = t + 64 * i;
      v[i] = c < cols ? ld(&xr[c]) : -INFINITY;
      m = fmaxf(m, v[i]);
    }
    m = group_max<64>(m);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      v[i] = t + 64 * i < cols ? ex(v[i] - m) : 0.f;
      s += v[i];
    }
    s = group_sum<64>(s);
    float* yr = y + r * cols;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int c = t + 64 * i;
      if (c < cols) st(&yr[c], v[i] / s);
    }
  }
}

// cols <= 64 W NE: one workgroup of W waves per row, NE elements per lane in
// registers; the waves' partial max / sum meet in LDS.
template <int NE, int W>
__global__ __launch_bounds__(64 * W) void k_softmax_block(const float* __restrict__ x, float* y, int64_t rows,
                                                         int cols) {
  __shared__ float red_m[W], red_s[W];
  const int t = threadIdx.x, w = t >> 6;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {  // uniform per workgroup
    const float* xr = x + r * cols;
    float v[NE];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int c = t + 64 * W * i;
      v[i] = c < cols ? ld(&xr[c]) : -INFINITY;
      m = fmaxf(m, v[i]);
    }
    m = group_max<64>(m);
    if ((t & 63) == 0) red_m[w] = m;
    __syncthreads();
    m = red_m[0];
#pragma unroll
    for (int k = 1; k < W; ++k) m = fmaxf(m, red_m[k]);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      v[i] = t + 64 * W * i < cols ? ex(v[i] - m) : 0.f;
      s += v[i];
    }
    s = group_sum<64>(s);
    if ((t & 63) == 0) red_s[w] = s;
    __syncthreads();
    s = red_s[0];
#pragma unroll
    for (int k = 1; k < W; ++k) s += red_s[k];
    float* yr = y + r * cols;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int c = t + 64 * W * i;
      if (c < cols) st(&yr[c], v[i] / s);
    }
    __syncthreads();  // red_m / red_s are reused by the next row
  }
}

// Any cols: one workgroup of W waves per row, two passes, four loads in
// flight per lane.  Pass 1: per lane a running max m and a (compensated) sum
// s of exp(x - m), rescaled when m grows; lanes, then waves (through LDS),
// merge their pairs to the row's (m, s).  Pass 2: y = exp(x - m) / s.
template <int W>
__global__ __launch_bounds__(64 * W) void k_softmax_stream(const float* __restrict__ x, float* y, int64_t rows,
                                                          int64_t cols) {
  constexpr int U = 4, STEP = 64 * W * U;
  __shared__ float red_m[W], red_s[W];
  const int t = threadIdx.x, w = t >> 6;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {  // uniform per workgroup
    const float* xr = x + r * cols;
    // s carries a Kahan compensation e: a lane adds cols / (64 W) terms in
    // sequence, which in plain fp32 would cost about that many roundings
    float m = -INFINITY, s = 0.f, e = 0.f;
    auto add = [&](float a) {
      const float yv = a - e, tv = s + yv;
      e = (tv - s) - yv;
      s = tv;
    };
    for (int64_t c0 = t; c0 < cols; c0 += STEP) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = c0 + 64 * W * u < cols ? ld(&xr[c0 + 64 * W * u]) : -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (v[u] > m) {
          const float f = ex(m - v[u]);  // m = -inf: exp(-inf) = 0
          s *= f;
          e *= f;
          add(1.f);
          m = v[u];
        } else if (v[u] != -INFINITY) {  // (-inf) - (-inf) would be NaN; exp(-inf - m) = 0
          add(ex(v[u] - m));
        }
      }
    }
    s -= e;
    // merge (m, s) pairs: a pair that saw no finite value has m = -inf and
    // s = 0 and adds nothing (NaN rows propagate NaN, as the reference's
    // x - max does)
    float rm = group_max<64>(m);
    s = group_sum<64>(s == 0.f ? 0.f : s * ex(m - rm));
    if ((t & 63) == 0) {
      red_m[w] = rm;
      red_s[w] = s;
    }
    __syncthreads();
    float bm = red_m[0];
#pragma unroll
    for (int k = 1; k < W; ++k) bm = fmaxf(bm, red_m[k]);
    float bs = 0.f;
#pragma unroll
    for (int k = 0; k < W; ++k) bs += red_s[k] == 0.f ? 0.f : red_s[k] * ex(red_m[k] - bm);
    float* yr = y + r * cols;
    for (int64_t c0 = t; c0 < cols; c0 += STEP) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = c0 + 64 * W * u < cols ? ld(&xr[c0 + 64 * W * u]) : 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (c0 + 64 * W * u < cols) st(&yr[c0 + 64 * W * u], ex(v[u] - bm) / bs);
    }
    __syncthreads();  // red_m / red_s are reused by the next row
  }
}

// Rows split over workgroups.  Workgroup id = row * nchunk + chunk holds
// columns [chunk * CW, chunk * CW + CW) of its row in registers (lane t: the
// 16-byte vectors at 4 t + 1024 k, k < NE4), forms the chunk's max m_c and
// sum s_c of exp(x - m_c), and publishes them as two 64-bit words
// (generation << 32 | float bits) in `slots` (two words per chunk, row
// major).  It then waits until every chunk of its row has published under
// the current generation, merges the partials into the row's (M, S) and
// writes y = exp(x - m_c) * (exp(m_c - M) / S): one read and one write of
// each element.  The generation is new for every launch on a slot buffer
// (the host counts the buffer's uses and zero-fills a new one), so words of
// earlier launches never match.  Each word is one relaxed agent-scope
// atomic (coherent across the XCDs' L2s); no other data crosses workgroups,
// so no fence is needed.
//
// The wait cannot deadlock: workgroups are dispatched in id order, so every
// row below the one at the dispatch front has all of its (at most 64)
// chunks resident or done, finishes, and frees slots for the front row.  It
// is bounded all the same: after about 2^20 polls a workgroup stops waiting
// and writes NaN for its chunk.  A workgroup writes only the chunk it has
// already read, so x == y (in place) is fine.
constexpr int kSplitMaxChunks = 64;
typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int NE4>
__global__ __launch_bounds__(kBlock) void k_softmax_split(const float* x, float* y, int64_t cols, int nchunk,
                                                         unsigned long long* slots, unsigned gen) {
  constexpr int CW = 1024 * NE4;  // columns per chunk
  __shared__ float red_m[4], red_s[4];
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
  const int64_t row = (int64_t)blockIdx.x / nchunk;
  const int chunk = (int)((int64_t)blockIdx.x - row * nchunk);
  const int64_t c0 = (int64_t)chunk * CW;
  const int64_t rem = cols - c0;  // > 0; columns of the row from this chunk on
  const float* xr = x + row * cols + c0;
  float* yr = y + row * cols + c0;
  f32x4v v[NE4];
#pragma unroll
  for (int k = 0; k < NE4; ++k) {
    const int c = 4 * t + 1024 * k;  // cols % 4 == 0: a vector is wholly inside or outside the row
    v[k] = c < rem ? __builtin_nontemporal_load(reinterpret_cast<const f32x4v*>(xr + c))
                   : f32x4v{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  }
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < NE4; ++k) m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
  m = group_max<64>(m);
  if (l == 0) red_m[w] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  // a chunk with no finite value (m = -inf) has every exp 0 and s = 0
  const float mb = m == -INFINITY ? 0.f : m;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NE4; ++k) {
    v[k].x = ex(v[k].x - mb);
    v[k].y = ex(v[k].y - mb);
    v[k].z = ex(v[k].z - mb);
    v[k].w = ex(v[k].w - mb);
    s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
  }
  s = group_sum<64>(s);
  if (l == 0) red_s[w] = s;
  __syncthreads();
  s = (red_s[0] + red_s[1]) + (red_s[2] + red_s[3]);

  unsigned long long* rs = slots + 2 * row * nchunk;
  const unsigned long long tag = (unsigned long long)gen << 32;
  if (t == 0) {
    __hip_atomic_store(rs + 2 * chunk, tag | __float_as_uint(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(rs + 2 * chunk + 1, tag | __float_as_uint(s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // thread j < nchunk waits for chunk j's partial and merges it
  float pm = -INFINITY, ps = 0.f;
  bool ok = true;
  if (t < nchunk) {
    unsigned long long a = 0, b = 0;
    for (int polls = 0;; ++polls) {
      a = __hip_atomic_load(rs + 2 * t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      b = __hip_atomic_load(rs + 2 * t + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((unsigned)(a >> 32) == gen && (unsigned)(b >> 32) == gen) break;
      if (polls >= (1 << 20)) {
        ok = false;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    pm = __uint_as_float((unsigned)a);
    ps = __uint_as_float((unsigned)b);
  }
  // (M, S) over the workgroup's threads; pairs with s = 0 add nothing
  float M = group_max<64>(pm);
  float S = group_sum<64>(ps == 0.f ? 0.f : ps * ex(pm - M));
  const int bad = __syncthreads_or(!ok);
  if (l == 0) {
    red_m[w] = M;
    red_s[w] = S;
  }
  __syncthreads();
  M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  S = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) S += red_s[k] == 0.f ? 0.f : red_s[k] * ex(red_m[k] - M);
  // exp(m - M) / S; a row with no finite value gives NaN (0 / 0 and
  // -inf - -inf), as the reference's x - max does
  const float f = bad ? NAN : (m == -INFINITY && M != -INFINITY ? 0.f : ex(m - M)) / S;
#pragma unroll
  for (int k = 0; k < NE4; ++k) {
    const int c = 4 * t + 1024 * k;
    if (c < rem) __builtin_nontemporal_store(v[k] * f, reinterpret_cast<f32x4v*>(yr + c));
  }
}

int blocks_for(int64_t rows, int64_t rows_per_block) {
  const int64_t b = (rows + rows_per_block - 1) / rows_per_block;
  return (int)(b < 65536 ? b : 65536);  // grid-stride beyond this
}

}  // namespace

}  // namespace tt

using namespace tt;

extern "C" int tt_softmax_rows_f32(const float* x, float* y, int64_t rows, int64_t cols, void* stream) {
  if (rows < 0 || cols < 0) return fail(TT_ERR_ARG, "tt_softmax_rows_f32: negative size");
  if (rows == 0 || cols == 0) return ok();
  if (!x || !y) return fail(TT_ERR_ARG, "tt_softmax_rows_f32: null pointer");
  if (cols > (int64_t(1) << 31) - 1) return fail(TT_ERR_ARG, "tt_softmax_rows_f32: row too long");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  // Long 16-byte aligned rows: split over workgroups (k_softmax_split), with
  // chunks of 4096 / 8192 / 16384 / 32768 columns for rows up to 16 Ki /
  // 64 Ki / 256 Ki / 2 Mi columns (measured best on the MI355X for each).
  const bool aligned = cols % 4 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0;
  if (aligned && cols > 8192 && cols <= int64_t(kSplitMaxChunks) * 32768) {
    const int ne4 = cols <= 16384 ? 4 : cols <= 65536 ? 8 : cols <= 262144 ? 16 : 32;
    const int64_t cw = 1024 * ne4, nchunk = (cols + cw - 1) / cw;
    if (grid_fits(rows * nchunk, kBlock)) {  // else the grid-stride kernels below
      unsigned long long* slots = nullptr;
      uint64_t uses = 0;
      const size_t bytes = (size_t)(rows * nchunk) * 2 * sizeof(unsigned long long);
      WorkspaceLease ws;  // held until the kernel that reads the slots is queued
      if ((rc = ws.get(s, kWsSoftmaxPartials, bytes, (void**)&slots, &uses))) return rc;
      const unsigned gen = (unsigned)(uses % 0xffffffffull) + 1;  // 1 .. 2^32 - 1
      if (gen == 1 &&  // a new buffer (or a wrapped count): no word may hold a live generation
          (rc = tt_elementwise(TT_EW_FILL, TT_F32, slots, nullptr, nullptr, (int64_t)(bytes / 4), 0.0, 0.0, 0, s)))
        return rc;
      const dim3 grid((unsigned)(rows * nchunk)), blk(kBlock);
      const int n = (int)nchunk;
      switch (ne4) {
        case 4: hipLaunchKernelGGL(k_softmax_split<4>, grid, blk, 0, s, x, y, cols, n, slots, gen); break;
        case 8: hipLaunchKernelGGL(k_softmax_split<8>, grid, blk, 0, s, x, y, cols, n, slots, gen); break;
        case 16: hipLaunchKernelGGL(k_softmax_split<16>, grid, blk, 0, s, x, y, cols, n, slots, gen); break;
        default: hipLaunchKernelGGL(k_softmax_split<32>, grid, blk, 0, s, x, y, cols, n, slots, gen); break;
      }
      TT_LAUNCHED("tt_softmax_rows_f32", s);
      return ok();
    }
  }
  const int c = (int)cols;
#define TT_SMALL(G)                                                                                 \
  hipLaunchKernelGGL(k_softmax_small<G>, dim3(blocks_for(rows, kBlock / G)), dim3(kBlock), 0, s, x, y, \
                     rows, c)
#define TT_REG(NE) \
  hipLaunchKernelGGL(k_softmax_reg<NE>, dim3(blocks_for(rows, kBlock / 64)), dim3(kBlock), 0, s, x, y, rows, c)
#define TT_BLOCK(NE, W) \
  hipLaunchKernelGGL((k_softmax_block<NE, W>), dim3(blocks_for(rows, 1)), dim3(64 * W), 0, s, x, y, rows, c)
  if (cols <= 1) TT_SMALL(1);
  else if (cols <= 2) TT_SMALL(2);
  else if (cols <= 4) TT_SMALL(4);
  else if (cols <= 8) TT_SMALL(8);
  else if (cols <= 16) TT_SMALL(16);
  else if (cols <= 32) TT_SMALL(32);
  else if (cols <= 64) TT_SMALL(64);
  else if (cols <= 128) TT_REG(2);
  else if (cols <= 256) TT_REG(4);
  else if (cols <= 512) TT_REG(8);
  else if (cols <= 1024) TT_REG(16);
  else if (cols <= 2048) TT_REG(32);
  else if (cols <= 4096) TT_BLOCK(16, 4);
  else if (cols <= 8192) TT_BLOCK(32, 4);
  else if (cols <= 16384) TT_BLOCK(16, 16);
  else if (cols <= 32768) TT_BLOCK(32, 16);
  else if (cols <= 65536) TT_BLOCK(64, 16);
  else
    hipLaunchKernelGGL(k_softmax_stream<16>, dim3(blocks_for(rows, 1)), dim3(1024), 0, s, x, y, rows, cols);
#undef TT_SMALL
#undef TT_REG
#undef TT_BLOCK
  TT_LAUNCHED("tt_softmax_rows_f32", s);
  return ok();
}

// ---------------------------------------------------------------- cross-entropy on softmax rows
// The loss and gradient that follow SoftmaxForward in the reference's
// softmax cross-entropy (src/Layers.cu:383-423, kernels
// src/Layers_kernels.cu:260-282): loss = sum_i -log p[i][label_i], and
// grad = p - onehot(label).  A label outside [0, cols) makes its row's loss
// term NaN and subtracts nothing from its gradient row (the reference reads
// out of bounds there).
namespace tt {
namespace {

constexpr int kCeThreads = 1024;

// One workgroup: each thread sums the rows t, t + 1024, ... in double, then a
// fixed-order tree over the workgroup, so the result does not depend on
// timing.
__global__ __launch_bounds__(kCeThreads) void k_ce_loss(const float* __restrict__ p, const int* __restrict__ labels,
                                                        float* __restrict__ loss, int64_t rows, int64_t cols) {
  __shared__ double part[kCeThreads];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < rows; i += kCeThreads) {
    const int lab = labels[i];
    acc += (lab >= 0 && lab < cols) ? -log((double)p[i * cols + lab]) : (double)NAN;
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kCeThreads / 2; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss[0] = (float)part[0];
}

__global__ __launch_bounds__(256) void k_ce_backward(const float* __restrict__ p, const int* __restrict__ labels,
                                                     float* __restrict__ grad, int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t i = e / cols, j = e - i * cols;
    grad[e] = p[e] - (labels[i] == j ? 1.f : 0.f);
  }
}

}  // namespace
}  // namespace tt

extern "C" int tt_cross_entropy_f32(const float* p, const int* labels, float* loss, int64_t rows, int64_t cols,
                                    void* stream) {
  using namespace tt;
  if (rows < 0 || cols < 0) return fail(TT_ERR_ARG, "tt_cross_entropy_f32: negative size");
  if (!loss || (rows > 0 && (!p || !labels || cols == 0)))
    return fail(TT_ERR_ARG, "tt_cross_entropy_f32: null pointer or no columns");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  hipLaunchKernelGGL(k_ce_loss, dim3(1), dim3(kCeThreads), 0, s, p, labels, loss, rows, cols);
  TT_LAUNCHED("tt_cross_entropy_f32", s);
  return ok();
}

extern "C" int tt_cross_entropy_backward_f32(const float* p, const int* labels, float* grad, int64_t rows,
                                             int64_t cols, void* stream) {
  using namespace tt;
  if (rows < 0 || cols < 0) return fail(TT_ERR_ARG, "tt_cross_entropy_backward_f32: negative size");
  if (rows == 0 || cols == 0) return ok();
  if (!p || !labels || !grad) return fail(TT_ERR_ARG, "tt_cross_entropy_backward_f32: null pointer");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  int64_t blocks = (rows * cols + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(k_ce_backward, dim3((unsigned)blocks), dim3(256), 0, s, p, labels, grad, rows, cols);
  TT_LAUNCHED("tt_cross_entropy_backward_f32", s);
  return ok();
}

