// Single-query decode attention for gfx950: o = softmax(s q K^T) V per (b, h).
//
// The reference's op chain with Lq = 1 (Q @ K^T -> * s -> softmax -> @ V,
// optimizer/operators.py:163-164, 234-239, 611-612, 416-419) is a pair of
// GEMVs over the K/V cache: about 1 flop per byte, so the kernel is bound by
// HBM bandwidth and is built to stream K and V exactly once.
//
// Split-KV: workgroup id = bh * nsplit + split owns keys [split*chunk, (split+1)*chunk)
// of one head.  Phase 1 streams its K rows (16-byte non-temporal loads, TPR
// threads per row, several rows in flight per thread) and writes the log2-domain scores
// to LDS; phase 2 reduces max and sum over the chunk; phase 3 streams the V
// rows and accumulates sum_j p_j V_j.  Each split writes a normalised partial
// (o_c, lse_c) in fp32; a combine kernel merges them by LSE rescaling:
//   lse = log2 sum_c 2^lse_c,  o = sum_c 2^(lse_c - lse) o_c.
// When one split covers a whole head, the split kernel writes o and lse
// itself and there is no combine launch.
#include <hip/hip_runtime.h>

#include <cmath>

#include "attn_common.h"
#include "attn_tiles.h"

namespace tt {

constexpr int DEC_THREADS = 256;
// Keys per split: the split kernel keeps the chunk's scores in LDS, and is
// built for chunks up to 1024 keys (4 KB of scores) and up to 8192 (32 KB).
constexpr int DEC_SMALL_CHUNK = 1024;
constexpr int DEC_MAX_CHUNK = 8192;

template <typename T> struct Vec16;  // 16 bytes of T as floats
template <> struct Vec16<u16> {
  static constexpr int N = 8;
  __device__ static void cvt(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <> struct Vec16<float> {
  static constexpr int N = 4;
  __device__ static void cvt(const uint4& v, float* f) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
};

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  // wave-level butterfly, then across the 4 waves through LDS
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float o = __shfl_xor(v, off, 64);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < DEC_THREADS / 64; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

// MAXC: largest chunk the LDS score buffer holds.  DIRECT (nsplit == 1): o
// and lse (natural log, may be null) are written here in the output type;
// otherwise the fp32 partials go to part_o / part_lse.
template <typename T, int D, int UNROLL, int MAXC, bool DIRECT>
__global__ __launch_bounds__(DEC_THREADS) void attn_decode_split_kernel(
    const T* __restrict__ q, const T* __restrict__ K, const T* __restrict__ V,
    float* __restrict__ part_o, float* __restrict__ part_lse, T* __restrict__ o, float* __restrict__ lse,
    int Lkv, int nsplit, int chunk, float sl2) {
  constexpr int EPT = Vec16<T>::N;     // elements per 16-byte load
  constexpr int TPR = D / EPT;         // threads per key row
  constexpr int RPP = DEC_THREADS / TPR;  // rows per pass
  __shared__ float sS[MAXC];
  __shared__ float sAcc[RPP * D];
  __shared__ float red[DEC_THREADS / 64];

  const int split = blockIdx.x % nsplit;
  const int64_t bh = blockIdx.x / nsplit;
  const int tid = threadIdx.x, col = tid % TPR, rsub = tid / TPR;
  const int kbeg = split * chunk;
  const int n = min(chunk, Lkv - kbeg);
  const T* Kh = K + (bh * Lkv + kbeg) * D + col * EPT;
  const T* Vh = V + (bh * Lkv + kbeg) * D + col * EPT;

  float qv[EPT];
  Vec16<T>::cvt(ldg16(q + bh * D + col * EPT), qv);
#pragma unroll
  for (int e = 0; e < EPT; ++e) qv[e] *= sl2;

  // Phase 1: scores s_j = (s log2 e) q . k_j
  for (int j0 = rsub; j0 < n; j0 += RPP * UNROLL) {
    uint4 kv[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int j = j0 + u * RPP;
      kv[u] = j < n ? ldg16_stream(Kh + (int64_t)j * D) : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      float kf[EPT];
      Vec16<T>::cvt(kv[u], kf);
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < EPT; ++e) dot += qv[e] * kf[e];
#pragma unroll
      for (int off = TPR / 2; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
      const int j = j0 + u * RPP;
      if (col == 0 && j < n) sS[j] = dot;
    }
  }
  __syncthreads();

  // Phase 2: max and sum over the chunk
  float mx = -INFINITY;
  for (int j = tid; j < n; j += DEC_THREADS) mx = fmaxf(mx, sS[j]);
  mx = block_reduce(mx, red, true);
  float sm = 0.f;
  for (int j = tid; j < n; j += DEC_THREADS) {
    const float p = fast_exp2(sS[j] - mx);
    sS[j] = p;
    sm += p;
  }
  sm = block_reduce(sm, red, false);  // its barriers also publish sS

  // Phase 3: acc = sum_j p_j V_j over this thread's rows
  float acc[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) acc[e] = 0.f;
  for (int j0 = rsub; j0 < n; j0 += RPP * UNROLL) {
    uint4 vv[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int j = j0 + u * RPP;
      vv[u] = j < n ? ldg16_stream(Vh + (int64_t)j * D) : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int j = j0 + u * RPP;
      const float p = j < n ? sS[j] : 0.f;
      float vf[EPT];
      Vec16<T>::cvt(vv[u], vf);
#pragma unroll
      for (int e = 0; e < EPT; ++e) acc[e] += p * vf[e];
    }
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e) sAcc[rsub * D + col * EPT + e] = acc[e];
  __syncthreads();
  const float inv = 1.f / sm;
  const int64_t pidx = bh * nsplit + split;
  for (int dd = tid; dd < D; dd += DEC_THREADS) {
    float s = 0.f;
#pragma unroll 8
    for (int r = 0; r < RPP; ++r) s += sAcc[r * D + dd];
    if constexpr (!DIRECT)
      part_o[pidx * D + dd] = s * inv;
    else if constexpr (sizeof(T) == 2)
      o[bh * D + dd] = f32_to_bf16(s * inv);
    else
      o[bh * D + dd] = s * inv;
  }
  if (tid == 0) {
    if constexpr (!DIRECT)
      part_lse[pidx] = mx + __log2f(sm);
    else if (lse)
      lse[bh] = (mx + __log2f(sm)) * kLn2;
  }
}

// One workgroup of D threads per (b, h): merge the nsplit partials.
template <typename T, int D>
__global__ __launch_bounds__(D) void attn_decode_combine_kernel(const float* __restrict__ part_o,
                                                                const float* __restrict__ part_lse,
                                                                T* __restrict__ o, float* __restrict__ lse,
                                                                int nsplit) {
  const int64_t bh = blockIdx.x;
  const int dd = threadIdx.x;
  const float* pl = part_lse + bh * nsplit;
  float mx = -INFINITY;
  for (int c = 0; c < nsplit; ++c) mx = fmaxf(mx, pl[c]);
  float sw = 0.f, acc = 0.f;
  for (int c = 0; c < nsplit; ++c) {
    const float wgt = fast_exp2(pl[c] - mx);
    sw += wgt;
    acc += wgt * part_o[(bh * nsplit + c) * D + dd];
  }
  const float val = acc / sw;
  if constexpr (sizeof(T) == 2)
    o[bh * D + dd] = f32_to_bf16(val);
  else
    o[bh * D + dd] = val;
  if (dd == 0 && lse) lse[bh] = (mx + __log2f(sw)) * kLn2;
}

template <typename T, int D>
static int launch_decode(const T* q, const T* k, const T* v, T* o, float* lse, int64_t BH, int64_t Lkv,
                         float scale, hipStream_t st) {
  // Split size: the longest split (fewer workgroups, each streaming more rows)
  // that still leaves >= 2048 workgroups, 8 per CU; else 256 keys.  At
  // B=64 H=32 Lkv=8192 (2048 heads) one split per head streams K/V at
  // 1.208 ms, against 1.232 / 1.244 / 1.259 / 1.301 ms for 4096 / 2048 /
  // 1024 / 512-key splits.
  auto splits = [&](int64_t c) { return BH * ((Lkv + c - 1) / c); };
  int chunk = 256;
  for (int c = DEC_MAX_CHUNK; c >= 512; c >>= 1)
    if (splits(c) >= 2048) {
      chunk = c;
      break;
    }
  if (Lkv < chunk) chunk = (int)((Lkv + 63) / 64 * 64);
  const int64_t nsplit = (Lkv + chunk - 1) / chunk;
  if (!grid_fits(BH * nsplit, DEC_THREADS)) return fail(TT_ERR_ARG, "attention decode: grid too large");
  const float sl2 = scale * kLog2e;
  const dim3 grid((unsigned)(nsplit * BH)), block(DEC_THREADS);
  if (nsplit == 1) {  // one split per head: no partials, no combine
    if (chunk <= DEC_SMALL_CHUNK)
      hipLaunchKernelGGL((attn_decode_split_kernel<T, D, 8, DEC_SMALL_CHUNK, true>), grid, block, 0, st, q, k, v,
                         nullptr, nullptr, o, lse, (int)Lkv, 1, chunk, sl2);
    else
      hipLaunchKernelGGL((attn_decode_split_kernel<T, D, 8, DEC_MAX_CHUNK, true>), grid, block, 0, st, q, k, v,
                         nullptr, nullptr, o, lse, (int)Lkv, 1, chunk, sl2);
    TT_LAUNCHED("attention decode launch", st);
    return ok();
  }
  void* ws = nullptr;
  const size_t need = (size_t)(BH * nsplit) * (D + 1) * sizeof(float);
  WorkspaceLease lease;  // held until both kernels are launched
  int rc = lease.get(st, kWsDecodePartials, need, &ws);
  if (rc) return rc;
  float* part_o = (float*)ws;
  float* part_lse = part_o + BH * nsplit * D;
  if (chunk <= DEC_SMALL_CHUNK)
    hipLaunchKernelGGL((attn_decode_split_kernel<T, D, 8, DEC_SMALL_CHUNK, false>), grid, block, 0, st, q, k, v,
                       part_o, part_lse, nullptr, nullptr, (int)Lkv, (int)nsplit, chunk, sl2);
  else
    hipLaunchKernelGGL((attn_decode_split_kernel<T, D, 8, DEC_MAX_CHUNK, false>), grid, block, 0, st, q, k, v,
                       part_o, part_lse, nullptr, nullptr, (int)Lkv, (int)nsplit, chunk, sl2);
  TT_LAUNCHED("attention decode split launch", st);
  hipLaunchKernelGGL((attn_decode_combine_kernel<T, D>), dim3((unsigned)BH), dim3(D), 0, st, part_o,
                     part_lse, o, lse, (int)nsplit);
  TT_LAUNCHED("attention decode combine launch", st);
  return ok();
}

template <typename T>
static int decode_entry(const char* fn, const T* q, const T* k, const T* v, T* o, float* lse, int64_t B,
                        int64_t H, int64_t Lkv, int64_t d, float scale, void* stream) {
  int rc = check_attn_shape(fn, B, H, 1, Lkv, d, 0);
  if (rc) return rc;
  const int64_t BH = B * H;
  if (BH == 0) return ok();
  if (!q || !k || !v || !o) return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
  const size_t qb = (size_t)(BH * d) * sizeof(T), kb = (size_t)(BH * Lkv * d) * sizeof(T);
  if ((rc = check_no_overlap(fn, {{q, qb, "q"}, {k, kb, "k"}, {v, kb, "v"}},
                             {{o, qb, "o"}, {lse, (size_t)BH * sizeof(float), "lse"}})))
    return rc;
  if ((rc = ensure_init())) return rc;
  hipStream_t st = stream_or_default(stream);
  switch (d) {
    case 32: return launch_decode<T, 32>(q, k, v, o, lse, BH, Lkv, scale, st);
    case 64: return launch_decode<T, 64>(q, k, v, o, lse, BH, Lkv, scale, st);
    case 128: return launch_decode<T, 128>(q, k, v, o, lse, BH, Lkv, scale, st);
    default: return fail(TT_ERR_UNSUPPORTED, std::string(fn) + ": unsupported head dim");
  }
}

}  // namespace tt

using namespace tt;

extern "C" int tt_attn_decode_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                                   float* lse, int64_t B, int64_t H, int64_t Lkv, int64_t d, float scale,
                                   void* stream) {
  return decode_entry<u16>("tt_attn_decode_bf16", q, k, v, o, lse, B, H, Lkv, d, scale, stream);
}

extern "C" int tt_attn_decode_f32(const float* q, const float* k, const float* v, float* o, float* lse,
                                  int64_t B, int64_t H, int64_t Lkv, int64_t d, float scale, void* stream) {
  return decode_entry<float>("tt_attn_decode_f32", q, k, v, o, lse, B, H, Lkv, d, scale, stream);
}
