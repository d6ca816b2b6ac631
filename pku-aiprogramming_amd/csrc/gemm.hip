// General matrix multiply on the MFMA units: the cudaGemm contract.
//
// Replaces cudaGemm (Task3/Tinytensor/src/Layers_kernels.cu:10-30), which
// creates a cuBLAS handle, calls cublasSgemm and destroys the handle on every
// call, at its call sites in FcForward / FcBackward / ConvForward /
// ConvBackward (src/Layers.cu:26-77, 197, 247-248).  Same contract, all
// matrices row-major:
//   C[m x n] = alpha op(A)[m x k] op(B)[k x n] + beta C
//   transa = 0: A stored m x k (lda = k);  transa = 1: A stored k x m (lda = m)
//   transb = 0: B stored k x n (ldb = n);  transb = 1: B stored n x k (ldb = k)
// beta = 0 does not read C.  fp32 on v_mfma_f32_32x32x2f32 (fp32 products,
// fp32 sums) and bf16 on v_mfma_f32_32x32x16_bf16 (fp32 sums, bf16 C).
//
// bf16 calls with k % 32 == 0 and aligned operands run k_gemm_dma: direct
// global -> LDS tile loads into swizzled, unpadded tiles.  Every other call
// runs k_gemm:
// Workgroup = 4 waves, a 128 x 128 (fp32) or 128 x 256 (bf16) tile of C
// (each wave 64 x 64 or 64 x 128: 2 x 2 or 2 x 4 MFMA blocks of 32 x 32);
// k in steps of BK through a two-stage LDS ring,
// global -> registers -> LDS, one barrier per step.  Each operand tile keeps
// its stored layout in LDS (rows padded against bank conflicts):
//   k contiguous in memory (A as stored with transa = 0, B with transb = 1):
//     [rows][BK], MFMA operands by row reads;
//   rows contiguous (A with transa = 1, B with transb = 0):
//     [BK][rows], bf16 operands by transpose reads (ds_read_b64_tr_b16),
//     fp32 operands by scalar reads.
// Tiles past m, n or k read zeros.  16-byte global loads when every row
// stride and base is 16-byte aligned, element loads otherwise.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "attn_common.h"
#include "tt_internal.h"

namespace tt {

namespace {

constexpr int GM = 128;  // C tile rows per workgroup

template <typename T>
struct GemmT;
template <>
struct GemmT<float> {
  static constexpr int GN = 128;          // C tile columns per workgroup
  static constexpr int BK = 16, EPC = 4;  // k per step; elements per 16-byte chunk
  static constexpr int PAD_K = 4;         // [rows][BK + PAD_K]: 80-byte rows keep 16-byte stores aligned
  static constexpr int PAD_R = 4;         // [BK][rows + PAD_R]
  static constexpr bool SWZ = false;      // k-contiguous tiles padded, not swizzled
  static __device__ __forceinline__ float to_f(float x) { return x; }
  static __device__ __forceinline__ float from_f(float x) { return x; }
};
template <>
struct GemmT<u16> {
  // 128 x 256 tiles (each wave 64 x 128) halve the operand traffic per MFMA
  // of 128 x 128 ones; BK = 32 keeps two workgroups' rings in LDS
  static constexpr int GN = 256;
  static constexpr int BK = 32, EPC = 8;
  // LDS has 64 banks of 4 bytes.  k-contiguous tiles: unpadded rows whose
  // 16-byte chunks are XOR-swizzled by row, so that both the 16 rows of a
  // 16-lane ds_read_b128 and the 4 rows x 4 chunks of a 16-lane store hit 16
  // distinct 4-bank groups.  [BK][rows] tiles: row stride = 16 banks mod 64,
  // so the 4 k-rows x 2 column halves read by 32 lanes of a transpose read
  // cover the 64 banks once.
  static constexpr int PAD_K = 0;
  static constexpr int PAD_R = 32;
  static constexpr bool SWZ = true;
  static __device__ __forceinline__ float to_f(u16 x) { return bf16_to_f32(x); }
  static __device__ __forceinline__ u16 from_f(float x) { return f32_to_bf16(x); }
};

// One operand tile (A: rows = m; B: rows = n) of R rows by BK k-values.
// KC: k is contiguous in memory (stored [row][k], leading dimension ld);
// otherwise stored [k][row].
template <typename T, int R, bool KC>
struct OpTile {
  using G = GemmT<T>;
  static constexpr int BK = G::BK, EPC = G::EPC;
  static constexpr int CH = R * BK / EPC / 256;  // 16-byte chunks per thread per step
  static_assert(R * BK % (EPC * 256) == 0, "tile must split into whole chunks");
  // LDS: KC ? [R][BK + PAD_K] : [BK][R + PAD_R]
  static constexpr int LD = KC ? BK + G::PAD_K : R + G::PAD_R;
  static constexpr int ELEMS = KC ? R * LD : BK * LD;
  static constexpr bool SWZ = KC && G::SWZ;
  static constexpr int NCH = BK / EPC;                    // 16-byte chunks per k-contiguous row
  static constexpr int RPB = NCH >= 16 ? 1 : 16 / NCH;    // rows per 64 banks

  // Element offset of chunk c (EPC elements) of tile row r.
  __device__ static __forceinline__ int chunk_off(int r, int c) {
    if constexpr (SWZ) return r * LD + ((c ^ ((r / RPB) % NCH)) * EPC);
    return r * LD + c * EPC;
  }

  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  u32x4 reg[CH];

  // chunk c of this thread: the row (of the stored matrix) and the first
  // element along the contiguous axis, relative to the tile origin
  __device__ static __forceinline__ void chunk_pos(int c, int& srow, int& scol) {
    const int id = (int)threadIdx.x + 256 * c;
    constexpr int PER_ROW = (KC ? BK : R) / EPC;  // chunks per stored row
    srow = id / PER_ROW;
    scol = (id % PER_ROW) * EPC;
  }

  // Global -> registers.  The tile covers rows [r0, r0 + R) and k [k0, k0 + BK)
  // of op(X); rows >= nrows or k >= K read 0.
  template <bool VEC>
  __device__ __forceinline__ void load(const T* X, int64_t ld, int r0, int k0, int nrows, int K) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int srow, scol;
      chunk_pos(c, srow, scol);
      // stored coordinates: KC -> (row, k); else (k, row)
      const int grow = KC ? r0 + srow : k0 + srow;
      const int gcol = KC ? k0 + scol : r0 + scol;
      const int rlim = KC ? nrows : K, clim = KC ? K : nrows;
      const T* p = X + (int64_t)grow * ld + gcol;
      if (VEC && grow < rlim && gcol + EPC <= clim) {
        reg[c] = *reinterpret_cast<const u32x4*>(p);
      } else {
        T v[EPC];
#pragma unroll
        for (int e = 0; e < EPC; ++e) v[e] = (grow < rlim && gcol + e < clim) ? p[e] : T(0);
        reg[c] = __builtin_bit_cast(u32x4, v);
      }
    }
  }
  // registers -> LDS tile at s
  __device__ __forceinline__ void store(T* s) const {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      int srow, scol;
      chunk_pos(c, srow, scol);
      const int off = KC ? chunk_off(srow, scol / EPC) : srow * LD + scol;
      *reinterpret_cast<u32x4*>(&s[off]) = reg[c];
    }
  }
};

// MFMA operand of 32 rows (rbase..rbase+31 of the tile) at k-step ks.
// bf16: lane l gets 8 k-values (8(l/32) + e) of row l % 32.
// fp32: lane l gets k-value l / 32 of row l % 32.
template <typename T, int R, bool KC>
__device__ __forceinline__ auto operand(const T* s, int rbase, int ks) {
  using Tile = OpTile<T, R, KC>;
  const int l = threadIdx.x & 63;
  if constexpr (sizeof(T) == 2) {
    const int k0 = 16 * ks;
    if constexpr (KC) {
      return *reinterpret_cast<const bf16x8*>(&s[Tile::chunk_off(rbase + (l & 31), k0 / 8 + (l >> 5))]);
    } else {
      // transpose reads: 16-lane group G = l / 16 takes rows (k) k0 + 8(G/2) + 0..3
      // (then + 4..7) of columns rbase + 16(G%2) + 0..15; lane s of the group
      // points at k-row + s/4, column + 4(s%4)
      const int G = l >> 4, sl = l & 15;
      const int kr = k0 + 8 * (G >> 1) + (sl >> 2);
      const int col = rbase + 16 * (G & 1) + 4 * (sl & 3);
      return lds_read_tr16x2(&s[kr * Tile::LD + col], &s[(kr + 4) * Tile::LD + col]);
    }
  } else {
    const int k = 2 * ks + (l >> 5), r = rbase + (l & 31);
    return KC ? s[r * Tile::LD + k] : s[k * Tile::LD + r];
  }
}

template <typename T, bool TA, bool TB, bool VEC>
__global__ __launch_bounds__(256, 2) void k_gemm(int M, int N, int K, float alpha, const T* __restrict__ A,
                                                int64_t lda, const T* __restrict__ B, int64_t ldb, float beta,
                                                T* C) {
  using G = GemmT<T>;
  constexpr int GN = G::GN, NB = GN / 64;  // MFMA blocks per wave along n
  constexpr int BK = G::BK, KS = sizeof(T) == 2 ? BK / 16 : BK / 2;  // MFMA k-steps per BK
  using TileA = OpTile<T, GM, !TA>;  // A as stored with transa = 0 is [m][k]: k contiguous
  using TileB = OpTile<T, GN, TB>;   // B as stored with transb = 1 is [n][k]: k contiguous
  __shared__ __align__(16) T sA[2][TileA::ELEMS];
  __shared__ __align__(16) T sB[2][TileB::ELEMS];

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
  const int wm = 64 * (w >> 1), wn = (GN / 2) * (w & 1);  // this wave's 64 x GN/2 of the tile

  f32x16 acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x16{};

  TileA ta;
  TileB tb;
  const int nk = (K + BK - 1) / BK;
  if (nk > 0) {
    ta.template load<VEC>(A, lda, m0, 0, M, K);
    tb.template load<VEC>(B, ldb, n0, 0, N, K);
    ta.store(sA[0]);
    tb.store(sB[0]);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {  // next step's tiles in flight during this step's MFMAs
      ta.template load<VEC>(A, lda, m0, BK * (kt + 1), M, K);
      tb.template load<VEC>(B, ldb, n0, BK * (kt + 1), N, K);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const auto a0 = operand<T, GM, !TA>(sA[cur], wm, ks);
      const auto a1 = operand<T, GM, !TA>(sA[cur], wm + 32, ks);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const auto b = operand<T, GN, TB>(sB[cur], wn + 32 * j, ks);
        if constexpr (sizeof(T) == 2) {
          acc[0][j] = mfma_bf16_32x32x16(a0, b, acc[0][j]);
          acc[1][j] = mfma_bf16_32x32x16(a1, b, acc[1][j]);
        } else {
          acc[0][j] = mfma_f32_32x32x2(a0, b, acc[0][j]);
          acc[1][j] = mfma_f32_32x32x2(a1, b, acc[1][j]);
        }
      }
    }
    if (kt + 1 < nk) {
      ta.store(sA[cur ^ 1]);
      tb.store(sB[cur ^ 1]);
    }
    __syncthreads();
  }

  // accumulator register r of block (i, j): C row m0 + wm + 32i + acc_row(r, l / 32),
  // column n0 + wn + 32j + l % 32
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = n0 + wn + 32 * j + (l & 31);
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + 32 * i + acc_row(r, l >> 5);
        if (m >= M) continue;
        T* p = C + (int64_t)m * N + n;
        float v = alpha * acc[i][j][r];
        if (beta != 0.f) v += beta * G::to_f(*p);
        *p = G::from_f(v);
      }
    }
}

// The direct-to-LDS kernel below serves full bf16 tiles.  A 2-deep ring (48
// KB of LDS, 155-167 VGPRs: three workgroups per CU) measured 1075-1093 TF at
// 8192^3 against 985-1018 for 3 stages and 845-892 for 4 (one or two
// workgroups per CU); 256 C columns per workgroup (128: 91 VGPRs but 15-20 %
// slower).
constexpr int kDmaStages = 2;
constexpr int kDmaGN = 256;

// bf16 kernel for k % 32 == 0 with 16-byte aligned operands (ragged m and n
// allowed): tiles go straight from global memory into LDS
// (global_load_lds_dwordx4, no register staging) through an S-deep ring, in
// unpadded XOR-swizzled layouts that the 64 contiguous 16-byte slots of a
// wave's load instruction can fill:
//   k contiguous ([rows][32], 64-byte rows): chunk c of row r at c ^ ((r >> 2) & 3);
//   rows contiguous ([32][rows], 256- or 512-byte k-rows): chunk c of k-row r at
//   c ^ ((r & 3) << 2).
// Both keep the MFMA operand reads (16-byte row reads, transpose reads) free
// of bank conflicts.
template <int R, bool KC>
struct DmaTile {
  static constexpr int BK = 32;
  static constexpr int NCH = KC ? BK / 8 : R / 8;  // 16-byte chunks per stored row
  static constexpr int ELEMS = R * BK;
  static constexpr int LOADS = ELEMS / 8 / 256;    // load instructions per wave per tile
  __device__ static __forceinline__ int pos(int row, int c) {
    return KC ? (c ^ ((row >> 2) & 3)) : (c ^ ((row & 3) << 2));
  }
  // element offset of chunk c of stored row `row`
  __device__ static __forceinline__ int off(int row, int c) { return row * NCH * 8 + pos(row, c) * 8; }
  // Load the tile whose first stored element is `src` (leading dimension ld)
  // into `dst`: slot p of the workgroup's instruction i holds stored row
  // p / NCH, chunk position p % NCH.  `nr` tile rows (m or n) exist; slots of
  // rows past them load the last one instead (a multiple of 8 when rows are
  // the contiguous axis), so every address stays inside the matrix: those
  // rows only feed C entries that are never stored.
  __device__ static __forceinline__ void load(const u16* src, int64_t ld, int nr, u16* dst) {
    const int w = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int p = (i * 4 + w) * 64 + l, ps = p % NCH;
      int row = p / NCH;
      int c = KC ? (ps ^ ((row >> 2) & 3)) : (ps ^ ((row & 3) << 2));  // the swizzle is an involution
      if (KC) row = min(row, nr - 1);
      else c = min(c, nr / 8 - 1);
      glds16(src, (uint32_t)(2 * ((int64_t)row * ld + 8 * c)), lds_addr(dst) + 1024u * (uint32_t)(i * 4 + w));
    }
  }
};

template <int R, bool KC>
__device__ __forceinline__ bf16x8 dma_operand(const u16* s, int rbase, int ks) {
  using Tile = DmaTile<R, KC>;
  const int l = threadIdx.x & 63;
  if constexpr (KC) {
    return *reinterpret_cast<const bf16x8*>(&s[Tile::off(rbase + (l & 31), 2 * ks + (l >> 5))]);
  } else {
    const int G = l >> 4, sl = l & 15;
    const int kr = 16 * ks + 8 * (G >> 1) + (sl >> 2);
    const int col = rbase + 16 * (G & 1) + 4 * (sl & 3);
    return lds_read_tr16x2(&s[Tile::off(kr, col >> 3) + (col & 4)], &s[Tile::off(kr + 4, col >> 3) + (col & 4)]);
  }
}

template <bool TA, bool TB>
__global__ __launch_bounds__(256, 3) void k_gemm_dma(int M, int N, int K, float alpha, const u16* __restrict__ A,
                                                    int64_t lda, const u16* __restrict__ B, int64_t ldb,
                                                    float beta, u16* C) {
  using G = GemmT<u16>;
  constexpr int GN = kDmaGN, NB = GN / 64, BK = 32, KS = BK / 16, S = kDmaStages;
  using TileA = DmaTile<GM, !TA>;
  using TileB = DmaTile<GN, TB>;
  constexpr int PER = TileA::LOADS + TileB::LOADS;
  static_assert(PER * (S - 2) < 64, "vmcnt range");
  __shared__ __align__(16) u16 sA[S][TileA::ELEMS];
  __shared__ __align__(16) u16 sB[S][TileB::ELEMS];

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
  const int wm = 64 * (w >> 1), wn = (GN / 2) * (w & 1);
  f32x16 acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = f32x16{};

  const int nk = K / BK;
  // stored origin of k-step t: A as stored is [m][k] (TA = 0) or [k][m]
  auto issue = [&](int t) {
    const int k0 = BK * t, b = t % S;
    TileA::load(TA ? A + (int64_t)k0 * lda + m0 : A + (int64_t)m0 * lda + k0, lda, M - m0, sA[b]);
    TileB::load(TB ? B + (int64_t)n0 * ldb + k0 : B + (int64_t)k0 * ldb + n0, ldb, N - n0, sB[b]);
  };
#pragma unroll
  for (int t = 0; t < S - 1; ++t)
    if (t < nk) issue(t);
  for (int t = 0; t < nk; ++t) {
    wait_vmem_tiles<PER, (S - 2 < 3 ? S - 2 : 3)>(min(S - 2, nk - 1 - t));  // tile t has landed
    __syncthreads();
    if (t + S - 1 < nk) issue(t + S - 1);  // into the buffer every wave finished at step t - 1
    const u16* a = sA[t % S];
    const u16* bb = sB[t % S];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const bf16x8 a0 = dma_operand<GM, !TA>(a, wm, ks);
      const bf16x8 a1 = dma_operand<GM, !TA>(a, wm + 32, ks);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const bf16x8 b = dma_operand<GN, TB>(bb, wn + 32 * j, ks);
        acc[0][j] = mfma_bf16_32x32x16(a0, b, acc[0][j]);
        acc[1][j] = mfma_bf16_32x32x16(a1, b, acc[1][j]);
      }
    }
  }
  wait_vmem_le<0>();  // nothing may be in flight into LDS when the workgroup exits

#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int n = n0 + wn + 32 * j + (l & 31);
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + wm + 32 * i + acc_row(r, l >> 5);
        if (m >= M) continue;
        u16* p = C + (int64_t)m * N + n;
        float v = alpha * acc[i][j][r];
        if (beta != 0.f) v += beta * G::to_f(*p);
        *p = G::from_f(v);
      }
    }
}

template <typename T>
int gemm_launch(const char* fn, int transa, int transb, int64_t m, int64_t n, int64_t k, float alpha, const T* A,
                const T* B, float beta, T* C, void* stream) {
  if (m < 0 || n < 0 || k < 0) return fail(TT_ERR_ARG, std::string(fn) + ": negative size");
  if (transa != 0 && transa != 1) return fail(TT_ERR_ARG, std::string(fn) + ": transa must be 0 or 1");
  if (transb != 0 && transb != 1) return fail(TT_ERR_ARG, std::string(fn) + ": transb must be 0 or 1");
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
    return fail(TT_ERR_ARG, std::string(fn) + ": dimension above 2^31 - 1");
  if (m == 0 || n == 0) return ok();
  if (!C || (k > 0 && (!A || !B))) return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
  constexpr int GN = GemmT<T>::GN;
  const int64_t gx = (n + GN - 1) / GN, gy = (m + GM - 1) / GM;
  if (gy > 65535) return fail(TT_ERR_ARG, std::string(fn) + ": m too large");
  if (!grid_fits(gx, 256)) return fail(TT_ERR_ARG, std::string(fn) + ": n too large");
  int rc = ensure_init();
  if (rc) return rc;
  hipStream_t s = stream_or_default(stream);
  const int64_t lda = transa ? m : k, ldb = transb ? k : n;
  constexpr int EPC = GemmT<T>::EPC;
  const bool vec = lda % EPC == 0 && ldb % EPC == 0 && (uintptr_t)A % 16 == 0 && (uintptr_t)B % 16 == 0;
  const dim3 grid((unsigned)gx, (unsigned)gy), block(256);
  if constexpr (sizeof(T) == 2) {
    // k in whole steps, aligned rows (m, n multiples of 8 where they are the
    // contiguous axis: vec), and every per-lane tile offset within 32 bits
    if (vec && k % 32 == 0 && lda < (int64_t(1) << 22) && ldb < (int64_t(1) << 22)) {
      const dim3 g2((unsigned)((n + kDmaGN - 1) / kDmaGN), (unsigned)gy);
#define TT_GEMM_D(TA, TB) \
  hipLaunchKernelGGL((k_gemm_dma<TA, TB>), g2, dim3(256), 0, s, (int)m, (int)n, (int)k, alpha, A, lda, B, ldb, beta, C)
      switch (transa * 2 + transb) {
        case 0: TT_GEMM_D(false, false); break;
        case 1: TT_GEMM_D(false, true); break;
        case 2: TT_GEMM_D(true, false); break;
        default: TT_GEMM_D(true, true); break;
      }
#undef TT_GEMM_D
      TT_LAUNCHED(fn, s);
      return ok();
    }
  }
#define TT_GEMM(TA, TB, V)                                                                                   \
  hipLaunchKernelGGL((k_gemm<T, TA, TB, V>), grid, block, 0, s, (int)m, (int)n, (int)k, alpha, A, lda, B, ldb, \
                     beta, C)
  switch (transa * 4 + transb * 2 + (vec ? 1 : 0)) {
    case 0: TT_GEMM(false, false, false); break;
    case 1: TT_GEMM(false, false, true); break;
    case 2: TT_GEMM(false, true, false); break;
    case 3: TT_GEMM(false, true, true); break;
    case 4: TT_GEMM(true, false, false); break;
    case 5: TT_GEMM(true, false, true); break;
    case 6: TT_GEMM(true, true, false); break;
    default: TT_GEMM(true, true, true); break;
  }
#undef TT_GEMM
  TT_LAUNCHED(fn, s);
  return ok();
}

}  // namespace

}  // namespace tt

using namespace tt;

extern "C" int tt_gemm_f32(int transa, int transb, int64_t m, int64_t n, int64_t k, float alpha, const float* A,
                           const float* B, float beta, float* C, void* stream) {
  return gemm_launch<float>("tt_gemm_f32", transa, transb, m, n, k, alpha, A, B, beta, C, stream);
}

extern "C" int tt_gemm_bf16(int transa, int transb, int64_t m, int64_t n, int64_t k, float alpha, const uint16_t* A,
                            const uint16_t* B, float beta, uint16_t* C, void* stream) {
  return gemm_launch<u16>("tt_gemm_bf16", transa, transb, m, n, k, alpha, A, B, beta, C, stream);
}
