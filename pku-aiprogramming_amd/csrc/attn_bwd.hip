// Fused attention backward for gfx950.
//
// Replaces O.backward(dO) over the reference's composition
// (optimizer/operators.py:115-119 -> autodiff.py:33-61) through the gradient
// rules MatMul (:421-429), Transpose (:338-340), MulScalar (:241-242),
// EWiseDiv (:296-298), BroadcastTo (:373-380), Summation (:400-408) and
// Exp (:469-470).  Closed form of that chain, with P recomputed from the LSE
// saved by the forward so no L x L tensor is ever stored:
//   D_i  = sum_d dO_id O_id                  (row pre-pass, fp32 [B,H,L])
//   P    = exp(s Q K^T + M - LSE)
//   dV   = P^T dO,   dP = dO V^T,   dS = P o (dP - D)
//   dQ   = s dS K,   dK = s dS^T Q
//
// Two kernels split the work so that every output row has one owner and no
// atomics are needed:
//   dkdv: workgroup = NW waves x 32 keys (lane = key; K rows in registers, V
//         rows in LDS); loops over query tiles that stream through a
//         STAGES-deep ring of LDS buffers.  The same tile feeds the S / dP
//         operands (16-byte row reads) and the transposed
//         dV^T += dO^T P, dK^T += Q^T dS operands (gfx950 transpose reads).
//   dq:   workgroup = NW waves x 32 queries (lane = query, as the forward);
//         loops over key tiles: S^T and dP^T from K / V row reads,
//         dQ^T += K^T dS^T from transpose reads of the same K tile.
// bf16: the dq kernel (attn_bwd_dq_pipe_kernel) runs first and also writes
// the rows -D and LSE log2(e) the dkdv kernel reads; at d = 128 the dK / dV
// role runs one wave per SIMD with 64 keys per wave (attn_bwd_w64.hip), at
// d = 32 and 64, and for short causal heads at d = 128, the kernel below.  fp32 (attn_bwd_f32.h): a separate row
// pre-pass (attn_bwd_delta_kernel), then one launch holding both roles.
// All bf16 tiles are filled by direct global->LDS loads.  Loads past the end
// of a sequence read a clamped (valid) row and the result is masked, so the
// inner loops carry no load guards.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "attn_bwd_f32.h"
#include "attn_common.h"
#include "attn_tiles.h"

namespace tt {

// Waves per workgroup, pipeline depth, and tile sizes of the bf16 kernels:
// 4-wave workgroups with 2 stages, so two workgroups with independent
// barriers share each CU (2 waves per SIMD); measured faster on the MI355X
// than one 8-wave workgroup with a 4-deep ring.
constexpr int bwd_nw(int) { return 4; }
constexpr int kBwdStages = 2;
// Query rows per LDS tile of the two-waves-per-SIMD dK/dV kernel: 64, or 32
// at d = 128, where two workgroups then fit the LDS of a CU (66.5 KB each).
template <int D>
constexpr int dkdv_bq() { return D >= 128 ? 32 : 64; }
// The d = 128 dK/dV role: the one-wave-per-SIMD persistent kernel
// (attn_bwd_w64.hip), except for causal heads of at most this many keys,
// where each of its 256-key items is short and its prologue and epilogue
// stand alone on the CU; the kernel below with two workgroups per CU then
// overlaps them (dK/dV at L = 512 / 1024 / 2048: -30 / -17 / -8 %; at 4096,
// and for non-causal heads, the one-wave kernel is 3-10 % faster).
constexpr int64_t kDkdvTwoWaveMaxLk128 = 2048;

// ND_i = -D_i = -sum_d dO[i][d] * O[i][d], one 16-byte chunk per thread
// (stored negated: the dK/dV kernel starts its dP accumulator at -D, so the
// MFMA yields dP - D directly); also L2_i = LSE_i * log2(e), the log-sum-exp
// in the log2 domain the MFMA kernels exponentiate in.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const T* __restrict__ O,
                                                             const T* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             float* __restrict__ NDelta, float* __restrict__ L2,
                                                             int64_t rows) {
  constexpr int EPT = 16 / sizeof(T);
  constexpr int TPR = D / EPT;  // threads per row (a power of two <= 32)
  constexpr int RPB = 256 / TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int col = threadIdx.x % TPR;
  float sum = 0.f;
  if (row < rows) {
    uint4 a = ldg16(O + row * D + col * EPT);
    uint4 b = ldg16(dO + row * D + col * EPT);
    if constexpr (sizeof(T) == 2) {
      const u16* pa = reinterpret_cast<const u16*>(&a);
      const u16* pb = reinterpret_cast<const u16*>(&b);
#pragma unroll
      for (int e = 0; e < 8; ++e) sum += bf16_to_f32(pa[e]) * bf16_to_f32(pb[e]);
    } else {
      const float* pa = reinterpret_cast<const float*>(&a);
      const float* pb = reinterpret_cast<const float*>(&b);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum += pa[e] * pb[e];
    }
  }
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if (col == 0 && row < rows) {
    NDelta[row] = -sum;
    L2[row] = LSE[row] * kLog2e;
  }
}

// ------------------------------------------------------------------ bf16 dK, dV
// At d = 64 the compiler fits this kernel in 166-168 VGPRs, which lets three
// workgroups share a CU (8 % faster than two); a change that needs more
// registers silently drops it to two.  At d = 128 (short causal heads only,
// kDkdvTwoWaveMaxLk128) it takes 251-252 VGPRs and 32-query tiles: two
// workgroups per CU.  Stating the three-workgroup bound
// instead produced other code and was 0-1 % slower; a variant with a second,
// branch-free copy of the loop needed 248 VGPRs (152 spilled under the bound).
template <int D, bool CAUSAL>
__global__ __launch_bounds__(64 * bwd_nw(D), 8 / bwd_nw(D)) void attn_bwd_dkdv_bf16_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ dO, const float* __restrict__ L2, const float* __restrict__ NDelta,
    u16* __restrict__ dK, u16* __restrict__ dV, int Lq, int Lk, int BH, int nkt, int order, float sl2,
    float scale) {
  using Tile = SwzTile<D>;
  constexpr int NW = bwd_nw(D), BN = 32 * NW, BQ = dkdv_bq<D>(), MT = BQ / 32, S = kBwdStages;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int TE = Tile::kElems(BQ);
  constexpr int VS = 64;  // stride of the LSE / D row buffers (one 64-lane load each)
  using Dma = TileDma<D, BQ, NW>;
  constexpr int IPT = 2 * Dma::kLoads;  // Q + dO loads per wave per tile
  // One LDS block, carved at fixed byte offsets so that every operand read
  // is a per-lane address plus an immediate: the ring of Q / dO tiles with
  // their LSE (log2) / D rows and the workgroup's V rows, all filled by direct
  // global->LDS loads.  50 KB at d = 64 lets three workgroups share a CU.
  constexpr int kOQ = 0, kOdO = kOQ + 2 * S * TE, kOV = kOdO + 2 * S * TE, kOL = kOV + 2 * Tile::kElems(BN),
                kOD = kOL + 4 * S * VS, kLds = kOD + 4 * S * VS;
  static_assert(kOV <= 65536, "Q / dO ring offsets exceed the 16-bit LDS immediate");
  __shared__ __align__(16) char smem[kLds];
  u16* const sQ = reinterpret_cast<u16*>(smem + kOQ);
  u16* const sdO = reinterpret_cast<u16*>(smem + kOdO);
  u16* const sV = reinterpret_cast<u16*>(smem + kOV);
  float* const sL = reinterpret_cast<float*>(smem + kOL);
  float* const sDl = reinterpret_cast<float*>(smem + kOD);
  const uint32_t a0 = lds_addr(smem);

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 5, r32 = l & 31;
  const int wu = __builtin_amdgcn_readfirstlane(w);  // w, known wave-uniform (scalar branches)
  int kt, bh;
  map_tile(blockIdx.x, nkt, BH, order, kt, bh, false);  // causal: key tile 0 sees every query
  const int k0 = kt * BN;
  const int key = k0 + 32 * w + r32;
  const int wk_lo = k0 + 32 * w;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;
  const int64_t lbase = (int64_t)bh * Lq;

  bf16x8 kf[NC];
  {
    const int kr = min(key, Lk - 1);  // rows past Lk compute garbage that is never stored
#pragma unroll
    for (int c = 0; c < NC; ++c)
      kf[c] = __builtin_bit_cast(bf16x8, ldg16(K + kbase + (int64_t)kr * D + 16 * c + 8 * g));
  }
  f32x16 adk[ND], adv[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) adk[dt] = adv[dt] = f32x16{};

  // transpose-read addressing (this lane as a source row/column)
  const int t16 = l & 15;
  const int trow = 4 * g + (t16 >> 2);
  const int tcol = 16 * ((l >> 4) & 1) + 4 * (t16 & 3);

  // Tile ring over query tiles [qstart, Lq): tile n lives in buffer n % S.
  // Query rows past Lq read row Lq - 1 and are masked (P = 0) in the edge step.
  const int qstart = CAUSAL ? k0 : 0;  // k0 is a multiple of BQ
  const int ntiles = Lq > qstart ? (Lq - qstart + BQ - 1) / BQ : 0;
  Dma dma;
  dma.init();
  int issued = 0;
  auto issue_next = [&]() {
    if (issued < ntiles) {
      const int b = (unsigned)issued % S, qb = qstart + issued * BQ;
      dma.issue(Q + qbase, qb, Lq, sQ + b * TE);
      dma.issue(dO + qbase, qb, Lq, sdO + b * TE);
      if (wu == 0) {
        load_vec_lds(L2 + lbase + qb, Lq - qb, sL + b * VS);
        load_vec_lds(NDelta + lbase + qb, Lq - qb, sDl + b * VS);
      }
      ++issued;
    }
  };

  // This lane's LDS byte addresses in Q buffer 0 (dO, other buffers and query
  // halves are immediates away), all loop invariant: 16-byte row reads
  // (chunk 2c + g of row r32; half mt adds 32 rows), the wave's V rows,
  // transpose reads at rows trow / trow + 8 of column 32 dt + tcol (half h
  // adds 16 rows), and the LSE / D rows.  The swizzle depends on the low four
  // row bits only, so those row offsets are plain immediates.
  uint32_t roff[NC], voff[NC], troff[2][ND];
  uint32_t lofs = a0 + kOL + 16 * g;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    roff[c] = a0 + kOQ + 2 * Tile::chunk(r32, 2 * c + g);
    voff[c] = a0 + kOV + 2 * Tile::chunk(32 * w + r32, 2 * c + g);
  }
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) {
    troff[0][dt] = a0 + kOQ + 2 * Tile::at4(trow, 32 * dt + tcol);
    troff[1][dt] = a0 + kOQ + 2 * Tile::at4(trow + 8, 32 * dt + tcol);
  }

  // Tile in ring buffer b: bq = b * (Q tile bytes), bl = b * (LSE row bytes).
  auto step = [&](int qb, int bq, int bl, auto mask_tag) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      // dP starts at -D of each query row (register r holds row acc_row(r, g)),
      // so the accumulator ends as dP - D
      f32x16 s = f32x16{}, dp;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 nd = lds_ld<f32x4>(lofs + (kOD - kOL) + bl + 128 * mt + 32 * j);
        dp[4 * j] = nd.x;
        dp[4 * j + 1] = nd.y;
        dp[4 * j + 2] = nd.z;
        dp[4 * j + 3] = nd.w;
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint32_t off = roff[c] + bq + 64 * mt * D;
        s = mfma_bf16_32x32x16(lds_ld<bf16x8>(off), kf[c], s);
        const bf16x8 vb = lds_ld<bf16x8>(voff[c]);
        dp = mfma_bf16_32x32x16(lds_ld<bf16x8>(off + (kOdO - kOQ)), vb, dp);
      }
      // transposed dO / Q operands of dV^T / dK^T MFMA i = h * ND + dt,
      // fetched one MFMA pair ahead
      auto tr_op = [&](int tile_off, int i) {
        const uint32_t o = tile_off + bq + 2 * (32 * mt + 16 * (i / ND)) * D;
        return lds_tr16x2_at(troff[0][i % ND] + o, troff[1][i % ND] + o);
      };
      // s[r] = S[query qb + 32mt + acc_row(r, g)][key]
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int qi = 32 * mt + 8 * j + 4 * g;  // rows acc_row(4j..4j+3, g)
        const f32x4 lv = lds_ld<f32x4>(lofs + bl + 128 * mt + 32 * j);
        const float la[4] = {lv.x, lv.y, lv.z, lv.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * j + u;
          float p = fast_exp2(fmaf(s[r], sl2, -la[u]));
          if constexpr (MASK) {
            const int q = qb + qi + u;
            if (q >= Lq || (CAUSAL && key > q)) p = 0.f;
          }
          pb[r >> 3][r & 7] = (__bf16)p;
          db[r >> 3][r & 7] = (__bf16)(p * dp[r]);
        }
      }
      // dV^T += dO^T P and dK^T += Q^T dS over the 32 queries of this half:
      // element e of k-chunk h is accumulator row acc_row(8h + e, g), query
      // 32mt + 16h + 8(e / 4) + 4g + e % 4, the order in which the transpose
      // reads of rows trow and trow + 8 deliver the dO / Q columns.
      bf16x8 ov[2], oq[2];
      ov[0] = tr_op(kOdO - kOQ, 0);
      oq[0] = tr_op(0, 0);
#pragma unroll
      for (int i = 0; i < 2 * ND; ++i) {
        if (i + 1 < 2 * ND) {
          ov[(i + 1) & 1] = tr_op(kOdO - kOQ, i + 1);
          oq[(i + 1) & 1] = tr_op(0, i + 1);
        }
        adv[i % ND] = mfma_bf16_32x32x16(ov[i & 1], pb[i / ND], adv[i % ND]);
        adk[i % ND] = mfma_bf16_32x32x16(oq[i & 1], db[i / ND], adk[i % ND]);
      }
    }
  };

  // One barrier per tile (see the forward kernel).  Masked (diagonal /
  // ragged) and unmasked query tiles run in separate loops so that neither
  // loop switches the accumulators' registers.
  int j = 0;
  // tile j at qb in ring buffer b (b < 0: j % S at run time)
  auto tile_at = [&](int qb, auto b_tag, auto mask_tag) __attribute__((always_inline)) {
    if constexpr (S == 2) {
      wait_vmem_le<0>();  // this tile's loads, issued after the previous tile's barrier
    } else if (wu == 0) {
      wait_vmem_tiles<IPT + 2, S - 1>(issued - 1 - j);
    } else {
      wait_vmem_tiles<IPT, S - 1>(issued - 1 - j);
    }
    __syncthreads();
    issue_next();
    if constexpr (CAUSAL && decltype(mask_tag)::value) {
      if (qb + BQ - 1 < wk_lo) return;  // every query of the tile precedes every key of the wave
    }
    constexpr int bc = decltype(b_tag)::value;
    const int b = bc >= 0 ? bc : (unsigned)j % S;
    // keep address + immediate addressing (no hoisted per-buffer copies)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      opaque(roff[c]);
      opaque(voff[c]);
    }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      opaque(troff[0][dt]);
      opaque(troff[1][dt]);
    }
    opaque(lofs);
    // LLVM's single-wave MFMA / LDS interleave strategy for the tile's
    // scheduling region
    __builtin_amdgcn_iglp_opt(1);
    step(qb, b * 2 * TE, b * 4 * VS, mask_tag);
  };
  using AnyBuf = std::integral_constant<int, -1>;
  auto run = [&](int lo, int hi, auto mask_tag) __attribute__((always_inline)) {
    for (int qb = lo; qb < hi; qb += BQ, ++j) tile_at(qb, AnyBuf{}, mask_tag);
  };
  // Unmasked tiles (no query precedes a key of the workgroup): with a
  // two-buffer ring the loop is unrolled by buffer, so every LDS address is
  // a loop-invariant lane offset plus an immediate.
  auto run_full = [&](int lo, int hi) __attribute__((always_inline)) {
    if constexpr (S == 2) {
      int qb = lo;
      if ((j & 1) && qb < hi) {
        tile_at(qb, std::integral_constant<int, 1>{}, std::false_type{});
        qb += BQ;
        ++j;
      }
      for (; qb + BQ < hi; qb += 2 * BQ) {
        tile_at(qb, std::integral_constant<int, 0>{}, std::false_type{});
        ++j;
        tile_at(qb + BQ, std::integral_constant<int, 1>{}, std::false_type{});
        ++j;
      }
      if (qb < hi) {
        tile_at(qb, std::integral_constant<int, 0>{}, std::false_type{});
        ++j;
      }
    } else {
      run(lo, hi, std::false_type{});
    }
  };
  // The V tile is issued first, so the first wait (which leaves at most the
  // later Q / dO tiles outstanding) also covers it.
  {
    TileDma<D, BN, NW> vdma;
    vdma.init();
    vdma.issue(V + kbase, k0, Lk, sV);
  }
  for (int s0 = 0; s0 < S - 1; ++s0) issue_next();
  // Retire the K row loads (and the first tiles with them) here: otherwise
  // the compiler, which does not see the tile loads, keeps the K loads
  // pending around the loop and waits for them on every iteration.
  wait_vmem_le<0>();
  const int qfull = (Lq / BQ) * BQ;
  const int qdiag = CAUSAL ? min(k0 + BN, Lq) : qstart;  // [qstart, qdiag): tiles crossing the diagonal
  run(qstart, qdiag, std::true_type{});
  run_full(qdiag, qfull);
  run(max(qdiag, qfull), Lq, std::true_type{});
  wait_vmem_le<0>();  // nothing may be in flight into LDS when the workgroup exits

  // dK (scaled), then dV, through LDS: rows 0 .. BN - 1 and BN .. 2 BN - 1
  static_assert(2 * BN * D * 2 <= kLds, "the LDS block holds the workgroup's dK and dV rows");
  u16* const stage = reinterpret_cast<u16*>(smem);
  __syncthreads();
  stage_rows_bf16<D, ND>(stage, 32 * w + r32, g, adk, scale);
  stage_rows_bf16<D, ND>(stage + BN * D, 32 * w + r32, g, adv, 1.f);
  __syncthreads();
  store_staged_rows<D>(stage, BN, dK + kbase, k0, Lk, 64 * NW);
  store_staged_rows<D>(stage + BN * D, BN, dV + kbase, k0, Lk, 64 * NW);
}

// ------------------------------------------------------------------ bf16 dQ, software-pipelined (D = 32, 64, 128)
// Workgroup = 4 waves x 32 queries (lane = query, as the forward); blocks of
// 32 keys (a K tile and a V tile) stream through a 4-deep LDS ring filled by
// direct global->LDS loads.  Iteration n of a wave:
//   MFMA  S^T_{n+1} = K_{n+1} Q^T,  dP^T_{n+1} = V_{n+1} dO^T        (next block)
//   VALU  dS^T_n = 2^(s S^T_n log2(e) - LSE_n log2(e)) o (dP^T_n - D) (this block)
//   MFMA  dQ^T += K_n^T dS^T_n                                         (this block)
// so the exponentials of one block run on the VALU while the matrix cores
// compute the next block's scores.  Barrier n makes tile n + 1 visible to
// every wave and retires every read of tile n - 1, whose buffer then takes
// tile n + 3 (two iterations of load lead).  The loop is unrolled by the
// ring depth, so every LDS operand address is a loop-invariant lane offset
// plus an immediate.
//
// This kernel runs first in the backward and also does the row pre-pass the
// dK/dV kernel needs: each lane forms D = sum_d dO o O of its query row from
// the dO it holds and one read of O (the other half of the row is in lane
// l ^ 32), and stores -D and LSE * log2(e) for the dK/dV kernel.
constexpr int DQP_BN = 32;     // keys per block / LDS tile
constexpr int DQP_STAGES = 4;  // LDS ring depth (the unrolled loop relies on it)

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_pipe_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ O, const u16* __restrict__ dO, const float* __restrict__ LSE,
    float* __restrict__ L2, float* __restrict__ NDelta, u16* __restrict__ dQ, int Lq, int Lk, int BH, int nqt,
    int order, float sl2, float scale) {
  using Tile = SwzTile<D>;
  constexpr int NW = 4, BM = 32 * NW, BN = DQP_BN, S = DQP_STAGES;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int TE = Tile::kElems(BN);
  using Dma = TileDma<D, BN, NW>;
  constexpr int PER = 2 * Dma::kLoads;  // K + V load instructions per wave per tile
  // ring buffer b: K tile at element 2 b TE, V tile at 2 b TE + TE
  __shared__ __align__(16) u16 smem[2 * S * TE];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, g = l >> 5, r32 = l & 31;
  int qt, bh;
  map_tile(blockIdx.x, nqt, BH, order, qt, bh, CAUSAL);
  const int q0 = qt * BM, wq0 = q0 + 32 * w, qrow = wq0 + r32;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;

  const int kend = CAUSAL ? min(Lk, q0 + BM) : Lk;  // >= 1
  const int ntiles = (kend + BN - 1) / BN;
  Dma dma;
  dma.init();
  int issued = 0;
  auto issue_tile = [&](int n) {  // tile n into ring buffer n % S (n < ntiles)
    u16* dst = smem + 2 * (n % S) * TE;
    dma.issue(K + kbase, BN * n, Lk, dst);
    dma.issue(V + kbase, BN * n, Lk, dst + TE);
  };
  // The first K / V tiles go out before the Q / dO / O row loads, so that
  // their HBM round trip overlaps the rows' (whose wait, for the D pre-pass
  // below, then also covers them: loads retire in issue order).
  for (; issued < S - 1 && issued < ntiles; ++issued) issue_tile(issued);

  bf16x8 qf[NC], dof[NC];
  float lse2, ndl;
  {
    const int qr = min(qrow, Lq - 1);  // padding rows read a valid row; never written back
    float dsum = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int64_t at = qbase + (int64_t)qr * D + 16 * c + 8 * g;
      qf[c] = __builtin_bit_cast(bf16x8, ldg16(Q + at));
      dof[c] = __builtin_bit_cast(bf16x8, ldg16(dO + at));
      const bf16x8 of = __builtin_bit_cast(bf16x8, ldg16(O + at));
#pragma unroll
      for (int e = 0; e < 8; ++e) dsum = fmaf((float)dof[c][e], (float)of[e], dsum);
    }
    dsum = sum_xor32(dsum);  // + the other half of the row (lane l ^ 32)
    const int64_t row = (int64_t)bh * Lq + qrow;
    // padding query rows: P = 2^(s - inf) = 0
    lse2 = qrow < Lq ? LSE[(int64_t)bh * Lq + qr] * kLog2e : INFINITY;
    ndl = qrow < Lq ? -dsum : 0.f;
    if (g == 0 && qrow < Lq) {
      NDelta[row] = ndl;
      L2[row] = lse2;
    }
  }
  f32x16 adq[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) adq[dt] = f32x16{};
  // At d <= 64 the dP^T accumulator starts at -D of the lane's query (16
  // registers holding ndl), so the MFMAs yield dP - D and forming dS takes
  // one VALU operation less per score; at d = 128 the kernel has no 16
  // registers to spare and adds -D itself.
  constexpr bool kDpInit = D <= 64;
  f32x16 dinit = f32x16{};
  if constexpr (kDpInit) {
#pragma unroll
    for (int r = 0; r < 16; ++r) dinit[r] = ndl;
  }

  // Last block this wave computes: its diagonal block (causal) or the last
  // one.  Every earlier block lies inside Lk and before every query of the
  // wave; the last one is always computed with the mask.
  const int last = CAUSAL ? min(wq0 / BN, ntiles - 1) : ntiles - 1;

  // Loop-invariant LDS element offsets of this lane: K / V row operands of
  // k-chunk c (16-byte chunk 2c + g of key row r32), and the transpose reads
  // of the K^T operand of d-tile dt (rows trow, trow + 8; key chunk h adds
  // 16 rows, which keeps the swizzle).
  int kidx[NC], tidx[2][ND];
#pragma unroll
  for (int c = 0; c < NC; ++c) kidx[c] = Tile::chunk(r32, 2 * c + g);
  {
    const int t16 = l & 15;
    const int trow = 4 * g + (t16 >> 2), tcol = 16 * ((l >> 4) & 1) + 4 * (t16 & 3);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) {
      tidx[0][dt] = Tile::at4(trow, 32 * dt + tcol);
      tidx[1][dt] = Tile::at4(trow + 8, 32 * dt + tcol);
    }
  }

  // S^T and dP^T of the block in ring buffer B
  auto sdp = [&](auto b_tag, f32x16& s, f32x16& dp) __attribute__((always_inline)) {
    constexpr int B = decltype(b_tag)::value;
    const u16* tK = smem + 2 * B * TE;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const bf16x8 ka = *reinterpret_cast<const bf16x8*>(&tK[kidx[c]]);
      const bf16x8 va = *reinterpret_cast<const bf16x8*>(&tK[TE + kidx[c]]);
      s = mfma_bf16_32x32x16(ka, qf[c], c == 0 ? f32x16{} : s);
      dp = mfma_bf16_32x32x16(va, dof[c], c == 0 ? dinit : dp);
    }
  };
  // dS^T of the block at keys kb in ring buffer B, then dQ^T += K^T dS^T
  auto dsq = [&](auto b_tag, const f32x16& s, const f32x16& dp, int kb, auto mask_tag)
                 __attribute__((always_inline)) {
    constexpr int B = decltype(b_tag)::value;
    constexpr bool MASK = decltype(mask_tag)::value;
    bf16x8 db[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float p = fast_exp2(fmaf(s[r], sl2, -lse2));
      if constexpr (MASK) {
        const int key = kb + acc_row(r, g);
        if (key >= Lk || (CAUSAL && key > qrow)) p = 0.f;
      }
      db[r >> 3][r & 7] = (__bf16)(p * (kDpInit ? dp[r] : dp[r] + ndl));
    }
    const u16* tK = smem + 2 * B * TE;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const bf16x8 a = lds_read_tr16x2(&tK[tidx[0][dt] + 16 * h * D], &tK[tidx[1][dt] + 16 * h * D]);
        adq[dt] = mfma_bf16_32x32x16(a, db[h], adq[dt]);
      }
  };
  // Barrier n: this wave's loads of tile n + 1 have landed (loads retire in
  // issue order), then every wave's are visible and tile n - 1 is retired;
  // tile n + S - 1 goes into its buffer.  (Spreading these loads over the
  // score MFMAs instead measured 9 % more cycles.)
  auto barrier_n = [&](int n) __attribute__((always_inline)) {
    const int ahead = issued - n - 2;
    wait_vmem_tiles<PER, S - 2>(ahead > 0 ? ahead : 0);
    __syncthreads();
    if (n + S - 1 < ntiles) {
      issue_tile(n + S - 1);
      ++issued;
    }
  };

  wait_vmem_le<0>();  // the first tiles, and the Q / dO / O / LSE loads, before the loop
  __syncthreads();

  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  using B2 = std::integral_constant<int, 2>;
  using B3 = std::integral_constant<int, 3>;
  // LLVM's interleave strategy for the scheduling region of each iteration:
  // at d = 128 its single-wave MFMA / LDS strategy (1), at d = 64 the small-GEMM
  // one (0).  Alternating builds on one box: c5 dQ 0.723 ms with (1) against 0.740
  // with the MFMA / exponential strategy (2) used before and 0.742 with (0); d = 64,
  // L = 4096 dQ 0.197 ms with (0) against 0.204 with (1) or (2).
  constexpr int kDqIglp = D >= 128 ? 1 : 0;
  f32x16 sA, pA, sB, pB;
  sdp(B0{}, sA, pA);
  // iteration n with a next block (n < last): buffer n % 4 = B
  auto it = [&](int n, auto b_tag, f32x16& sc, f32x16& pc, f32x16& sn, f32x16& pn) __attribute__((always_inline)) {
    constexpr int B = decltype(b_tag)::value;
    barrier_n(n);
    iglp<kDqIglp>();
    sdp(std::integral_constant<int, (B + 1) % 4>{}, sn, pn);
    dsq(b_tag, sc, pc, BN * n, std::false_type{});
  };
  // Steady state without branches: while every barrier of a group of four
  // issues a next tile that lies wholly inside Lk, barrier n always leaves
  // exactly one tile (n + 2) in flight and loads tile n + S - 1 unclamped.
  // (The scalar code of the general barrier -- its wait count chosen at run
  // time, the issue test and the clamp test -- put six branches into every
  // block.)
  auto it_full = [&](int n, auto b_tag, f32x16& sc, f32x16& pc, f32x16& sn, f32x16& pn)
                     __attribute__((always_inline)) {
    constexpr int B = decltype(b_tag)::value;
    wait_vmem_le<(S - 3) * PER>();
    __syncthreads();
    u16* dst = smem + 2 * ((B + S - 1) % S) * TE;  // tile n + S - 1 goes where tile n - 1 was
    dma.issue_full(K + kbase, BN * (n + S - 1), dst);
    dma.issue_full(V + kbase, BN * (n + S - 1), dst + TE);
    ++issued;
    iglp<kDqIglp>();
    sdp(std::integral_constant<int, (B + 1) % 4>{}, sn, pn);
    dsq(b_tag, sc, pc, BN * n, std::false_type{});
  };
  static_assert(S == 4, "the unrolled loops follow the ring depth");
  const int nfull = min(ntiles, Lk / BN);  // tiles that lie wholly inside Lk
  int n = 0;
  for (; n + 4 <= last && n + 3 + S <= nfull; n += 4) {
    it_full(n, B0{}, sA, pA, sB, pB);
    it_full(n + 1, B1{}, sB, pB, sA, pA);
    it_full(n + 2, B2{}, sA, pA, sB, pB);
    it_full(n + 3, B3{}, sB, pB, sA, pA);
  }
  for (; n + 4 <= last; n += 4) {
    it(n, B0{}, sA, pA, sB, pB);
    it(n + 1, B1{}, sB, pB, sA, pA);
    it(n + 2, B2{}, sA, pA, sB, pB);
    it(n + 3, B3{}, sB, pB, sA, pA);
  }
  const int rem = last - n;  // 0..3 iterations with a next block, then the last block
  if (rem >= 1) it(n, B0{}, sA, pA, sB, pB);
  if (rem >= 2) it(n + 1, B1{}, sB, pB, sA, pA);
  if (rem >= 3) it(n + 2, B2{}, sA, pA, sB, pB);
  // the last block, then the barriers and loads of the later waves' blocks
  for (int m = last; m < ntiles; ++m) {
    barrier_n(m);
    if (m == last) {
      switch (rem) {
        case 0: dsq(B0{}, sA, pA, BN * last, std::true_type{}); break;
        case 1: dsq(B1{}, sB, pB, BN * last, std::true_type{}); break;
        case 2: dsq(B2{}, sA, pA, BN * last, std::true_type{}); break;
        default: dsq(B3{}, sB, pB, BN * last, std::true_type{}); break;
      }
    }
  }
  wait_vmem_le<0>();  // nothing may be in flight into LDS when the workgroup exits

  // dQ through LDS: the ring is free once every wave has passed its wait
  static_assert(2 * S * TE >= BM * D, "the tile ring holds the workgroup's dQ rows");
  __syncthreads();
  stage_rows_bf16<D, ND>(smem, 32 * w + r32, g, adq, scale);
  __syncthreads();
  store_staged_rows<D>(smem, BM, dQ + qbase, q0, Lq, 64 * NW);
}

// ------------------------------------------------------------------ launchers
// dK / dV at d = 128 with one wave per SIMD (attn_bwd_w64.hip).
int launch_dkdv_w64(const u16* q, const u16* k, const u16* v, const u16* dout, const float* l2, const float* nd,
                    u16* dk, u16* dv, int64_t BH, int64_t Lq, int64_t Lk, float sl2, float scale, bool causal,
                    hipStream_t st);

// `delta`: device scratch of 2 * BH * Lq floats that the kernels of this call
// own until they finish: -D (negated row sums of dO o O), then LSE * log2(e).
template <typename T, int D, bool CAUSAL>
static int launch_bwd(const T* q, const T* k, const T* v, const T* o, const float* lse, const T* dout,
                      T* dq, T* dk, T* dv, int64_t BH, int64_t Lq, int64_t Lk, float scale, hipStream_t st,
                      float* delta) {
  constexpr bool BF = sizeof(T) == 2;
  const int64_t rows = BH * Lq;
  float* l2 = delta + rows;
  const float sl2 = scale * kLog2e;
  if constexpr (BF) {
    // dQ first: it also writes -D and LSE * log2(e) for the dK/dV kernel
    constexpr int NW = bwd_nw(D);
    const int64_t nkt = (Lk + 32 * NW - 1) / (32 * NW);
    const int64_t nqp = (Lq + 127) / 128;
    if (!grid_fits(nkt * BH, 64 * NW) || !grid_fits(nqp * BH, 256))
      return fail(TT_ERR_ARG, "attention backward: grid too large");
    constexpr int LD = attention_light_div(CAUSAL, D);
    const int gp = tile_order(BH, nqp, 32 * 2, LD), gk = tile_order(BH, nkt, 32 * 8 / NW, LD);
    hipLaunchKernelGGL((attn_bwd_dq_pipe_kernel<D, CAUSAL>), dim3((unsigned)(nqp * BH)), dim3(256), 0, st, q, k, v, o,
                       dout, lse, l2, delta, dq, (int)Lq, (int)Lk, (int)BH, (int)nqp, gp, sl2, scale);
    TT_LAUNCHED("attention backward dQ launch", st);
    if (D == 128 && !(CAUSAL && Lk <= kDkdvTwoWaveMaxLk128))
      return launch_dkdv_w64(q, k, v, dout, l2, delta, dk, dv, BH, Lq, Lk, sl2, scale, CAUSAL, st);
    hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<D, CAUSAL>), dim3((unsigned)(nkt * BH)), dim3(64 * NW), 0, st, q,
                       k, v, dout, l2, delta, dk, dv, (int)Lq, (int)Lk, (int)BH, (int)nkt, gk, sl2, scale);
    TT_LAUNCHED("attention backward dK/dV launch", st);
  } else {
    constexpr int TPR = D / (16 / (int)sizeof(T));
    const int64_t dblk = (rows + (256 / TPR) - 1) / (256 / TPR);
    if (!grid_fits(dblk, 256)) return fail(TT_ERR_ARG, "attention backward: grid too large");
    hipLaunchKernelGGL((attn_bwd_delta_kernel<T, D>), dim3((unsigned)dblk), dim3(256), 0, st, o, dout, lse, delta,
                       l2, rows);
    TT_LAUNCHED("attention backward delta launch", st);

    {
      // fp32: dK/dV and dQ workgroups in one launch
      const int64_t nkt = (Lk + BWD_F32_BN - 1) / BWD_F32_BN;
      const int64_t nqt = (Lq + BWD_F32_BM - 1) / BWD_F32_BM;
      if (!grid_fits((nkt + nqt) * BH, 256)) return fail(TT_ERR_ARG, "attention backward: grid too large");
      const int gk = pick_group(BH, nkt, 32), gq = pick_group(BH, nqt, 32);
      hipLaunchKernelGGL((attn_bwd_f32_kernel<D, CAUSAL>), dim3((unsigned)((nkt + nqt) * BH)), dim3(256), 0, st,
                         q, k, v, dout, lse, delta, dq, dk, dv, (int)Lq, (int)Lk, (int)BH, (int)nkt, (int)nqt,
                         (int)(nkt * BH), gk, gq, sl2, scale);
      TT_LAUNCHED("attention backward dQ / dK / dV launch", st);
    }
  }
  return ok();
}

template <typename T>
static int dispatch_bwd(const char* fn, const T* q, const T* k, const T* v, const T* o, const float* lse,
                        const T* dout, T* dq, T* dk, T* dv, int64_t BH, int64_t Lq, int64_t Lk, int64_t d, float scale,
                        int causal, hipStream_t st, float* delta) {
  switch (d * 2 + (causal ? 1 : 0)) {
    case 64: return launch_bwd<T, 32, false>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st, delta);
    case 65: return launch_bwd<T, 32, true>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st, delta);
    case 128: return launch_bwd<T, 64, false>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st, delta);
    case 129: return launch_bwd<T, 64, true>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st, delta);
    case 256: return launch_bwd<T, 128, false>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st, delta);
    case 257: return launch_bwd<T, 128, true>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st, delta);
    default: return fail(TT_ERR_UNSUPPORTED, std::string(fn) + ": unsupported head dim");
  }
}

// Shared argument checks of the backward entry points.  Returns TT_OK with
// *done = true when nothing is left to launch (no heads, or no queries: then
// dK and dV are zero-filled by a kernel, not a memset, so that the call can
// sit inside a captured graph).
template <typename T>
static int bwd_prologue(const char* fn, const T* q, const T* k, const T* v, const T* o, const float* lse,
                        const T* dout, T* dq, T* dk, T* dv, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                        int causal, hipStream_t st, bool* done) {
  *done = true;
  int rc = check_attn_shape(fn, B, H, Lq, Lk, d, causal);
  if (rc) return rc;
  const int64_t BH = B * H;
  if (BH == 0) return ok();
  if (Lq == 0) {  // no queries: every key gets zero gradient
    if (Lk > 0) {
      if (!dk || !dv) return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
      const int dt = sizeof(T) == 2 ? TT_BF16 : TT_F32;
      if ((rc = tt_elementwise(TT_EW_FILL, dt, dk, nullptr, nullptr, BH * Lk * d, 0.0, 0.0, 0, st))) return rc;
      if ((rc = tt_elementwise(TT_EW_FILL, dt, dv, nullptr, nullptr, BH * Lk * d, 0.0, 0.0, 0, st))) return rc;
    }
    return ok();
  }
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv)
    return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
  const size_t qb = (size_t)(BH * Lq * d) * sizeof(T), kb = (size_t)(BH * Lk * d) * sizeof(T);
  if ((rc = check_no_overlap(fn,
                             {{q, qb, "q"}, {k, kb, "k"}, {v, kb, "v"}, {o, qb, "o"},
                              {lse, (size_t)(BH * Lq) * sizeof(float), "lse"}, {dout, qb, "dO"}},
                             {{dq, qb, "dQ"}, {dk, kb, "dK"}, {dv, kb, "dV"}})))
    return rc;
  *done = false;
  return TT_OK;
}

template <typename T>
static int bwd_entry(const char* fn, const T* q, const T* k, const T* v, const T* o, const float* lse,
                     const T* dout, T* dq, T* dk, T* dv, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                     int64_t d, float scale, int causal, void* stream) {
  int rc = check_attn_shape(fn, B, H, Lq, Lk, d, causal);
  if (rc) return rc;
  if (B * H == 0) return ok();
  if (Lq > 0 && (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv))  // before touching the device
    return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
  if ((rc = ensure_init())) return rc;
  hipStream_t st = stream_or_default(stream);
  bool done = false;
  if ((rc = bwd_prologue(fn, q, k, v, o, lse, dout, dq, dk, dv, B, H, Lq, Lk, d, causal, st, &done)) || done)
    return rc;
  const int64_t BH = B * H;
  float* delta = nullptr;
  WorkspaceLease ws;  // held until the kernels that read the buffer are launched
  if ((rc = ws.get(st, kWsBackwardRows, (size_t)(2 * BH * Lq) * sizeof(float), (void**)&delta))) return rc;
  return dispatch_bwd(fn, q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, d, scale, causal, st, delta);
}

}  // namespace tt

using namespace tt;

extern "C" int tt_attn_bwd_f32(const float* q, const float* k, const float* v, const float* o,
                               const float* lse, const float* do_, float* dq, float* dk, float* dv,
                               int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d, float scale,
                               int causal, void* stream) {
  return bwd_entry<float>("tt_attn_bwd_f32", q, k, v, o, lse, do_, dq, dk, dv, B, H, Lq, Lk, d, scale,
                          causal, stream);
}

extern "C" int tt_attn_bwd_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                const uint16_t* o, const float* lse, const uint16_t* do_, uint16_t* dq,
                                uint16_t* dk, uint16_t* dv, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                                int64_t d, float scale, int causal, void* stream) {
  return bwd_entry<u16>("tt_attn_bwd_bf16", q, k, v, o, lse, do_, dq, dk, dv, B, H, Lq, Lk, d, scale,
                        causal, stream);
}

// The bf16 backward with its row scratch in the library's static device
// array instead of an allocated workspace (see include/tt_attn.h).
extern "C" int tt_attn_bwd_bf16_noalloc(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                        const uint16_t* o, const float* lse, const uint16_t* do_, uint16_t* dq,
                                        uint16_t* dk, uint16_t* dv, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                                        int64_t d, float scale, int causal, void* stream) {
  const char* fn = "tt_attn_bwd_bf16_noalloc";
  int rc = check_attn_shape(fn, B, H, Lq, Lk, d, causal);
  if (rc) return rc;
  if (B * H == 0) return ok();
  size_t cap = 0;
  float* scratch = static_cast<float*>(noalloc_scratch(&cap));
  if (!scratch)
    return fail(TT_ERR_ARG, std::string(fn) + ": call tt_init first (this entry point does no set-up of its own)");
  if (B * H * Lq > (int64_t)(cap / (2 * sizeof(float))))
    return fail(TT_ERR_ARG, std::string(fn) + ": B*H*Lq = " + std::to_string(B * H * Lq) +
                                " rows exceed the static scratch maximum of " +
                                std::to_string(cap / (2 * sizeof(float))) + " rows");
  hipStream_t st = stream_or_default(stream);
  bool done = false;
  if ((rc = bwd_prologue<u16>(fn, q, k, v, o, lse, do_, dq, dk, dv, B, H, Lq, Lk, d, causal, st, &done)) || done)
    return rc;
  return dispatch_bwd<u16>(fn, q, k, v, o, lse, do_, dq, dk, dv, B * H, Lq, Lk, d, scale, causal, st, scratch);
}
