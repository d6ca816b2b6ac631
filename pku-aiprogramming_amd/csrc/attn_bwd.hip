// Fused attention backward for gfx950.
//
// Replaces O.backward(dO) over the reference's composition
// (optimizer/operators.py:115-119 -> autodiff.py:33-61) through the gradient
// rules MatMul (:421-429), Transpose (:338-340), MulScalar (:241-242),
// EWiseDiv (:296-298), BroadcastTo (:373-380), Summation (:400-408) and
// Exp (:469-470).  Closed form of that chain, with P recomputed from the LSE
// saved by the forward so no L x L tensor is ever stored:
//   D_i  = sum_d dO_id O_id                  (pre-pass, fp32 [B,H,L])
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
// All tiles are filled by direct global->LDS loads.  Loads past the end of a
// sequence read a clamped (valid) row and the result is masked, so the
// inner loops carry no load guards.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "attn_bwd_f32.h"
#include "attn_common.h"
#include "attn_tiles.h"

namespace tt {

// Waves per workgroup, pipeline depth, and tile sizes of the bf16 kernels.
// Default: 4-wave workgroups with 2 stages, so two workgroups with
// independent barriers share each CU (2 waves per SIMD); measured faster on
// the MI355X than one 8-wave workgroup with a 4-deep ring.
#ifndef TT_BWD_WAVES
#define TT_BWD_WAVES 4
#endif
#ifndef TT_BWD_STAGES
#define TT_BWD_STAGES 2
#endif
constexpr int bwd_nw(int D) { return D == 32 ? 4 : TT_BWD_WAVES; }
constexpr int kBwdStages = TT_BWD_STAGES;
static_assert(kBwdStages >= 2 && kBwdStages <= 4, "tile ring depth must be 2..4");
constexpr int DQ_BN = 64;  // keys per LDS tile of the dQ kernel
// Query rows per LDS tile of the dK/dV kernel: the ring of Q / dO tiles
// plus the V rows of the workgroup fit 160 KB of LDS.
constexpr int dkdv_bq(int D) { return D == 128 ? 32 : 64; }
// K chunks (16 columns each) the dK/dV kernel keeps in LDS rather than in
// registers.  At d = 128 the dK / dV accumulators (128 VGPRs) and the K rows
// (32) leave too little of the 256 registers of a 2-waves-per-SIMD kernel;
// each parked chunk frees 4 VGPRs for one extra 16-byte LDS read per query
// tile.
#ifndef TT_DKDV_KLDS
#define TT_DKDV_KLDS 3
#endif
constexpr int dkdv_klds(int D) { return D == 128 ? TT_DKDV_KLDS : 0; }

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
template <int D, bool CAUSAL>
__global__ __launch_bounds__(64 * bwd_nw(D), 8 / bwd_nw(D)) void attn_bwd_dkdv_bf16_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ dO, const float* __restrict__ L2, const float* __restrict__ NDelta,
    u16* __restrict__ dK, u16* __restrict__ dV, int Lq, int Lk, int BH, int nkt, int group, float sl2,
    float scale) {
  using Tile = SwzTile<D>;
  constexpr int NW = bwd_nw(D), BN = 32 * NW, BQ = dkdv_bq(D), MT = BQ / 32, S = kBwdStages;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int KL = dkdv_klds(D), KR = NC - KL;  // K chunks parked in LDS / held in registers
  static_assert(KL >= 0 && KL <= NC, "bad K chunk split");
  constexpr int TE = Tile::kElems(BQ);
  constexpr int VS = 64;  // stride of the LSE / D row buffers (one 64-lane load each)
  using Dma = TileDma<D, BQ, NW>;
  constexpr int IPT = 2 * Dma::kLoads;  // Q + dO loads per wave per tile
  // Ring of Q / dO tiles with their LSE (log2) / D rows, and the workgroup's
  // V rows, all filled by direct global->LDS loads
  __shared__ __align__(16) u16 sQ[S * TE];
  __shared__ __align__(16) u16 sdO[S * TE];
  __shared__ __align__(16) u16 sV[Tile::kElems(BN)];
  __shared__ __align__(16) float sL[S * VS];
  __shared__ __align__(16) float sDl[S * VS];
  // parked K chunks, lane-linear: chunk KR + c of lane l of wave w at 16 (64 (c NW + w) + l) bytes
  __shared__ __align__(16) u16 sKf[(KL > 0 ? KL : 1) * NW * 512];

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 5, r32 = l & 31;
  int kt, bh;
  map_tile(blockIdx.x, nkt, BH, group, kt, bh, false);  // causal: key tile 0 sees every query
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
#pragma unroll
    for (int c = KR; c < NC; ++c) *reinterpret_cast<bf16x8*>(&sKf[((c - KR) * NW + w) * 512 + 8 * l]) = kf[c];
  }
  // K operand of chunk c (each lane reads back only what it parked itself)
  auto kop = [&](int c) {
    return c < KR ? kf[c] : *reinterpret_cast<const bf16x8*>(&sKf[((c - KR) * NW + w) * 512 + 8 * l]);
  };
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
      const int b = issued % S, qb = qstart + issued * BQ;
      dma.issue(Q + qbase, qb, Lq, sQ + b * TE);
      dma.issue(dO + qbase, qb, Lq, sdO + b * TE);
      if (w == 0) {
        load_vec_lds(L2 + lbase + qb, Lq - qb, sL + b * VS);
        load_vec_lds(NDelta + lbase + qb, Lq - qb, sDl + b * VS);
      }
      ++issued;
    }
  };

  auto step = [&](int qb, const u16* tQ, const u16* tdO, const float* tL, const float* tD, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      // dP starts at -D of each query row (register r holds row acc_row(r, g)),
      // so the accumulator ends as dP - D
      f32x16 s = f32x16{}, dp;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 nd = *reinterpret_cast<const float4*>(&tD[32 * mt + 8 * j + 4 * g]);
        dp[4 * j] = nd.x;
        dp[4 * j + 1] = nd.y;
        dp[4 * j + 2] = nd.z;
        dp[4 * j + 3] = nd.w;
      }
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int off = Tile::chunk(32 * mt + r32, 2 * c + g);
        s = mfma_bf16_32x32x16(*reinterpret_cast<const bf16x8*>(&tQ[off]), kop(c), s);
        const bf16x8 vb = *reinterpret_cast<const bf16x8*>(&sV[Tile::chunk(32 * w + r32, 2 * c + g)]);
        dp = mfma_bf16_32x32x16(*reinterpret_cast<const bf16x8*>(&tdO[off]), vb, dp);
      }
      // transposed dO / Q operands of dV^T / dK^T MFMA i = h * ND + dt,
      // fetched one MFMA pair ahead
      auto tr_op = [&](const u16* tile_, int i) {
        const int r0 = 32 * mt + 16 * (i / ND) + trow, col = 32 * (i % ND) + tcol;
        return lds_read_tr16x2(&tile_[Tile::at4(r0, col)], &tile_[Tile::at4(r0 + 8, col)]);
      };
      // s[r] = S[query qb + 32mt + acc_row(r, g)][key]
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int qi = 32 * mt + 8 * j + 4 * g;  // rows acc_row(4j..4j+3, g)
        const float4 lv = *reinterpret_cast<const float4*>(&tL[qi]);
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
      // k-chunk h holds queries 32mt + 16h + perm16 order.
      bf16x8 ov[2], oq[2];
      ov[0] = tr_op(tdO, 0);
      oq[0] = tr_op(tQ, 0);
#pragma unroll
      for (int i = 0; i < 2 * ND; ++i) {
        if (i + 1 < 2 * ND) {
          ov[(i + 1) & 1] = tr_op(tdO, i + 1);
          oq[(i + 1) & 1] = tr_op(tQ, i + 1);
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
  auto run = [&](int lo, int hi, auto mask_tag) {
    for (int qb = lo; qb < hi; qb += BQ, ++j) {
      if (w == 0)
        wait_vmem_tiles<IPT + 2>(issued - 1 - j);
      else
        wait_vmem_tiles<IPT>(issued - 1 - j);
      __syncthreads();
      issue_next();
      if (CAUSAL && qb + BQ - 1 < wk_lo) continue;  // every query of the tile precedes every key of the wave
      const int b = j % S;
      step(qb, sQ + b * TE, sdO + b * TE, sL + b * VS, sDl + b * VS, mask_tag);
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
  run(qdiag, qfull, std::false_type{});
  run(max(qdiag, qfull), Lq, std::true_type{});
  wait_vmem_le<0>();  // nothing may be in flight into LDS when the workgroup exits

  if (key < Lk) {
    u16* dkrow = dK + kbase + (int64_t)key * D;
    u16* dvrow = dV + kbase + (int64_t)key * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const int d0 = 32 * dt + acc_row(r, g);
        uint2 a, b;
        a.x = pack_bf16x2(adk[dt][r] * scale, adk[dt][r + 1] * scale);
        a.y = pack_bf16x2(adk[dt][r + 2] * scale, adk[dt][r + 3] * scale);
        b.x = pack_bf16x2(adv[dt][r], adv[dt][r + 1]);
        b.y = pack_bf16x2(adv[dt][r + 2], adv[dt][r + 3]);
        *reinterpret_cast<uint2*>(dkrow + d0) = a;
        *reinterpret_cast<uint2*>(dvrow + d0) = b;
      }
  }
}

// ------------------------------------------------------------------ bf16 dQ
template <int D, bool CAUSAL>
__global__ __launch_bounds__(64 * bwd_nw(D), 8 / bwd_nw(D)) void attn_bwd_dq_bf16_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ dO, const float* __restrict__ L2, const float* __restrict__ NDelta,
    u16* __restrict__ dQ, int Lq, int Lk, int BH, int nqt, int group, float sl2, float scale) {
  using Tile = SwzTile<D>;
  constexpr int NW = bwd_nw(D), BM = 32 * NW, BN = DQ_BN, S = kBwdStages;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int TE = Tile::kElems(BN);
  using Dma = TileDma<D, BN, NW>;
  constexpr int IPT = 2 * Dma::kLoads;  // K + V loads per wave per tile
  // rings of K / V tiles filled by direct global->LDS loads
  __shared__ __align__(16) u16 sK[S * TE];
  __shared__ __align__(16) u16 sV[S * TE];

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 5, r32 = l & 31;
  int qt, bh;
  map_tile(blockIdx.x, nqt, BH, group, qt, bh, CAUSAL);
  const int q0 = qt * BM;
  const int qrow = q0 + 32 * w + r32;
  const int wq_lo = q0 + 32 * w, wq_hi = wq_lo + 31;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;

  bf16x8 qf[NC], dof[NC];
  {
    const int qr = min(qrow, Lq - 1);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qf[c] = __builtin_bit_cast(bf16x8, ldg16(Q + qbase + (int64_t)qr * D + 16 * c + 8 * g));
      dof[c] = __builtin_bit_cast(bf16x8, ldg16(dO + qbase + (int64_t)qr * D + 16 * c + 8 * g));
    }
  }
  // padding query rows (qrow >= Lq): P = 2^(s - inf) = 0
  const float lse2 = qrow < Lq ? L2[(int64_t)bh * Lq + qrow] : INFINITY;
  const float ndl = qrow < Lq ? NDelta[(int64_t)bh * Lq + qrow] : 0.f;
  f32x16 adq[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) adq[dt] = f32x16{};

  const int t16 = l & 15;
  const int trow = 4 * g + (t16 >> 2);
  const int tcol = 16 * ((l >> 4) & 1) + 4 * (t16 & 3);

  // Tile ring over key tiles; rows past Lk read row Lk - 1 and are masked.
  const int kend = CAUSAL ? min(Lk, q0 + BM) : Lk;
  const int ntiles = (kend + BN - 1) / BN;
  Dma dma;
  dma.init();
  int issued = 0;
  auto issue_next = [&]() {
    if (issued < ntiles) {
      const int b = issued % S;
      dma.issue(K + kbase, issued * BN, Lk, sK + b * TE);
      dma.issue(V + kbase, issued * BN, Lk, sV + b * TE);
      ++issued;
    }
  };

  auto tile = [&](int kb, const u16* tK, const u16* tV, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    // Operand fetches run one step ahead of the MFMAs that consume them.
    auto kv_row = [&](const u16* tile_, int t, int c) {
      return *reinterpret_cast<const bf16x8*>(&tile_[Tile::chunk(32 * t + r32, 2 * c + g)]);
    };
    auto kt_op = [&](int t, int i) {  // K^T operand of dQ^T MFMA i = h * ND + dt
      const int r0 = 32 * t + 16 * (i / ND) + trow, col = 32 * (i % ND) + tcol;
      return lds_read_tr16x2(&tK[Tile::at4(r0, col)], &tK[Tile::at4(r0 + 8, col)]);
    };
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x16 s = f32x16{}, dp = f32x16{};
      bf16x8 ka[2], va[2];
      ka[0] = kv_row(tK, t, 0);
      va[0] = kv_row(tV, t, 0);
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        if (c + 1 < NC) {
          ka[(c + 1) & 1] = kv_row(tK, t, c + 1);
          va[(c + 1) & 1] = kv_row(tV, t, c + 1);
        }
        s = mfma_bf16_32x32x16(ka[c & 1], qf[c], s);
        dp = mfma_bf16_32x32x16(va[c & 1], dof[c], dp);
      }
      bf16x8 qa[2];
      qa[0] = kt_op(t, 0);  // in flight during the softmax
      bf16x8 db[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], sl2, -lse2));
        if constexpr (MASK) {
          const int kk = kb + 32 * t + acc_row(r, g);
          if (kk >= Lk || (CAUSAL && kk > qrow)) p = 0.f;
        }
        db[r >> 3][r & 7] = (__bf16)(p * (dp[r] + ndl));
      }
#pragma unroll
      for (int i = 0; i < 2 * ND; ++i) {
        if (i + 1 < 2 * ND) qa[(i + 1) & 1] = kt_op(t, i + 1);
        adq[i % ND] = mfma_bf16_32x32x16(qa[i & 1], db[i / ND], adq[i % ND]);
      }
    }
  };

  int j = 0;
  auto run = [&](int lo, int hi, auto mask_tag) {
    for (int kb = lo; kb < hi; kb += BN, ++j) {
      wait_vmem_tiles<IPT>(issued - 1 - j);
      __syncthreads();
      issue_next();
      if (CAUSAL && kb > wq_hi) continue;
      const int b = j % S;
      tile(kb, sK + b * TE, sV + b * TE, mask_tag);
    }
  };
  for (int s0 = 0; s0 < S - 1; ++s0) issue_next();
  wait_vmem_le<0>();  // retire the Q / dO / LSE / D loads (see the dK/dV kernel)
  const int kfull = CAUSAL ? min(q0, (Lk / BN) * BN) : (Lk / BN) * BN;  // unmasked tiles
  run(0, kfull, std::false_type{});
  run(kfull, kend, std::true_type{});

  if (qrow < Lq) {
    u16* row = dQ + qbase + (int64_t)qrow * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        uint2 v;
        v.x = pack_bf16x2(adq[dt][r] * scale, adq[dt][r + 1] * scale);
        v.y = pack_bf16x2(adq[dt][r + 2] * scale, adq[dt][r + 3] * scale);
        *reinterpret_cast<uint2*>(row + 32 * dt + acc_row(r, g)) = v;
      }
  }
}

// ------------------------------------------------------------------ launchers
template <typename T, int D, bool CAUSAL>
static int launch_bwd(const T* q, const T* k, const T* v, const T* o, const float* lse, const T* dout,
                      T* dq, T* dk, T* dv, int64_t BH, int64_t Lq, int64_t Lk, float scale, hipStream_t st) {
  constexpr bool BF = sizeof(T) == 2;
  // workspace: -D (negated row sums of dO o O) and LSE * log2(e), fp32 [B*H*Lq] each
  float* delta = nullptr;
  int rc = workspace(0, (size_t)(2 * BH * Lq) * sizeof(float), (void**)&delta);
  if (rc) return rc;
  const int64_t rows = BH * Lq;
  float* l2 = delta + rows;
  constexpr int TPR = D / (16 / (int)sizeof(T));
  const int64_t dblk = (rows + (256 / TPR) - 1) / (256 / TPR);
  if (dblk > 0x7fffffff) return fail(TT_ERR_ARG, "attention backward: grid too large");
  hipLaunchKernelGGL((attn_bwd_delta_kernel<T, D>), dim3((unsigned)dblk), dim3(256), 0, st, o, dout, lse, delta,
                     l2, rows);
  TT_LAUNCHED("attention backward delta launch", st);

  const float sl2 = scale * kLog2e;
  if constexpr (BF) {
    constexpr int NW = bwd_nw(D);
    const int64_t nkt = (Lk + 32 * NW - 1) / (32 * NW);
    const int64_t nqt = (Lq + 32 * NW - 1) / (32 * NW);
    if (nkt * BH > 0x7fffffff || nqt * BH > 0x7fffffff) return fail(TT_ERR_ARG, "attention backward: grid too large");
    // heads in flight per XCD: tiles for the resident workgroups of its 32 CUs
    const int gk = pick_group(BH, nkt, 32 * 8 / NW), gq = pick_group(BH, nqt, 32 * 8 / NW);
    hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<D, CAUSAL>), dim3((unsigned)(nkt * BH)), dim3(64 * NW), 0, st,
                       q, k, v, dout, l2, delta, dk, dv, (int)Lq, (int)Lk, (int)BH, (int)nkt, gk, sl2, scale);
    TT_LAUNCHED("attention backward dK/dV launch", st);
    hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<D, CAUSAL>), dim3((unsigned)(nqt * BH)), dim3(64 * NW), 0, st,
                       q, k, v, dout, l2, delta, dq, (int)Lq, (int)Lk, (int)BH, (int)nqt, gq, sl2, scale);
    TT_LAUNCHED("attention backward dQ launch", st);
  } else {
    const int64_t nkt = (Lk + BWD_F32_BN - 1) / BWD_F32_BN;
    const int64_t nqt = (Lq + BWD_F32_BM - 1) / BWD_F32_BM;
    if (nkt * BH > 0x7fffffff || nqt * BH > 0x7fffffff) return fail(TT_ERR_ARG, "attention backward: grid too large");
    const int gk = pick_group(BH, nkt, 32), gq = pick_group(BH, nqt, 32);
    hipLaunchKernelGGL((attn_bwd_dkdv_f32_kernel<D, CAUSAL>), dim3((unsigned)(nkt * BH)), dim3(256), 0, st,
                       q, k, v, dout, lse, delta, dk, dv, (int)Lq, (int)Lk, (int)BH, (int)nkt, gk, sl2, scale);
    TT_LAUNCHED("attention backward dK/dV launch", st);
    hipLaunchKernelGGL((attn_bwd_dq_f32_kernel<D, CAUSAL>), dim3((unsigned)(nqt * BH)), dim3(256), 0, st,
                       q, k, v, dout, lse, delta, dq, (int)Lq, (int)Lk, (int)BH, (int)nqt, gq, sl2, scale);
    TT_LAUNCHED("attention backward dQ launch", st);
  }
  return ok();
}

template <typename T>
static int bwd_entry(const char* fn, const T* q, const T* k, const T* v, const T* o, const float* lse,
                     const T* dout, T* dq, T* dk, T* dv, int64_t B, int64_t H, int64_t Lq, int64_t Lk,
                     int64_t d, float scale, int causal, void* stream) {
  int rc = check_attn_shape(fn, B, H, Lq, Lk, d, causal);
  if (rc) return rc;
  const int64_t BH = B * H;
  if (BH == 0) return ok();
  if (Lq == 0) {  // no queries: every key gets zero gradient
    if (Lk > 0) {
      if (!dk || !dv) return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
      if ((rc = ensure_init())) return rc;
      hipStream_t st = stream_or_default(stream);
      TT_HIP(hipMemsetAsync(dk, 0, (size_t)(BH * Lk * d) * sizeof(T), st));
      TT_HIP(hipMemsetAsync(dv, 0, (size_t)(BH * Lk * d) * sizeof(T), st));
    }
    return ok();
  }
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv)
    return fail(TT_ERR_ARG, std::string(fn) + ": null pointer");
  if ((rc = ensure_init())) return rc;
  hipStream_t st = stream_or_default(stream);
  switch (d * 2 + (causal ? 1 : 0)) {
    case 64: return launch_bwd<T, 32, false>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st);
    case 65: return launch_bwd<T, 32, true>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st);
    case 128: return launch_bwd<T, 64, false>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st);
    case 129: return launch_bwd<T, 64, true>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st);
    case 256: return launch_bwd<T, 128, false>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st);
    case 257: return launch_bwd<T, 128, true>(q, k, v, o, lse, dout, dq, dk, dv, BH, Lq, Lk, scale, st);
    default: return fail(TT_ERR_UNSUPPORTED, std::string(fn) + ": unsupported head dim");
  }
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
