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
#ifndef TT_DKDV_BQ128
#define TT_DKDV_BQ128 32
#endif
constexpr int dkdv_bq(int D) { return D == 128 ? TT_DKDV_BQ128 : 64; }
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
// MAT: also store dS for attn_bwd_dq_gemm_kernel, as one 2 KB image per
// (32 keys, 32 queries) block (see ds_image_row); query tiles a wave skips
// (all of its keys after all of the tile's queries) are stored as zeros.
// Requires Lq, Lk multiples of the key tile.
template <int D, bool CAUSAL, bool MAT>
__global__ __launch_bounds__(64 * bwd_nw(D), 8 / bwd_nw(D)) void attn_bwd_dkdv_bf16_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ dO, const float* __restrict__ L2, const float* __restrict__ NDelta,
    u16* __restrict__ dK, u16* __restrict__ dV, u16* __restrict__ dST, int Lq, int Lk, int BH, int nkt,
    int group, float sl2, float scale) {
  using Tile = SwzTile<D>;
  constexpr int NW = bwd_nw(D), BN = 32 * NW, BQ = dkdv_bq(D), MT = BQ / 32, S = kBwdStages;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int KL = dkdv_klds(D), KR = NC - KL;  // K chunks parked in LDS / held in registers
  static_assert(KL >= 0 && KL <= NC, "bad K chunk split");
  constexpr int TE = Tile::kElems(BQ);
  constexpr int VS = 64;  // stride of the LSE / D row buffers (one 64-lane load each)
  using Dma = TileDma<D, BQ, NW>;
  constexpr int IPT = 2 * Dma::kLoads;  // Q + dO loads per wave per tile
  constexpr int kStores = MAT ? 2 * MT : 0;  // dS image stores per wave per tile
  // One LDS block, carved at fixed byte offsets so that every operand read
  // is a per-lane address plus an immediate: the ring of Q / dO tiles with
  // their LSE (log2) / D rows and the workgroup's V rows, all filled by direct
  // global->LDS loads, then the parked K chunks (lane-linear: chunk KR + c of
  // lane l of wave w at 16 (64 (c NW + w) + l) bytes).
  constexpr int kOQ = 0, kOdO = kOQ + 2 * S * TE, kOV = kOdO + 2 * S * TE, kOL = kOV + 2 * Tile::kElems(BN),
                kOD = kOL + 4 * S * VS, kOK = kOD + 4 * S * VS, kLds = kOK + (KL > 0 ? KL : 1) * NW * 1024;
  static_assert(kOV <= 65536, "Q / dO ring offsets exceed the 16-bit LDS immediate");
  __shared__ __align__(16) char smem[kLds];
  u16* const sQ = reinterpret_cast<u16*>(smem + kOQ);
  u16* const sdO = reinterpret_cast<u16*>(smem + kOdO);
  u16* const sV = reinterpret_cast<u16*>(smem + kOV);
  float* const sL = reinterpret_cast<float*>(smem + kOL);
  float* const sDl = reinterpret_cast<float*>(smem + kOD);
  u16* const sKf = reinterpret_cast<u16*>(smem + kOK);
  const uint32_t a0 = lds_addr(smem);

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, g = l >> 5, r32 = l & 31;
  const int wu = __builtin_amdgcn_readfirstlane(w);  // w, known wave-uniform (scalar branches)
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
  uint32_t kofs = a0 + kOK + 16 * (64 * w + l);
  auto kop = [&](int c) { return c < KR ? kf[c] : lds_ld<bf16x8>(kofs + (c - KR) * NW * 1024); };
  // dS image of (this wave's 32 keys, the 32 queries at q): this lane's 16
  // accumulator values, 32 contiguous bytes at row ds_image_row(l) of image
  // ((bh, q / 128, key / 32), (q / 32) % 4).  Stored non-temporal: the dQ
  // GEMM reads it back from HBM.
  u16* const dsimg = MAT ? dST + (((int64_t)bh * (Lq / 128)) * (Lk / 32) + key / 32) * 4096 + 16 * ds_image_row(l)
                         : nullptr;
  const int64_t img_row = (int64_t)(Lk / 32) * 4096;  // elements per 128 query rows of dS images
  auto store_ds = [&](int q, const bf16x8 (&db)[2]) {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const unsigned uq = q;  // q >= 0: unsigned division is a shift
    u16* p = dsimg + (int64_t)(uq / 128) * img_row + (uq / 32 % 4) * 1024;
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, db[0]), reinterpret_cast<u32x4*>(p));
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, db[1]), reinterpret_cast<u32x4*>(p + 8));
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
        s = mfma_bf16_32x32x16(lds_ld<bf16x8>(off), kop(c), s);
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
      if constexpr (MAT) store_ds(qb + 32 * mt, db);
      // dV^T += dO^T P and dK^T += Q^T dS over the 32 queries of this half:
      // k-chunk h holds queries 32mt + 16h + perm16 order.
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
      // In flight: this tile's loads (issued after the previous tile's
      // barrier), then the previous tile's dS stores.  Loads and stores retire
      // in issue order, so the stores need not drain here.
      wait_vmem_le<kStores>();
    } else if (wu == 0) {
      wait_vmem_tiles<IPT + 2 + kStores, S - 1>(issued - 1 - j);
    } else {
      wait_vmem_tiles<IPT + kStores, S - 1>(issued - 1 - j);
    }
    __syncthreads();
    issue_next();
    if constexpr (CAUSAL && decltype(mask_tag)::value) {
      if (qb + BQ - 1 < wk_lo) {  // every query of the tile precedes every key of the wave
        if constexpr (MAT) {
          const bf16x8 zero[2] = {bf16x8{}, bf16x8{}};
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) store_ds(qb + 32 * mt, zero);
        }
        return;
      }
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
    opaque(kofs);
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

// ------------------------------------------------------------------ bf16 dQ from stored dS
// dQ = s dS K as one GEMM over the dS the dK/dV kernel stored, so dQ needs
// no recompute of S and dP.  dS is stored as 2 KB images, one per (32 keys,
// 32 queries) block, in [BH][Lq/128][Lk/32][4] order (the images one
// workgroup reads form one contiguous stream): the dK/dV accumulator
// registers as they are (lane l = key l % 32 of queries with g = l / 32;
// register r = query 8(r/4) + 4g + r%4), row l at row ds_image_row(l).
//
// Workgroup = 4 waves x 32 queries = DQG_BM queries (one dK/dV key tile wide,
// so every block it reads was written; above the diagonal as zeros).  Stages
// of 32 keys (K rows, and the 4 dS images of the workgroup's queries, 8 KB
// contiguous) stream through a TT_DQG_STAGES-deep LDS ring.  Per stage and
// wave dQ^T (d x 32 queries) += K^T dS^T, both operands by LDS transpose
// reads.  The dS operand puts query q(n) = 8(n%16 / 4) + 4(n / 16 % 2) + n % 4
// of the wave's 32 in MFMA column n and keys in natural order (the K^T
// operand reads its rows in the same order); output rows follow q(n).
// Requires Lq, Lk multiples of DQG_BM.
constexpr int DQG_BM = 128;
constexpr int DQG_BN = 32;  // keys per stage
// dS images are read once: loading them non-temporal keeps the K rows, which
// every query tile of a head re-reads, in L2 (8 % less HBM fetch, same time).
#ifndef TT_DQG_NT
#define TT_DQG_NT 1
#endif
#ifndef TT_DQG_STAGES
#define TT_DQG_STAGES 4
#endif
constexpr size_t kMaxDsBytes = size_t(8) << 30;  // largest dS workspace (bf16, Lq x Lk per head)

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_gemm_kernel(const u16* __restrict__ K,
                                                                  const u16* __restrict__ dS,
                                                                  u16* __restrict__ dQ, int Lq, int Lk, int BH,
                                                                  int nqt, int group, float scale) {
  constexpr int NW = 4, BM = DQG_BM, BN = DQG_BN, ND = D / 32, S = TT_DQG_STAGES;
  static_assert(S >= 2 && S <= 4, "ring depth 2..4");
  using KTile = SwzTile<D>;
  constexpr int KE = KTile::kElems(BN), SE = (BM / 32) * 1024;  // elements per stage
  using KDma = TileDma<D, BN, NW>;
  constexpr int SL = SE / (NW * 512);  // dS load instructions per wave per stage (1 KB each)
  constexpr int PER = KDma::kLoads + SL;
  __shared__ __align__(16) u16 sK[S * KE];
  __shared__ __align__(16) u16 sS[S * SE];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, g = l >> 5;
  int qt, bh;
  map_tile(blockIdx.x, nqt, BH, group, qt, bh, CAUSAL);
  const int q0 = qt * BM;
  const int64_t kbase = (int64_t)bh * Lk * D;
  // images of key block n and the workgroup's 4 query blocks: 8 KB at simg + 4096 n
  const u16* simg = dS + ((int64_t)bh * (Lq / BM) + qt) * (Lk / 32) * 4096;

  // Transpose reads: lane s of each 16-lane group points at row base + s / 4,
  // 8-byte piece s % 4; the group then receives 4 consecutive rows of 16
  // columns.  K^T operand of key chunk kc, half g: keys 16kc + 8g + (0..3)
  // and 16kc + 8g + 4 + (0..3), d columns 32dt + 16G + (0..15).  dS operand:
  // image rows 32G + the same keys, all 16 register columns.
  const int t16 = l & 15, G = (l >> 4) & 1;
  const int krow = 8 * g + (t16 >> 2), kcol = 16 * G + 4 * (t16 & 3);
  const int srow = 32 * G + 8 * g, scol = 4 * (t16 & 3);

  f32x16 acc[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) acc[dt] = f32x16{};

  const int ntiles = (CAUSAL ? min(Lk, q0 + BM) : Lk) / BN;
  KDma kdma;
  kdma.init();
  int issued = 0;
  auto issue_next = [&]() {
    if (issued < ntiles) {
      const int b = issued % S;
      kdma.issue(K + kbase, BN * issued, Lk, sK + b * KE);
      const u16* src = simg + (int64_t)issued * 4096;
      const uint32_t lds = lds_addr(sS + b * SE);
#pragma unroll
      for (int i = 0; i < SL; ++i) {
        const uint32_t off = 1024u * (uint32_t)(i * NW + w);
#if TT_DQG_NT
        glds16_nt(src, off + 16u * (uint32_t)l, lds + off);
#else
        glds16(src, off + 16u * (uint32_t)l, lds + off);
#endif
      }
      ++issued;
    }
  };
  for (int s0 = 0; s0 < S - 1; ++s0) issue_next();
  for (int n = 0; n < ntiles; ++n) {
    wait_vmem_tiles<PER>(issued - 1 - n);  // tiles n + 1 .. issued - 1 may stay in flight
    __syncthreads();
    issue_next();
    const u16* tK = sK + (n % S) * KE;
    const u16* tS = sS + (n % S) * SE + w * 1024;  // this wave's query block
#pragma unroll
    for (int kc = 0; kc < BN / 16; ++kc) {
      const int sr = srow + 16 * kc;  // a multiple of 4; rows sr .. sr + 3 and sr + 4 .. sr + 7
      const bf16x8 b = lds_read_tr16x2(&tS[16 * (ds_image_row(sr) + (t16 >> 2)) + scol],
                                       &tS[16 * (ds_image_row(sr + 4) + (t16 >> 2)) + scol]);
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const int r0 = 16 * kc + krow;
        const bf16x8 a =
            lds_read_tr16x2(&tK[KTile::at4(r0, 32 * dt + kcol)], &tK[KTile::at4(r0 + 4, 32 * dt + kcol)]);
        acc[dt] = mfma_bf16_32x32x16(a, b, acc[dt]);
      }
    }
  }
  wait_vmem_le<0>();  // nothing may be in flight into LDS when the workgroup exits

  const int n = l & 31;
  const int q = q0 + 32 * w + 8 * ((n & 15) >> 2) + 4 * ((n >> 4) & 1) + (n & 3);
  u16* row = dQ + ((int64_t)bh * Lq + q) * D;
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int r = 0; r < 16; r += 4) {
      uint2 v;
      v.x = pack_bf16x2(acc[dt][r] * scale, acc[dt][r + 1] * scale);
      v.y = pack_bf16x2(acc[dt][r + 2] * scale, acc[dt][r + 3] * scale);
      *reinterpret_cast<uint2*>(row + 32 * dt + acc_row(r, g)) = v;
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
    // dQ: one GEMM over the stored dS when the tiles are full and the dS
    // workspace stays under kMaxDsBytes; otherwise recompute S and dP.
    if constexpr (D >= 64) {
      const size_t ds_bytes = (size_t)BH * (size_t)Lk * (size_t)Lq * sizeof(u16);
      const bool mat = (32 * NW) % DQG_BM == 0 && Lq % DQG_BM == 0 && Lk % (32 * NW) == 0 &&
                       Lq <= (int64_t(1) << 24) && ds_bytes <= kMaxDsBytes;
      if (mat) {
        u16* ds = nullptr;
        if ((rc = workspace(2, ds_bytes, (void**)&ds))) return rc;
        hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<D, CAUSAL, true>), dim3((unsigned)(nkt * BH)), dim3(64 * NW),
                           0, st, q, k, v, dout, l2, delta, dk, dv, ds, (int)Lq, (int)Lk, (int)BH, (int)nkt, gk, sl2,
                           scale);
        TT_LAUNCHED("attention backward dK/dV launch", st);
        const int64_t nqg = Lq / DQG_BM;
        const int gg = pick_group(BH, nqg, 32 * 2);
        hipLaunchKernelGGL((attn_bwd_dq_gemm_kernel<D, CAUSAL>), dim3((unsigned)(nqg * BH)), dim3(256), 0, st, k, ds,
                           dq, (int)Lq, (int)Lk, (int)BH, (int)nqg, gg, scale);
        TT_LAUNCHED("attention backward dQ launch", st);
        return ok();
      }
    }
    hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<D, CAUSAL, false>), dim3((unsigned)(nkt * BH)), dim3(64 * NW), 0,
                       st, q, k, v, dout, l2, delta, dk, dv, nullptr, (int)Lq, (int)Lk, (int)BH, (int)nkt, gk, sl2,
                       scale);
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
