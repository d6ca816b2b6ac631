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
//   dkdv: workgroup = 128 keys (32 per wave, lane = key, K/V rows held in
//         registers); loops over query tiles of 64 staged once in LDS.  The
//         same LDS tile feeds the S / dP operands (16-byte row reads) and the
//         transposed dV^T += dO^T P, dK^T += Q^T dS operands (gfx950
//         transpose reads), so nothing is transposed on the way in.
//   dq:   workgroup = 128 queries (lane = query, as in the forward); loops over
//         key tiles of 64: S^T and dP^T from K / V row reads, dQ^T += K^T dS^T
//         from transpose reads of the same K tile.
// Loads past the end of a sequence read a clamped (valid) row and the
// result is masked, so the inner loops carry no load guards.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "attn_common.h"
#include "attn_tiles.h"

namespace tt {

constexpr int DKDV_BN = 128;  // keys per workgroup
constexpr int DKDV_BQ = 64;   // queries per LDS step (fp32 kernel)
constexpr int DQ_BM = 128;    // queries per workgroup
constexpr int DQ_BN = 64;     // keys per LDS step

// D_i = sum_d dO[i][d] * O[i][d], one 16-byte chunk per thread; also
// L2_i = LSE_i * log2(e), the log-sum-exp in the log2 domain the MFMA
// kernels exponentiate in.
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const T* __restrict__ O,
                                                             const T* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             float* __restrict__ Delta, float* __restrict__ L2,
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
    Delta[row] = sum;
    L2[row] = LSE[row] * kLog2e;
  }
}

// ------------------------------------------------------------------ bf16 dK, dV
// Query rows per LDS step of the dK/dV kernel: 32 at d = 128 keeps the
// double-buffered Q / dO tiles plus the V tile at 64.5 KB, so two
// workgroups (2 waves per SIMD) share a CU.
constexpr int dkdv_bq(int D) { return D == 128 ? 32 : 64; }

template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkdv_bf16_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ dO, const float* __restrict__ L2, const float* __restrict__ Delta,
    u16* __restrict__ dK, u16* __restrict__ dV, int Lq, int Lk, int BH, int nkt, int group, float sl2,
    float scale) {
  using Tile = SwzTile<D>;
  constexpr int BN = DKDV_BN, BQ = dkdv_bq(D), MT = BQ / 32;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int TE = Tile::kElems(BQ);
  constexpr int VS = 64;  // stride of the LSE / D row buffers (one 64-lane load each)
  // Q / dO tiles and their LSE (log2) / D rows, double-buffered, and the
  // workgroup's V rows, all filled by direct global->LDS loads
  __shared__ __align__(16) u16 sQ[2 * TE];
  __shared__ __align__(16) u16 sdO[2 * TE];
  __shared__ __align__(16) u16 sV[Tile::kElems(BN)];
  __shared__ __align__(16) float sL[2 * VS];
  __shared__ __align__(16) float sDl[2 * VS];

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, r32 = l & 31;
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
  }
  load_tile_lds<D, BN>(V + kbase, k0, Lk, sV);  // published by the first loop barrier
  f32x16 adk[ND], adv[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) adk[dt] = adv[dt] = f32x16{};

  // transpose-read addressing (this lane as a source row/column)
  const int t16 = l & 15;
  const int trow = 4 * g + (t16 >> 2);
  const int tcol = 16 * ((l >> 4) & 1) + 4 * (t16 & 3);

  // Query rows past Lq read row Lq - 1 and are masked (P = 0) in the edge step.
  auto issue = [&](int qb, int buf) {
    load_tile_lds<D, BQ>(Q + qbase, qb, Lq, sQ + buf * TE);
    load_tile_lds<D, BQ>(dO + qbase, qb, Lq, sdO + buf * TE);
    if (w == 0) {
      load_vec_lds(L2 + lbase + qb, Lq - qb, sL + buf * VS);
      load_vec_lds(Delta + lbase + qb, Lq - qb, sDl + buf * VS);
    }
  };

  auto step = [&](int qb, const u16* tQ, const u16* tdO, const float* tL, const float* tD, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int off = Tile::chunk(32 * mt + r32, 2 * c + g);
        s = mfma_bf16_32x32x16(*reinterpret_cast<const bf16x8*>(&tQ[off]), kf[c], s);
        const bf16x8 vb = *reinterpret_cast<const bf16x8*>(&sV[Tile::chunk(32 * w + r32, 2 * c + g)]);
        dp = mfma_bf16_32x32x16(*reinterpret_cast<const bf16x8*>(&tdO[off]), vb, dp);
      }
      // s[r] = S[query qb + 32mt + acc_row(r, g)][key]
      bf16x8 pb[2], db[2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int qi = 32 * mt + 8 * j + 4 * g;  // rows acc_row(4j..4j+3, g)
        const float4 lv = *reinterpret_cast<const float4*>(&tL[qi]);
        const float4 dv = *reinterpret_cast<const float4*>(&tD[qi]);
        const float la[4] = {lv.x, lv.y, lv.z, lv.w};
        const float da[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * j + u;
          float p = fast_exp2(fmaf(s[r], sl2, -la[u]));
          if constexpr (MASK) {
            const int q = qb + qi + u;
            if (q >= Lq || (CAUSAL && key > q)) p = 0.f;
          }
          pb[r >> 3][r & 7] = (__bf16)p;
          db[r >> 3][r & 7] = (__bf16)(p * (dp[r] - da[u]));
        }
      }
      // dV^T += dO^T P and dK^T += Q^T dS over the 32 queries of this half:
      // k-chunk h holds queries 32mt + 16h + perm16 order.
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const int r0 = 32 * mt + 16 * h + trow;
          const int o0 = Tile::at4(r0, 32 * dt + tcol), o1 = Tile::at4(r0 + 8, 32 * dt + tcol);
          adv[dt] = mfma_bf16_32x32x16(lds_read_tr16x2(&tdO[o0], &tdO[o1]), pb[h], adv[dt]);
          adk[dt] = mfma_bf16_32x32x16(lds_read_tr16x2(&tQ[o0], &tQ[o1]), db[h], adk[dt]);
        }
    }
  };

  // Masked (diagonal / ragged) and unmasked query tiles run in separate
  // loops so that neither loop switches the accumulators' registers.
  int j = 0;
  auto run = [&](int lo, int hi, auto mask_tag) {
    for (int qb = lo; qb < hi; qb += BQ, ++j) {
      wait_vmem();
      __syncthreads();  // publishes tile j, retires all reads of the buffer refilled next
      if (qb + BQ < Lq) issue(qb + BQ, (j + 1) & 1);
      if (CAUSAL && qb + BQ - 1 < wk_lo) continue;  // every query of the tile precedes every key of the wave
      const int b = j & 1;
      step(qb, sQ + b * TE, sdO + b * TE, sL + b * VS, sDl + b * VS, mask_tag);
    }
  };
  const int qstart = CAUSAL ? k0 : 0;  // k0 is a multiple of BQ
  if (qstart < Lq) issue(qstart, 0);
  const int qfull = (Lq / BQ) * BQ;
  const int qdiag = CAUSAL ? min(k0 + BN, Lq) : qstart;  // [qstart, qdiag): tiles crossing the diagonal
  run(qstart, qdiag, std::true_type{});
  run(qdiag, qfull, std::false_type{});
  run(max(qdiag, qfull), Lq, std::true_type{});

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
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_bf16_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ dO, const float* __restrict__ L2, const float* __restrict__ Delta,
    u16* __restrict__ dQ, int Lq, int Lk, int BH, int nqt, int group, float sl2, float scale) {
  using Tile = SwzTile<D>;
  constexpr int BM = DQ_BM, BN = DQ_BN;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int TE = Tile::kElems(BN);
  // K / V tiles, double-buffered, filled by direct global->LDS loads
  __shared__ __align__(16) u16 sK[2 * TE];
  __shared__ __align__(16) u16 sV[2 * TE];

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, r32 = l & 31;
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
  const float dl = qrow < Lq ? Delta[(int64_t)bh * Lq + qrow] : 0.f;
  f32x16 adq[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) adq[dt] = f32x16{};

  const int t16 = l & 15;
  const int trow = 4 * g + (t16 >> 2);
  const int tcol = 16 * ((l >> 4) & 1) + 4 * (t16 & 3);

  // key rows past Lk read row Lk - 1 and are masked (P = 0) in the edge tile
  auto issue = [&](int kb, int buf) {
    load_tile_lds<D, BN>(K + kbase, kb, Lk, sK + buf * TE);
    load_tile_lds<D, BN>(V + kbase, kb, Lk, sV + buf * TE);
  };

  auto tile = [&](int kb, const u16* tK, const u16* tV, auto mask_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int off = Tile::chunk(32 * t + r32, 2 * c + g);
        s = mfma_bf16_32x32x16(*reinterpret_cast<const bf16x8*>(&tK[off]), qf[c], s);
        dp = mfma_bf16_32x32x16(*reinterpret_cast<const bf16x8*>(&tV[off]), dof[c], dp);
      }
      bf16x8 db[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], sl2, -lse2));
        if constexpr (MASK) {
          const int kk = kb + 32 * t + acc_row(r, g);
          if (kk >= Lk || (CAUSAL && kk > qrow)) p = 0.f;
        }
        db[r >> 3][r & 7] = (__bf16)(p * (dp[r] - dl));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const int r0 = 32 * t + 16 * h + trow;
          const bf16x8 a = lds_read_tr16x2(&tK[Tile::at4(r0, 32 * dt + tcol)], &tK[Tile::at4(r0 + 8, 32 * dt + tcol)]);
          adq[dt] = mfma_bf16_32x32x16(a, db[h], adq[dt]);
        }
    }
  };

  const int kend = CAUSAL ? min(Lk, q0 + BM) : Lk;
  int j = 0;
  auto run = [&](int lo, int hi, auto mask_tag) {
    for (int kb = lo; kb < hi; kb += BN, ++j) {
      wait_vmem();
      __syncthreads();  // publishes tile j, retires all reads of the buffer refilled next
      if (kb + BN < kend) issue(kb + BN, (j + 1) & 1);
      if (CAUSAL && kb > wq_hi) continue;
      tile(kb, sK + (j & 1) * TE, sV + (j & 1) * TE, mask_tag);
    }
  };
  if (kend > 0) issue(0, 0);
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

// ------------------------------------------------------------------ fp32 dK, dV
// Same schedule on v_mfma_f32_32x32x2f32.  Each fp32 MFMA takes one k-value
// per lane half, so the transposed operands are plain column reads of the
// row-major tiles (consecutive lanes, consecutive columns).
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Delta,
    float* __restrict__ dK, float* __restrict__ dV, int Lq, int Lk, int BH, int nkt, int group,
    float sl2, float scale) {
  constexpr int BN = DKDV_BN, BQ = DKDV_BQ;
  constexpr int P = D + 1;
  constexpr int NC = D / 2, ND = D / 32, CPR = D / 4;
  constexpr int LPT = BQ * CPR / 256;
  __shared__ float sQ[BQ * P];
  __shared__ float sdO[BQ * P];
  __shared__ float sL[BQ];
  __shared__ float sDl[BQ];

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, r32 = l & 31;
  int kt, bh;
  map_tile(blockIdx.x, nkt, BH, group, kt, bh, false);
  const int k0 = kt * BN;
  const int key = k0 + 32 * w + r32;
  const int wk_lo = k0 + 32 * w;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;
  const int64_t lbase = (int64_t)bh * Lq;

  float kf[NC], vf[NC];
  {
    const int kr = min(key, Lk - 1);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      kf[c] = K[kbase + (int64_t)kr * D + 2 * c + g];
      vf[c] = V[kbase + (int64_t)kr * D + 2 * c + g];
    }
  }
  f32x16 adk[ND], adv[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) adk[dt] = adv[dt] = f32x16{};

  float4 qreg[LPT], oreg[LPT];
  float lreg = 0.f, dreg = 0.f;
  auto gload = [&](int qb) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + 256 * i;
      const int row = min(qb + c / CPR, Lq - 1), ch = c % CPR;
      qreg[i] = *reinterpret_cast<const float4*>(Q + qbase + (int64_t)row * D + 4 * ch);
      oreg[i] = *reinterpret_cast<const float4*>(dO + qbase + (int64_t)row * D + 4 * ch);
    }
    if (tid < BQ) {
      const bool in = qb + tid < Lq;
      lreg = in ? LSE[lbase + qb + tid] * kLog2e : INFINITY;
      dreg = in ? Delta[lbase + qb + tid] : 0.f;
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + 256 * i;
      const int row = c / CPR, ch = c % CPR;
      float* pq = &sQ[row * P + 4 * ch];
      float* po = &sdO[row * P + 4 * ch];
      pq[0] = qreg[i].x; pq[1] = qreg[i].y; pq[2] = qreg[i].z; pq[3] = qreg[i].w;
      po[0] = oreg[i].x; po[1] = oreg[i].y; po[2] = oreg[i].z; po[3] = oreg[i].w;
    }
    if (tid < BQ) {
      sL[tid] = lreg;
      sDl[tid] = dreg;
    }
  };

  const int qstart = CAUSAL ? (k0 / BQ) * BQ : 0;
  if (qstart < Lq) gload(qstart);
  for (int qb = qstart; qb < Lq; qb += BQ) {
    __syncthreads();
    sstore();
    __syncthreads();
    if (qb + BQ < Lq) gload(qb + BQ);
    if (CAUSAL && qb + BQ - 1 < wk_lo) continue;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        s = mfma_f32_32x32x2(sQ[(32 * mt + r32) * P + 2 * c + g], kf[c], s);
        dp = mfma_f32_32x32x2(sdO[(32 * mt + r32) * P + 2 * c + g], vf[c], dp);
      }
      const bool need_mask = CAUSAL && (qb + 32 * mt < wk_lo + 31);
      float pr[16], dsr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = 32 * mt + acc_row(r, g);
        float p = fast_exp2(fmaf(s[r], sl2, -sL[qi]));
        if (need_mask && key > qb + qi) p = 0.f;
        pr[r] = p;
        dsr[r] = p * (dp[r] - sDl[qi]);
      }
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = 32 * mt + acc_row(r, g);
          adv[dt] = mfma_f32_32x32x2(sdO[qi * P + 32 * dt + r32], pr[r], adv[dt]);
          adk[dt] = mfma_f32_32x32x2(sQ[qi * P + 32 * dt + r32], dsr[r], adk[dt]);
        }
    }
  }

  if (key < Lk) {
    float* dkrow = dK + kbase + (int64_t)key * D;
    float* dvrow = dV + kbase + (int64_t)key * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const int d0 = 32 * dt + acc_row(r, g);
        float4 a = {adk[dt][r] * scale, adk[dt][r + 1] * scale, adk[dt][r + 2] * scale, adk[dt][r + 3] * scale};
        float4 b = {adv[dt][r], adv[dt][r + 1], adv[dt][r + 2], adv[dt][r + 3]};
        *reinterpret_cast<float4*>(dkrow + d0) = a;
        *reinterpret_cast<float4*>(dvrow + d0) = b;
      }
  }
}

// ------------------------------------------------------------------ fp32 dQ
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void attn_bwd_dq_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Delta,
    float* __restrict__ dQ, int Lq, int Lk, int BH, int nqt, int group, float sl2, float scale) {
  constexpr int BM = DQ_BM, BN = DQ_BN;
  constexpr int P = D + 1;
  constexpr int NC = D / 2, ND = D / 32, CPR = D / 4;
  constexpr int LPT = BN * CPR / 256;
  __shared__ float sK[BN * P];
  __shared__ float sV[BN * P];

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, r32 = l & 31;
  int qt, bh;
  map_tile(blockIdx.x, nqt, BH, group, qt, bh, CAUSAL);
  const int q0 = qt * BM;
  const int qrow = q0 + 32 * w + r32;
  const int wq_lo = q0 + 32 * w, wq_hi = wq_lo + 31;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;

  float qf[NC], dof[NC];
  {
    const int qr = min(qrow, Lq - 1);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qf[c] = Q[qbase + (int64_t)qr * D + 2 * c + g];
      dof[c] = dO[qbase + (int64_t)qr * D + 2 * c + g];
    }
  }
  const float lse2 = qrow < Lq ? LSE[(int64_t)bh * Lq + qrow] * kLog2e : INFINITY;
  const float dl = qrow < Lq ? Delta[(int64_t)bh * Lq + qrow] : 0.f;
  f32x16 adq[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) adq[dt] = f32x16{};

  float4 kreg[LPT], vreg[LPT];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + 256 * i;
      const int row = min(kb + c / CPR, Lk - 1), ch = c % CPR;
      kreg[i] = *reinterpret_cast<const float4*>(K + kbase + (int64_t)row * D + 4 * ch);
      vreg[i] = *reinterpret_cast<const float4*>(V + kbase + (int64_t)row * D + 4 * ch);
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + 256 * i;
      const int row = c / CPR, ch = c % CPR;
      float* pk = &sK[row * P + 4 * ch];
      float* pv = &sV[row * P + 4 * ch];
      pk[0] = kreg[i].x; pk[1] = kreg[i].y; pk[2] = kreg[i].z; pk[3] = kreg[i].w;
      pv[0] = vreg[i].x; pv[1] = vreg[i].y; pv[2] = vreg[i].z; pv[3] = vreg[i].w;
    }
  };

  const int kend = CAUSAL ? min(Lk, q0 + BM) : Lk;
  if (kend > 0) gload(0);
  for (int kb = 0; kb < kend; kb += BN) {
    __syncthreads();
    sstore();
    __syncthreads();
    if (kb + BN < kend) gload(kb + BN);
    if (CAUSAL && kb > wq_hi) continue;
    const bool need_mask = (kb + BN > Lk) || (CAUSAL && kb + BN - 1 > wq_lo);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        s = mfma_f32_32x32x2(sK[(32 * t + r32) * P + 2 * c + g], qf[c], s);
        dp = mfma_f32_32x32x2(sV[(32 * t + r32) * P + 2 * c + g], dof[c], dp);
      }
      float dsr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], sl2, -lse2));
        if (need_mask) {
          const int kk = kb + 32 * t + acc_row(r, g);
          if (kk >= Lk || (CAUSAL && kk > qrow)) p = 0.f;
        }
        dsr[r] = p * (dp[r] - dl);
      }
#pragma unroll
      for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          adq[dt] = mfma_f32_32x32x2(sK[(32 * t + acc_row(r, g)) * P + 32 * dt + r32], dsr[r], adq[dt]);
    }
  }

  if (qrow < Lq) {
    float* row = dQ + qbase + (int64_t)qrow * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        float4 v = {adq[dt][r] * scale, adq[dt][r + 1] * scale, adq[dt][r + 2] * scale, adq[dt][r + 3] * scale};
        *reinterpret_cast<float4*>(row + 32 * dt + acc_row(r, g)) = v;
      }
  }
}

// ------------------------------------------------------------------ launchers
template <typename T, int D, bool CAUSAL>
static int launch_bwd(const T* q, const T* k, const T* v, const T* o, const float* lse, const T* dout,
                      T* dq, T* dk, T* dv, int64_t BH, int64_t Lq, int64_t Lk, float scale, hipStream_t st) {
  constexpr bool BF = sizeof(T) == 2;
  // workspace: D (row sums of dO o O) and LSE * log2(e), fp32 [B*H*Lq] each
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
  const int64_t nkt = (Lk + DKDV_BN - 1) / DKDV_BN;
  const int64_t nqt = (Lq + DQ_BM - 1) / DQ_BM;
  if (nkt * BH > 0x7fffffff || nqt * BH > 0x7fffffff) return fail(TT_ERR_ARG, "attention backward: grid too large");
  const int gk = pick_group(BH, nkt, 32), gq = pick_group(BH, nqt, 32);
  if constexpr (BF) {
    hipLaunchKernelGGL((attn_bwd_dkdv_bf16_kernel<D, CAUSAL>), dim3((unsigned)(nkt * BH)), dim3(256), 0, st,
                       q, k, v, dout, l2, delta, dk, dv, (int)Lq, (int)Lk, (int)BH, (int)nkt, gk, sl2, scale);
    TT_LAUNCHED("attention backward dK/dV launch", st);
    hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<D, CAUSAL>), dim3((unsigned)(nqt * BH)), dim3(256), 0, st,
                       q, k, v, dout, l2, delta, dq, (int)Lq, (int)Lk, (int)BH, (int)nqt, gq, sl2, scale);
    TT_LAUNCHED("attention backward dQ launch", st);
  } else {
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
