// fp32 attention backward kernels (dK/dV and dQ) on v_mfma_f32_32x32x2f32,
// included by attn_bwd.hip.  Each fp32 MFMA takes one k-value per lane half,
// so the transposed operands are plain column reads of row-major LDS tiles.
// In the contractions over d, MFMA step c takes d-index c in lane half 0 and
// D/2 + c in lane half 1: a lane's row operands are D/2 consecutive floats
// (16-byte global loads), and the two lane halves read disjoint banks of the
// odd-pitch LDS tiles.
#pragma once

#include "attn_common.h"
#include "attn_tiles.h"

namespace tt {

constexpr int BWD_F32_BN = 128;  // keys per dK/dV workgroup
constexpr int BWD_F32_BM = 128;  // queries per dQ workgroup
constexpr int BWD_F32_KN = 64;   // keys per LDS step of the dQ kernel
// Queries per LDS step of the dK/dV role: 64, or 32 at d = 128, where a lane
// already holds 64 floats of its key's K row, 64 of its V row and 128
// accumulators, and the register-staged prefetch of two 64-query tiles (64
// more) made the causal kernel spill 61 VGPRs to scratch memory (232 bytes
// per lane); with 32-query tiles no scratch is used (36 VGPRs are parked in
// unused AGPRs instead).
template <int D>
constexpr int bwd_f32_bq() { return D >= 128 ? 32 : 64; }

// LDS floats of each role: Q and dO tiles plus their LSE / -D rows; K and V tiles.
template <int D>
constexpr int bwd_f32_dkdv_lds() { return 2 * bwd_f32_bq<D>() * (D + 1) + 2 * bwd_f32_bq<D>(); }
template <int D>
constexpr int bwd_f32_dq_lds() { return 2 * BWD_F32_KN * (D + 1); }

// dK / dV of the BWD_F32_BN keys of tile `id` (see map_tile), looping over
// the query tiles.
template <int D, bool CAUSAL>
__device__ __forceinline__ void bwd_f32_dkdv(int id, float* smem, const float* __restrict__ Q,
                                             const float* __restrict__ K, const float* __restrict__ V,
                                             const float* __restrict__ dO, const float* __restrict__ LSE,
                                             const float* __restrict__ NDelta, float* __restrict__ dK,
                                             float* __restrict__ dV, int Lq, int Lk, int BH, int nkt, int group,
                                             float sl2, float scale) {
  constexpr int BN = BWD_F32_BN, BQ = bwd_f32_bq<D>(), MT = BQ / 32;
  constexpr int P = D + 1;
  constexpr int NC = D / 2, ND = D / 32, CPR = D / 4;
  constexpr int LPT = BQ * CPR / 256;
  static_assert(BQ * CPR % 256 == 0 && BQ <= 256, "a query tile splits evenly over the 256 threads");
  float* sQ = smem;
  float* sdO = sQ + BQ * P;
  float* sL = sdO + BQ * P;
  float* sDl = sL + BQ;

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, r32 = l & 31;
  int kt, bh;
  map_tile(id, nkt, BH, group, kt, bh, false);
  const int k0 = kt * BN;
  const int key = k0 + 32 * w + r32;
  const int wk_lo = k0 + 32 * w;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;
  const int64_t lbase = (int64_t)bh * Lq;

  float kf[NC], vf[NC];
  {
    const int kr = min(key, Lk - 1);
    const int64_t at = kbase + (int64_t)kr * D + g * (D / 2);
#pragma unroll
    for (int c4 = 0; c4 < NC / 4; ++c4) {
      const float4 kx = *reinterpret_cast<const float4*>(K + at + 4 * c4);
      const float4 vx = *reinterpret_cast<const float4*>(V + at + 4 * c4);
      kf[4 * c4] = kx.x, kf[4 * c4 + 1] = kx.y, kf[4 * c4 + 2] = kx.z, kf[4 * c4 + 3] = kx.w;
      vf[4 * c4] = vx.x, vf[4 * c4 + 1] = vx.y, vf[4 * c4 + 2] = vx.z, vf[4 * c4 + 3] = vx.w;
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
      dreg = in ? NDelta[lbase + qb + tid] : 0.f;
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
    for (int mt = 0; mt < MT; ++mt) {
      f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        s = mfma_f32_32x32x2(sQ[(32 * mt + r32) * P + g * (D / 2) + c], kf[c], s);
        dp = mfma_f32_32x32x2(sdO[(32 * mt + r32) * P + g * (D / 2) + c], vf[c], dp);
      }
      const bool need_mask = CAUSAL && (qb + 32 * mt < wk_lo + 31);
      float pr[16], dsr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qi = 32 * mt + acc_row(r, g);
        float p = fast_exp2(fmaf(s[r], sl2, -sL[qi]));
        if (need_mask && key > qb + qi) p = 0.f;
        pr[r] = p;
        dsr[r] = p * (dp[r] + sDl[qi]);
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

// dQ of the BWD_F32_BM queries of tile `id`, looping over the key tiles.
template <int D, bool CAUSAL>
__device__ __forceinline__ void bwd_f32_dq(int id, float* smem, const float* __restrict__ Q,
                                           const float* __restrict__ K, const float* __restrict__ V,
                                           const float* __restrict__ dO, const float* __restrict__ LSE,
                                           const float* __restrict__ NDelta, float* __restrict__ dQ, int Lq,
                                           int Lk, int BH, int nqt, int group, float sl2, float scale) {
  constexpr int BM = BWD_F32_BM, BN = BWD_F32_KN;
  constexpr int P = D + 1;
  constexpr int NC = D / 2, ND = D / 32, CPR = D / 4;
  constexpr int LPT = BN * CPR / 256;
  float* sK = smem;
  float* sV = sK + BN * P;

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, r32 = l & 31;
  int qt, bh;
  map_tile(id, nqt, BH, group, qt, bh, CAUSAL);
  const int q0 = qt * BM;
  const int qrow = q0 + 32 * w + r32;
  const int wq_lo = q0 + 32 * w, wq_hi = wq_lo + 31;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;

  float qf[NC], dof[NC];
  {
    const int qr = min(qrow, Lq - 1);
    const int64_t at = qbase + (int64_t)qr * D + g * (D / 2);
#pragma unroll
    for (int c4 = 0; c4 < NC / 4; ++c4) {
      const float4 qx = *reinterpret_cast<const float4*>(Q + at + 4 * c4);
      const float4 ox = *reinterpret_cast<const float4*>(dO + at + 4 * c4);
      qf[4 * c4] = qx.x, qf[4 * c4 + 1] = qx.y, qf[4 * c4 + 2] = qx.z, qf[4 * c4 + 3] = qx.w;
      dof[4 * c4] = ox.x, dof[4 * c4 + 1] = ox.y, dof[4 * c4 + 2] = ox.z, dof[4 * c4 + 3] = ox.w;
    }
  }
  const float lse2 = qrow < Lq ? LSE[(int64_t)bh * Lq + qrow] * kLog2e : INFINITY;
  const float ndl = qrow < Lq ? NDelta[(int64_t)bh * Lq + qrow] : 0.f;
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
        s = mfma_f32_32x32x2(sK[(32 * t + r32) * P + g * (D / 2) + c], qf[c], s);
        dp = mfma_f32_32x32x2(sV[(32 * t + r32) * P + g * (D / 2) + c], dof[c], dp);
      }
      float dsr[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = fast_exp2(fmaf(s[r], sl2, -lse2));
        if (need_mask) {
          const int kk = kb + 32 * t + acc_row(r, g);
          if (kk >= Lk || (CAUSAL && kk > qrow)) p = 0.f;
        }
        dsr[r] = p * (dp[r] + ndl);
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

// Both roles in one launch: workgroups [0, nkblk) compute dK / dV, the rest
// dQ.  Each role alone puts one workgroup per key or query tile on the chip
// (one wave per SIMD at these register counts), so a small problem fills
// only part of the CUs with either; together they fill twice as many.
// nkblk is nkt * BH, a multiple of 8 when BH is, so the dQ workgroups keep
// their XCD mapping.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, 1) void attn_bwd_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ NDelta,
    float* __restrict__ dQ, float* __restrict__ dK, float* __restrict__ dV, int Lq, int Lk, int BH, int nkt,
    int nqt, int nkblk, int gk, int gq, float sl2, float scale) {
  constexpr int kLds = bwd_f32_dkdv_lds<D>() > bwd_f32_dq_lds<D>() ? bwd_f32_dkdv_lds<D>() : bwd_f32_dq_lds<D>();
  __shared__ float smem[kLds];
  const int id = blockIdx.x;
  if (id < nkblk)
    bwd_f32_dkdv<D, CAUSAL>(id, smem, Q, K, V, dO, LSE, NDelta, dK, dV, Lq, Lk, BH, nkt, gk, sl2, scale);
  else
    bwd_f32_dq<D, CAUSAL>(id - nkblk, smem, Q, K, V, dO, LSE, NDelta, dQ, Lq, Lk, BH, nqt, gq, sl2, scale);
}

}  // namespace tt
