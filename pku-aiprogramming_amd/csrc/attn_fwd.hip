// Fused attention forward for gfx950:  O = softmax(s Q K^T + M) V, LSE.
//
// Replaces the reference's op chain Q @ K^T -> * s -> + mask -> softmax -> @ V
// (optimizer/operators.py:163-164, 234-239, 194-196, 611-612, 416-419; GPU
// softmax order max -> sub -> exp -> sum -> div of src/Layers.cu:324-349)
// with one kernel that never writes the L x L score matrix.
//
// bf16 kernel (every head size): workgroup = NW wavefronts = 32*NW queries of
// one (b, h); wave w owns queries q0 + 32w .. q0 + 32w + 31, one per lane
// column.  K/V tiles of 64 keys stream through a ring of LDS buffers filled
// by direct global->LDS loads, one tile ahead of the one consumed, and the
// scores of the next tile are computed while the current one's softmax runs
// (see attn_fwd_bf16_pipe_kernel).  Per tile and wave:
//   S^T (64 keys x 32 queries) = K Q^T     (bf16 MFMA, Q held in registers)
//   online softmax in the log2 domain      (running max m, running sum l)
//   O^T (d x 32 queries) += V^T P^T        (P rounded to bf16, fp32 accum.;
//                                           V^T read by LDS transpose reads)
// The fp32 variant runs a simpler 2-stage schedule on v_mfma_f32_32x32x2f32
// with P kept in fp32, which keeps the fp32 configs inside 1e-4.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "attn_common.h"
#include "attn_tiles.h"

namespace tt {

constexpr int FWD_BN = 64;  // keys per LDS tile
constexpr int FWD_F32_BM = 128;  // queries per workgroup of the fp32 kernel

// ---------------------------------------------------------------------------
// Software-pipelined bf16 forward (D = 32, 64, 128).
//
// Workgroup = NW waves x 32 queries (lane l: query wq0 + l % 32), two
// workgroups per CU (two waves per SIMD).  Key tiles of 64; iteration j:
//   phase 1  MFMA  S_{j+1} = K_{j+1} Q^T
//            VALU  P_j = 2^(s S_j - m), P_j -> bf16
//   phase 2  MFMA  O^T += V_j^T P_j^T
//            VALU  l += sum P_j; running max from S_{j+1} (lazy, branch-free)
// so the softmax of one tile runs on the VALU while the matrix cores compute
// the next tile's scores (__builtin_amdgcn_sched_group_barrier interleaves
// the two instruction streams), and the other wave of the SIMD fills what is
// left.  The K ring runs one tile ahead of the V ring: pair n = (K_{n+1},
// V_n) is waited for at barrier n (before iteration n) and pair n + 1 is
// issued right after it into the buffers of K_n and V_{n-1}, which
// iterations up to n - 1 have finished with.
// 4-wave workgroups, two per CU (8-wave workgroups measured 6 % slower).
// The compiler's scheduler interleaves the VALU and MFMA work of the loop
// body (an explicit sched_group_barrier pattern measured 3 % slower).
constexpr int FWDP_NW = 4;

template <int D, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_fwd_bf16_pipe_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    u16* __restrict__ O, float* __restrict__ LSE, int Lq, int Lk, int BH, int nqt, int order,
    float sl2) {
  using Tile = SwzTile<D>;
  constexpr int BM = 32 * NW, BN = 64;
  constexpr int NC = D / 16, ND = D / 32;
  constexpr int TE = Tile::kElems(BN);
  using Dma = TileDma<D, BN, NW>;
  __shared__ __align__(16) u16 sK[2 * TE];
  __shared__ __align__(16) u16 sV[2 * TE];

  // the wave index is wave-uniform: loop bounds derived from it stay scalar
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, g = l >> 5, r32 = l & 31;
  int qt, bh;
  map_tile(blockIdx.x, nqt, BH, order, qt, bh, CAUSAL);
  const int q0 = qt * BM, wq0 = q0 + 32 * w, qrow = wq0 + r32;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;

  bf16x8 qf[NC];
  {
    const int qr = min(qrow, Lq - 1);  // padding rows read a valid row; never written back
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qf[c] = __builtin_bit_cast(bf16x8, ldg16(Q + qbase + (int64_t)qr * D + 16 * c + 8 * g));
  }

  const int kend = CAUSAL ? min(Lk, q0 + BM) : Lk;  // >= 1: Lk >= 1, and q0 < Lq = Lk when causal
  const int ntiles = (kend + BN - 1) / BN;
  // Last tile this wave computes: its diagonal tile (causal) or the last
  // tile.  Every earlier tile lies inside Lk and before every query of the
  // wave, so only the last one can need a mask.
  const int last = CAUSAL ? min(wq0 / BN, ntiles - 1) : ntiles - 1;
  const bool mask_last = CAUSAL || (Lk % BN) != 0;

  // Per-lane LDS element offsets.  K operand of chunk c: key row r32 (+32
  // for the second key half), 16-byte chunk 2c + g.  V^T operand of d-tile
  // dt: transpose reads of rows vrow and vrow + 8 (+16 per key chunk),
  // column 32 dt + vcol.  Rows 16 apart share a swizzle, so the key-half and
  // key-chunk steps are constant offsets.
  int kidx[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) kidx[c] = Tile::chunk(r32, 2 * c + g);
  const int t16 = l & 15;
  const int vcol = 16 * ((l >> 4) & 1) + 4 * (t16 & 3);
  const int vrow = 4 * g + (t16 >> 2);
  int vidx[2][ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) {
    vidx[0][dt] = Tile::at4(vrow, 32 * dt + vcol);
    vidx[1][dt] = Tile::at4(vrow + 8, 32 * dt + vcol);
  }

  f32x16 o[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) o[dt] = f32x16{};
  f32x16 sa[2], sb[2];  // S^T of two consecutive tiles (key half t = 0, 1)
  bf16x8 pb[4];         // P^T operands (16-key chunk)
  float m, lsum = 0.f, alpha = 1.f;
  bool rescale = false;

  // `load(c)` runs after the MFMAs of chunk c; the pipelined loop issues
  // one tile-load instruction of the next pair there (K, then V).
  constexpr int kLoads = Dma::kLoads;
  static_assert(2 * kLoads <= NC, "a K and a V tile load per chunk of the contraction");
  auto qk = [&](const u16* tK, f32x16(&s)[2], auto load) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(&tK[kidx[c]]);
      const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(&tK[kidx[c] + 32 * D]);
      s[0] = mfma_bf16_32x32x16(k0, qf[c], c == 0 ? f32x16{} : s[0]);
      s[1] = mfma_bf16_32x32x16(k1, qf[c], c == 0 ? f32x16{} : s[1]);
      load(c);
    }
  };
  auto no_load = [](int) {};
  auto mask_tile = [&](f32x16(&s)[2], int kb) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb + 32 * t + acc_row(r, g);
        if (key >= Lk || (CAUSAL && key > qrow)) s[t][r] = -INFINITY;
      }
  };
  // Running max per query, in the log2 domain.  It moves only when some
  // lane's tile max exceeds it by more than 8, so p = 2^(x - m) <= 256 and
  // the O rescale is skipped on most tiles; the result is exact either way
  // (numerator and denominator share m).  Returns whether O must be
  // rescaled by alpha before the next PV.
  auto row_max = [&](const f32x16(&s)[2], bool first) {
    // four independent v_max3 chains over the 32 scores of this lane
    float x[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      x[c] = vmax(s[c >> 1][8 * (c & 1)], s[c >> 1][8 * (c & 1) + 1]);
#pragma unroll
      for (int r = 2; r < 8; r += 2) x[c] = vmax3(x[c], s[c >> 1][8 * (c & 1) + r], s[c >> 1][8 * (c & 1) + r + 1]);
    }
    const float mx = max_xor32(vmax(vmax3(x[0], x[1], x[2]), x[3])) * sl2;
    if (first) {
      m = mx;
      return false;
    }
    const bool need = wave_any(mx > m + 8.f);
    const float mn = need ? vmax(m, mx) : m;
    alpha = fast_exp2(m - mn);  // exactly 1 when m is unchanged; 0 when m was -inf
    m = mn;
    lsum *= alpha;
    return need;
  };
  // p = 2^(s sl2 - m) in place, and the bf16 P^T operands
  auto exp_cvt = [&](f32x16(&s)[2]) {
    const float mb = m == -INFINITY ? 0.f : m;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[t][r] = fast_exp2(fmaf(s[t][r], sl2, -mb));
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[kc][e] = (__bf16)s[kc >> 1][8 * (kc & 1) + e];
  };
  // Row sum of the bf16-rounded P, the weights the PV MFMAs apply:
  // v_dot2_f32_bf16 against (1, 1) adds two of them per instruction.
  auto add_sum = [&]() {
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int e = 0; e < 4; ++e) ps[e] = sum_bf16x2(pb[kc], e, ps[e]);
    lsum += (ps[0] + ps[1]) + (ps[2] + ps[3]);
  };
  auto pv = [&](const u16* tV) {
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const bf16x8 v = lds_read_tr16x2(&tV[vidx[0][dt] + 16 * D * kc], &tV[vidx[1][dt] + 16 * D * kc]);
        o[dt] = mfma_bf16_32x32x16(v, pb[kc], o[dt]);
      }
  };
  auto rescale_o = [&]() {
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o[dt] *= alpha;
  };

  Dma dma;
  dma.init();
  auto issue_k = [&](int n) {
    if (n < ntiles) dma.issue(K + kbase, BN * n, Lk, sK + (n & 1) * TE);
  };
  auto issue_v = [&](int n) {
    if (n < ntiles) dma.issue(V + kbase, BN * n, Lk, sV + (n & 1) * TE);
  };
  auto step = [&](int n) {
    wait_vmem_le<0>();
    __syncthreads();
    issue_k(n + 2);
    issue_v(n + 1);
  };

  // Iteration j: barrier j, S_{j+1} from K_{j+1} into `nx` while the
  // softmax of `cur` (tile j) runs, then PV of tile j and the max of tile j + 1.
  // PAR = j & 1 when known at compile time (the buffers' LDS offsets then
  // fold into the read instructions), -1 otherwise.  SPREAD: the pair this
  // iteration loads (K_{j+2}, V_{j+1}) exists and lies inside Lk, and its
  // load instructions are spread over the phase-1 MFMAs (early enough to land
  // by the next barrier) instead of issued back to back after the barrier.
  auto body = [&](int j, f32x16(&cur)[2], f32x16(&nx)[2], auto mask_tag, auto par_tag, auto spread_tag) {
    constexpr bool MASK = decltype(mask_tag)::value;
    constexpr int PAR = decltype(par_tag)::value;
    constexpr bool SPREAD = decltype(spread_tag)::value;
    static_assert(!SPREAD || PAR >= 0, "spread loads need the ring parity");
    const int kbuf = PAR < 0 ? ((j + 1) & 1) : 1 - PAR, vbuf = PAR < 0 ? (j & 1) : PAR;
    auto load_kv = [&](int c) {
      if (c < kLoads)
        dma.issue_one(K + kbase, BN * (j + 2), sK + PAR * TE, c);
      else if (c < 2 * kLoads)
        dma.issue_one(V + kbase, BN * (j + 1), sV + (1 - PAR) * TE, c - kLoads);
    };
    if constexpr (SPREAD) {
      wait_vmem_le<0>();
      __syncthreads();
    } else {
      step(j);
    }
    // the rare O rescale goes first, so that both phases form one basic
    // block for the scheduler
    if (rescale) rescale_o();
    // LLVM's MFMA / transcendental interleave strategy for this block: one
    // v_exp_f32 between consecutive MFMAs (2.5 % fewer cycles at d = 128)
    __builtin_amdgcn_iglp_opt(3);
    if constexpr (SPREAD)
      qk(sK + kbuf * TE, nx, load_kv);
    else
      qk(sK + kbuf * TE, nx, no_load);
    exp_cvt(cur);
    pv(sV + vbuf * TE);
    add_sum();
    if constexpr (MASK) mask_tile(nx, BN * (j + 1));
    rescale = row_max(nx, false);
  };

  // Prologue: K_0, then pair 0 (K_1, V_0); S_0 once K_0 has landed.
  issue_k(0);
  issue_k(1);
  issue_v(0);
  if (ntiles > 1)
    wait_vmem_le<2 * Dma::kLoads>();
  else
    wait_vmem_le<Dma::kLoads>();
  __syncthreads();
  qk(sK, sa, no_load);
  if (last == 0 && mask_last) mask_tile(sa, 0);
  row_max(sa, true);

  // Unmasked iterations 0 .. last - 2 in pairs (the score tiles swap roles),
  // then iteration last - 1, whose next tile is the wave's last one.
  using Even = std::integral_constant<int, 0>;
  using Odd = std::integral_constant<int, 1>;
  using Any = std::integral_constant<int, -1>;
  // In the pair loop (j + 1 < last - 1) the pairs loaded, up to K_{last},
  // all exist; they lie inside Lk when the workgroup's key range ends on a
  // tile boundary.
  int j = 0;
  if (kend % BN == 0) {
    for (; j + 1 < last - 1; j += 2) {
      body(j, sa, sb, std::false_type{}, Even{}, std::true_type{});
      body(j + 1, sb, sa, std::false_type{}, Odd{}, std::true_type{});
    }
  } else {
    for (; j + 1 < last - 1; j += 2) {
      body(j, sa, sb, std::false_type{}, Even{}, std::false_type{});
      body(j + 1, sb, sa, std::false_type{}, Odd{}, std::false_type{});
    }
  }
  if (j < last - 1) {
    body(j, sa, sb, std::false_type{}, Any{}, std::false_type{});
    sa[0] = sb[0];
    sa[1] = sb[1];
    ++j;
  }
  if (last >= 1) {
    // always the masking body: a second copy for unmasked last tiles made the
    // non-causal d = 128 kernel spill a Q fragment inside its main loop
    body(j, sa, sb, std::true_type{}, Any{}, std::false_type{});
    sa[0] = sb[0];
    sa[1] = sb[1];
  }
  // Last tile of this wave: softmax and PV only.
  step(last);
  if (rescale) rescale_o();
  exp_cvt(sa);
  pv(sV + (last & 1) * TE);
  add_sum();
  // Later tiles belong to other waves of the workgroup: take part in their
  // barriers and loads.
  for (int n = last + 1; n < ntiles; ++n) step(n);
  wait_vmem_le<0>();  // nothing may be in flight into LDS when the workgroup exits

  const float ls = sum_xor32(lsum);
  const float inv = ls > 0.f ? 1.f / ls : 0.f;
  if (qrow < Lq && g == 0 && LSE) LSE[(int64_t)bh * Lq + qrow] = (m + __log2f(ls)) * kLn2;
  if constexpr (D >= 128) {
    // O through LDS (the K ring is free once every wave has passed its last
    // wait; 128 rows of D bf16 fit the two K buffers): c5 -0.5 %; at d = 64
    // the two extra barriers cost more than the 8-byte stores (+1.7 % at c3)
    static_assert(2 * TE >= BM * D, "the K ring holds the workgroup's O rows");
    __syncthreads();
    stage_rows_bf16<D, ND>(sK, 32 * w + r32, g, o, inv);
    __syncthreads();
    store_staged_rows<D>(sK, BM, O + qbase, q0, Lq, 64 * NW);
  } else if (qrow < Lq) {
    u16* orow = O + qbase + (int64_t)qrow * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        uint2 v;
        v.x = pack_bf16x2(o[dt][r] * inv, o[dt][r + 1] * inv);
        v.y = pack_bf16x2(o[dt][r + 2] * inv, o[dt][r + 3] * inv);
        *reinterpret_cast<uint2*>(orow + 32 * dt + acc_row(r, g)) = v;
      }
  }
}

// fp32 forward.  With nsplit > 1 the key range of each query tile is split
// over nsplit workgroups (workgroup id = split * nqt * BH + tile id), each
// writing its unnormalised O, running max and row sum to `part`; the combine
// kernel below merges them.  Small problems (B = H = 8, L = 256: 128 query
// tiles) then still put a workgroup on every CU.
template <int D, bool CAUSAL>
__global__ __launch_bounds__(256, (D >= 128 ? 1 : 2)) void attn_fwd_f32_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    float* __restrict__ O, float* __restrict__ LSE, int Lq, int Lk, int BH, int nqt, int order,
    float sl2, int nsplit, float* __restrict__ part) {
  constexpr int BM = FWD_F32_BM, BN = FWD_BN;
  constexpr int NC = D / 2;   // k-steps of the d contraction (2 per MFMA)
  constexpr int ND = D / 32;
  constexpr int CPR = D / 4;  // 16-byte chunks per row
  constexpr int LPT = BN * CPR / 256;
  // MFMA step c contracts d-indices c (lane half 0) and D/2 + c (lane half 1):
  // a lane's Q values and K operands are then D/2 consecutive floats, read
  // 16 bytes at a time (one K read feeds four MFMAs).  V is stored
  // transposed, sV[d][key], so that the four keys of four consecutive
  // accumulator rows are adjacent.  Row pitches of 4 mod 64 floats put the 16
  // rows of a 16-lane read pass on distinct banks.
  constexpr int PK = D + 4, PV = BN + 4;
  __shared__ __align__(16) float sK[BN * PK];
  __shared__ __align__(16) float sV[D * PV];

  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, g = l >> 5, r32 = l & 31;
  const int ntq = nqt * BH;
  const int split = blockIdx.x / ntq;
  int qt, bh;
  map_tile(blockIdx.x - split * ntq, nqt, BH, order, qt, bh, CAUSAL);
  const int q0 = qt * BM;
  const int qrow = q0 + 32 * w + r32;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;

  float qf[NC];
  {
    const int qr = min(qrow, Lq - 1);
    const float* qp = Q + qbase + (int64_t)qr * D + g * (D / 2);
#pragma unroll
    for (int c4 = 0; c4 < NC / 4; ++c4) {
      const float4 x = *reinterpret_cast<const float4*>(qp + 4 * c4);
      qf[4 * c4] = x.x;
      qf[4 * c4 + 1] = x.y;
      qf[4 * c4 + 2] = x.z;
      qf[4 * c4 + 3] = x.w;
    }
  }

  f32x16 acc[ND];
#pragma unroll
  for (int dt = 0; dt < ND; ++dt) acc[dt] = f32x16{};
  float m = -INFINITY, lsum = 0.f;
  // this workgroup's key tiles: [kb_lo, kb_hi) of [0, kend), split `split`
  // of nsplit equal runs of whole tiles (a run may be empty)
  const int kend = CAUSAL ? min(Lk, q0 + BM) : Lk;
  const int per = ((kend + BN - 1) / BN + nsplit - 1) / nsplit * BN;
  const int kb_lo = min(kend, split * per), kb_hi = min(kend, kb_lo + per);
  const int wq_lo = q0 + 32 * w, wq_hi = wq_lo + 31;

  // The staged tile rows are native 4-float vectors: copies of the float4
  // struct kept this array in scratch memory (a private-memory round trip per
  // tile) instead of registers.
  f32x4 kreg[LPT], vreg[LPT];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + 256 * i;
      const int row = min(kb + c / CPR, Lk - 1), ch = c % CPR;  // rows past Lk are masked
      kreg[i] = *reinterpret_cast<const f32x4*>(K + kbase + (int64_t)row * D + 4 * ch);
      vreg[i] = *reinterpret_cast<const f32x4*>(V + kbase + (int64_t)row * D + 4 * ch);
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int c = tid + 256 * i;
      const int key = c / CPR, ch = c % CPR;  // d-indices 4ch .. 4ch + 3
      *reinterpret_cast<f32x4*>(&sK[key * PK + 4 * ch]) = kreg[i];
      float* pv = &sV[4 * ch * PV + key];
      pv[0] = vreg[i].x;
      pv[PV] = vreg[i].y;
      pv[2 * PV] = vreg[i].z;
      pv[3 * PV] = vreg[i].w;
    }
  };

  if (kb_lo < kb_hi) gload(kb_lo);
  for (int kb = kb_lo; kb < kb_hi; kb += BN) {
    __syncthreads();
    sstore();
    __syncthreads();
    if (kb + BN < kb_hi) gload(kb + BN);
    if (CAUSAL && kb > wq_hi) continue;

    f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x16{};
      const float* kr = &sK[(32 * t + r32) * PK + g * (D / 2)];
#pragma unroll
      for (int c4 = 0; c4 < NC / 4; ++c4) {
        const float4 kk = *reinterpret_cast<const float4*>(kr + 4 * c4);
        s[t] = mfma_f32_32x32x2(kk.x, qf[4 * c4], s[t]);
        s[t] = mfma_f32_32x32x2(kk.y, qf[4 * c4 + 1], s[t]);
        s[t] = mfma_f32_32x32x2(kk.z, qf[4 * c4 + 2], s[t]);
        s[t] = mfma_f32_32x32x2(kk.w, qf[4 * c4 + 3], s[t]);
      }
    }
    const bool need_mask = (kb + BN > Lk) || (CAUSAL && kb + BN - 1 > wq_lo);
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x = s[t][r] * sl2;
        if (need_mask) {
          const int key = kb + 32 * t + acc_row(r, g);
          if (key >= Lk || (CAUSAL && key > qrow)) x = -INFINITY;
        }
        s[t][r] = x;
        mx = vmax(mx, x);
      }
    mx = vmax(mx, wave_xor32(mx));
    const float mnew = vmax(m, mx);
    const float mb = (mnew == -INFINITY) ? 0.f : mnew;
    const float alpha = fast_exp2(m - mb);
    m = mnew;
    float ps = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(s[t][r] - mb);
        s[t][r] = p;
        ps += p;
      }
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) acc[dt] *= alpha;
    // O^T += V^T P^T, two keys (one per lane half) per MFMA: accumulator
    // rows 4j .. 4j + 3 of lane half g are keys 32t + 8j + 4g + 0..3, one
    // 16-byte read of the transposed V tile.
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 vv = *reinterpret_cast<const float4*>(&sV[(32 * dt + r32) * PV + 32 * t + 8 * j + 4 * g]);
          acc[dt] = mfma_f32_32x32x2(vv.x, s[t][4 * j], acc[dt]);
          acc[dt] = mfma_f32_32x32x2(vv.y, s[t][4 * j + 1], acc[dt]);
          acc[dt] = mfma_f32_32x32x2(vv.z, s[t][4 * j + 2], acc[dt]);
          acc[dt] = mfma_f32_32x32x2(vv.w, s[t][4 * j + 3], acc[dt]);
        }
  }

  lsum += wave_xor32(lsum);
  if (qrow < Lq) {
    const int64_t row = (int64_t)bh * Lq + qrow;
    const float inv = nsplit > 1 ? 1.f : (lsum > 0.f ? 1.f / lsum : 0.f);
    float* orow = nsplit > 1 ? part + ((int64_t)split * BH * Lq + row) * D : O + qbase + (int64_t)qrow * D;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        float4 v = {acc[dt][r] * inv, acc[dt][r + 1] * inv, acc[dt][r + 2] * inv, acc[dt][r + 3] * inv};
        *reinterpret_cast<float4*>(orow + 32 * dt + acc_row(r, g)) = v;
      }
    if (g == 0) {
      if (nsplit > 1) {
        float* ml = part + (int64_t)nsplit * BH * Lq * D + 2 * ((int64_t)split * BH * Lq + row);
        ml[0] = m;
        ml[1] = lsum;
      } else if (LSE) {
        LSE[row] = (m + __log2f(lsum)) * kLn2;
      }
    }
  }
}

// Merges the nsplit partial results of the split fp32 forward: per query
// row, with M = max of the splits' running maxima, O = sum_s 2^(m_s - M) O_s /
// sum_s 2^(m_s - M) l_s and LSE = (M + log2 of that denominator) ln 2.  A split
// with no keys for the row has m_s = -inf and weight 0; split 0 always holds
// key 0, which every query sees.  D / 4 threads per row, one float4 each.
template <int D>
__global__ __launch_bounds__(256) void attn_fwd_f32_combine_kernel(const float* __restrict__ part,
                                                                   float* __restrict__ O, float* __restrict__ LSE,
                                                                   int64_t rows, int nsplit) {
  constexpr int TPR = D / 4;
  const int64_t row = (int64_t)blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int c = threadIdx.x % TPR;
  if (row >= rows) return;
  const float* ml = part + (int64_t)nsplit * rows * D;
  float mx = -INFINITY;
  for (int sp = 0; sp < nsplit; ++sp) mx = fmaxf(mx, ml[2 * (sp * rows + row)]);
  float den = 0.f;
  float4 num = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < nsplit; ++sp) {
    const int64_t pr = sp * rows + row;
    const float wgt = fast_exp2(ml[2 * pr] - mx);  // 0 for an empty split (m = -inf)
    den += wgt * ml[2 * pr + 1];
    const float4 o = *reinterpret_cast<const float4*>(part + pr * D + 4 * c);
    num.x += wgt * o.x;
    num.y += wgt * o.y;
    num.z += wgt * o.z;
    num.w += wgt * o.w;
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  *reinterpret_cast<float4*>(O + row * D + 4 * c) = float4{num.x * inv, num.y * inv, num.z * inv, num.w * inv};
  if (c == 0 && LSE) LSE[row] = (mx + __log2f(den)) * kLn2;
}

template <typename T, typename KernelPtr>
static int launch_fwd(KernelPtr kern, int bm, int threads, int wg_per_cu, int light_div, const T* q, const T* k,
                      const T* v, T* o, float* lse, int64_t BH, int64_t Lq, int64_t Lk, float scale, hipStream_t s) {
  const int64_t nqt = (Lq + bm - 1) / bm;
  const int64_t nblk = nqt * BH;
  if (!grid_fits(nblk, threads)) return fail(TT_ERR_ARG, "attention forward: grid too large");
  // heads in flight per XCD: enough tiles for the resident workgroups of its
  // 32 CUs
  const int order = tile_order(BH, nqt, 32 * wg_per_cu, light_div);
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(threads), 0, s, q, k, v, o, lse, (int)Lq, (int)Lk,
                     (int)BH, (int)nqt, order, scale * kLog2e);
  TT_LAUNCHED("attention forward launch", s);
  return ok();
}

template <int D, bool CAUSAL>
static int fwd_bf16(const u16* q, const u16* k, const u16* v, u16* o, float* lse, int64_t BH, int64_t Lq,
                    int64_t Lk, float scale, hipStream_t st) {
  // two waves per SIMD: two FWDP_NW-wave workgroups per CU (at d = 32 this
  // kernel measured 5-10 % faster than the simpler two-stage kernel it
  // replaced there, non-causal and at L = 4096, and the same at
  // [16,16,1024,32] causal)
  constexpr int NW = FWDP_NW;
  return launch_fwd(attn_fwd_bf16_pipe_kernel<D, CAUSAL, NW>, 32 * NW, 64 * NW, 8 / NW,
                    attention_light_div(CAUSAL, D), q, k, v, o, lse, BH, Lq, Lk, scale, st);
}

template <int D, bool CAUSAL>
static int fwd_f32(const float* q, const float* k, const float* v, float* o, float* lse, int64_t BH, int64_t Lq,
                   int64_t Lk, float scale, hipStream_t st) {
  constexpr int wg_per_cu = D >= 128 ? 1 : 2;
  const int64_t nqt = (Lq + FWD_F32_BM - 1) / FWD_F32_BM;
  const int64_t ntq = nqt * BH;
  // Split the keys when the query tiles alone leave CUs idle: up to 4 splits,
  // each with at least one key tile.
  const int64_t slots = 256 * wg_per_cu, ktiles = (Lk + FWD_BN - 1) / FWD_BN;
  int64_t nsplit = ntq >= slots ? 1 : (slots + ntq - 1) / ntq;
  if (nsplit > 4) nsplit = 4;
  if (nsplit > ktiles) nsplit = ktiles;
  if (nsplit < 1) nsplit = 1;
  if (!grid_fits(ntq * nsplit, 256)) return fail(TT_ERR_ARG, "attention forward: grid too large");
  const int order = tile_order(BH, nqt, 32 * wg_per_cu, attention_light_div(CAUSAL, D));
  const float sl2 = scale * kLog2e;
  if (nsplit == 1) {
    hipLaunchKernelGGL((attn_fwd_f32_kernel<D, CAUSAL>), dim3((unsigned)ntq), dim3(256), 0, st, q, k, v, o, lse,
                       (int)Lq, (int)Lk, (int)BH, (int)nqt, order, sl2, 1, nullptr);
    TT_LAUNCHED("attention forward launch", st);
    return ok();
  }
  const int64_t rows = BH * Lq;
  void* ws = nullptr;
  WorkspaceLease lease;  // held until both kernels are launched
  int rc = lease.get(st, kWsForwardSplits, (size_t)(nsplit * rows) * (D + 2) * sizeof(float), &ws);
  if (rc) return rc;
  float* part = (float*)ws;
  hipLaunchKernelGGL((attn_fwd_f32_kernel<D, CAUSAL>), dim3((unsigned)(ntq * nsplit)), dim3(256), 0, st, q, k, v,
                     o, lse, (int)Lq, (int)Lk, (int)BH, (int)nqt, order, sl2, (int)nsplit, part);
  TT_LAUNCHED("attention forward split launch", st);
  constexpr int RPB = 256 / (D / 4);  // rows per combine workgroup
  hipLaunchKernelGGL((attn_fwd_f32_combine_kernel<D>), dim3((unsigned)((rows + RPB - 1) / RPB)), dim3(256), 0, st,
                     (const float*)part, o, lse, rows, (int)nsplit);
  TT_LAUNCHED("attention forward combine launch", st);
  return ok();
}

}  // namespace tt

using namespace tt;

#define TT_FWD_DISPATCH(FN)                                                  \
  switch (d * 2 + (causal ? 1 : 0)) {                                        \
    case 64: return FN<32, false>(q, k, v, o, lse, BH, Lq, Lk, scale, st);   \
    case 65: return FN<32, true>(q, k, v, o, lse, BH, Lq, Lk, scale, st);    \
    case 128: return FN<64, false>(q, k, v, o, lse, BH, Lq, Lk, scale, st);  \
    case 129: return FN<64, true>(q, k, v, o, lse, BH, Lq, Lk, scale, st);   \
    case 256: return FN<128, false>(q, k, v, o, lse, BH, Lq, Lk, scale, st); \
    case 257: return FN<128, true>(q, k, v, o, lse, BH, Lq, Lk, scale, st);  \
    default: return fail(TT_ERR_UNSUPPORTED, "attention forward: unsupported head dim"); \
  }

extern "C" int tt_attn_fwd_f32(const float* q, const float* k, const float* v, float* o, float* lse,
                               int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d, float scale,
                               int causal, void* stream) {
  int rc = check_attn_shape("tt_attn_fwd_f32", B, H, Lq, Lk, d, causal);
  if (rc) return rc;
  const int64_t BH = B * H;
  if (BH == 0 || Lq == 0) return ok();
  if (!q || !k || !v || !o) return fail(TT_ERR_ARG, "tt_attn_fwd_f32: null pointer");
  {
    const size_t qb = (size_t)(BH * Lq * d) * sizeof(float), kb = (size_t)(BH * Lk * d) * sizeof(float);
    if ((rc = check_no_overlap("tt_attn_fwd_f32", {{q, qb, "q"}, {k, kb, "k"}, {v, kb, "v"}},
                               {{o, qb, "o"}, {lse, (size_t)(BH * Lq) * sizeof(float), "lse"}})))
      return rc;
  }
  if ((rc = ensure_init())) return rc;
  hipStream_t st = stream_or_default(stream);
  TT_FWD_DISPATCH(fwd_f32)
}

extern "C" int tt_attn_fwd_bf16(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                                float* lse, int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t d,
                                float scale, int causal, void* stream) {
  int rc = check_attn_shape("tt_attn_fwd_bf16", B, H, Lq, Lk, d, causal);
  if (rc) return rc;
  const int64_t BH = B * H;
  if (BH == 0 || Lq == 0) return ok();
  if (!q || !k || !v || !o) return fail(TT_ERR_ARG, "tt_attn_fwd_bf16: null pointer");
  {
    const size_t qb = (size_t)(BH * Lq * d) * sizeof(uint16_t), kb = (size_t)(BH * Lk * d) * sizeof(uint16_t);
    if ((rc = check_no_overlap("tt_attn_fwd_bf16", {{q, qb, "q"}, {k, kb, "k"}, {v, kb, "v"}},
                               {{o, qb, "o"}, {lse, (size_t)(BH * Lq) * sizeof(float), "lse"}})))
      return rc;
  }
  if ((rc = ensure_init())) return rc;
  hipStream_t st = stream_or_default(stream);
  TT_FWD_DISPATCH(fwd_bf16)
}
