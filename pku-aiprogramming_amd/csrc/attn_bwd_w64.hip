// bf16 attention dK / dV at d = 128, one wave per SIMD, 64 keys per wave.
//
// Part of the backward of the reference's attention composition (gradient
// rules MatMul, optimizer/operators.py:421-429, EWiseDiv :296-298 and Exp
// :469-470 through autodiff.py:33-61): for the keys of a workgroup,
//   P  = 2^(s log2(e) Q K^T - LSE log2(e)),  dP = dO V^T
//   dV = P^T dO,  dK = s (P o (dP - D))^T Q
// with P recomputed from the forward's LSE (no L x L tensor is stored) and
// the rows -D and LSE log2(e) written by the dQ kernel, which runs first.
//
// Workgroup = 4 waves, one per SIMD (one workgroup per CU), 256 keys.  Wave w
// owns two halves of 32 keys (lane = key) at k0 + 32 w and k0 + 128 + 32 w, so
// every Q / dO operand it reads from LDS feeds one MFMA per half: a tile of
// 32 queries costs a wave 64 MFMAs against 48 KB of operand reads from LDS
// (0.75 KB per MFMA, against 1.25 KB for a wave of 32 keys).  The dK / dV accumulators (256
// registers) live in the accumulation registers (AGPRs) of the 512-register
// file a lone wave owns; K rows, scores and operands live in the 256
// architectural VGPRs.  V rows sit in LDS; Q / dO tiles with their LSE and -D
// rows stream through a 4-deep ring filled by direct global->LDS loads.
//
// The loop is software-pipelined so that the wave's matrix core never waits
// for its own VALU work: iteration n is 64 slots of one MFMA each,
//   slots  0-15  MFMA dP_n = dO_n V^T - D      VALU P_n = 2^(S_n sl2 - LSE)   (S_n from iteration n - 1)
//   slots 16-31  MFMA dV^T += dO_n^T P_n       VALU dS_n = P_n o (dP_n - D)
//   slots 32-47  MFMA S_{n+1} = Q_{n+1} K^T    (into the registers S_n and dP_n no longer need)
//   slots 48-63  MFMA dK^T += Q_n^T dS_n       VALU half of P_{n+1}
// with every LDS read issued a few slots ahead of its MFMA and a scheduling
// barrier closing each slot.  In the causal diagonal tiles a wave skips the
// MFMAs of a key half that lies wholly after the tile's queries (in the first
// four tiles of a 256-key block every wave's second half; 5 % of the kernel's
// MFMAs at L = 4096, 1 % of its time).  Tile n is read until the end of iteration n, so
// the tile issued after barrier n + 1 (tile n + 3) goes into the buffer of
// tile n - 1: a 4-deep ring.  On the MI355X this runs at 72 % MFMA-busy
// cycles for long non-causal heads against 62 % for the two-waves-per-SIMD
// 32-key kernel; a naive (compiler-scheduled) version of the same algorithm
// ran at 38 %.
//
// The dK / dV MFMAs are written as inline asm with AGPR operands: the
// compiler otherwise gives every MFMA of a kernel with more than 256 registers
// an AGPR destination, and the scores would then need 64 more AGPRs than the
// file has.  This file is built with -mllvm -amdgpu-mfma-vgpr-form=1 so the
// builtin MFMAs (S, dP) write VGPRs.  The compiler's hazard recognizer does
// not look inside inline asm, so the asm carries its own wait states, sized by
// the CDNA4 ISA reference guide, chapter "Matrix Arithmetic Instructions",
// table "Dependency Resolution: Required Independent Instructions" (the same
// counts as LLVM's GCNHazardRecognizer for gfx950, checkMAIHazards90A and
// checkMAIVALUHazards):
//   * "VALU write VGPR -> MFMA read of that VGPR (SrcA/B/C)": 2 wait states.
//     Each asm MFMA's P / dS operand (SrcB) comes from VALU conversions, and
//     its first SrcC from the v_accvgpr_write that zeroes the accumulator:
//     the "s_nop 1" (2 wait states) in mfma_acc_agpr covers it whatever the
//     schedule; the slot schedule also keeps every such write at least one
//     MFMA slot ahead.
//   * "XDL write VGPR/AGPR -> VALU read, VMEM / LDS read or export of it":
//     passes + 3 wait states, one more on gfx950 for XDL ops of more than two
//     passes; v_mfma_f32_32x32x16_bf16 is 8 passes (32 cycles), so 11 or 12.
//     agpr_drain gives 3 x "s_nop 7" = 24 before the epilogue's first
//     v_accvgpr_read of an accumulator.
//   * "XDL write -> XDL read as SrcC of the same registers, same opcode,
//     back to back" (the dK / dV accumulation chains): no wait states.
// The operands the asm reads from LDS (SrcA) need a data wait, not a wait
// state: the compiler's s_waitcnt insertion does see inline-asm operands.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "attn_common.h"
#include "attn_tiles.h"

namespace tt {

namespace {

// acc += a b on the matrix core, acc in AGPRs.  "s_nop 1": the 2 wait states
// of the rule "VALU write VGPR -> MFMA read" (file comment).
__device__ __forceinline__ void mfma_acc_agpr(f32x16& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Keeps a value's computation in the scheduling slot that produced it (the
// compiler would otherwise sink arithmetic towards its first use).
template <typename T>
__device__ __forceinline__ void pin(T& x) {
  asm volatile("" : "+v"(x));
}

// Wait states between the last asm MFMA and the first read of its result:
// 24, against the 11 (12 on gfx950) of the rule "XDL write -> VALU read" for
// an 8-pass MFMA (file comment).
__device__ __forceinline__ void agpr_drain(f32x16 (&a)[2][4], f32x16 (&b)[2][4]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(a[0][0]), "+a"(a[0][1]), "+a"(a[0][2]), "+a"(a[0][3]), "+a"(a[1][0]), "+a"(a[1][1]),
                 "+a"(a[1][2]), "+a"(a[1][3]), "+a"(b[0][0]), "+a"(b[0][1]), "+a"(b[0][2]), "+a"(b[0][3]),
                 "+a"(b[1][0]), "+a"(b[1][1]), "+a"(b[1][2]), "+a"(b[1][3]));
}

constexpr int DKW_BN = 256, DKW_BQ = 32, DKW_STAGES = 4;
// LDS reads run this many slots ahead of their MFMA (6 and 8 measured the
// same as 4; whole dP slot pairs, so the carried operands are whole chunks).
constexpr int DKW_READ_AHEAD = 4;
static_assert(DKW_READ_AHEAD % 2 == 0 && DKW_READ_AHEAD >= 2 && DKW_READ_AHEAD <= 12, "read-ahead in whole dP slot pairs");

// Bytes of the kernel's LDS block: Q and dO rings, LSE / -D rows, V rows.
constexpr int kDkwLds = 2 * DKW_STAGES * 2 * DKW_BQ * 128 + 2 * 4 * DKW_STAGES * 64 + 2 * DKW_BN * 128;

// f(integral_constant<int, I>) for I = B .. E - 1, in order, inlined.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Static schedule of the persistent kernel: item `round` of workgroup b of G,
// as (key block kt, head bh); false when b has no more items.  With P > 0
// (BH % 8 == 0, G = 8 W): workgroup b runs on XCD b % 8 (consecutive
// workgroup ids go round-robin over the 8 XCDs), which owns heads
// x + 8 i; its items are taken P heads at a time (their K / V and Q / dO
// stay in that XCD's L2), within a group heaviest key block first, and
// dealt out snake-wise -- round r gives the XCD's W workgroups the next W
// items in forward order for even r and backward for odd r -- so that under a
// causal mask every workgroup pairs heavy with light blocks (at c5 each of
// the 256 workgroups gets exactly 544 query tiles).  P = 0: the same over
// all items, heads interleaved.
__device__ __forceinline__ bool sched_item(int b, int G, int round, int nkt, int BH, int P, int& kt, int& bh) {
  if (P > 0) {
    const int x = b & 7, W = G >> 3, j = b >> 3;
    const int idx = round * W + ((round & 1) ? W - 1 - j : j);
    if (idx >= (BH >> 3) * nkt) return false;
    const int gsz = P * nkt;
    const int gi = idx / gsz, e = idx - gi * gsz;
    kt = e / P;
    bh = x + 8 * (gi * P + (e - kt * P));
  } else {
    const int idx = round * G + ((round & 1) ? G - 1 - b : b);
    if (idx >= nkt * BH) return false;
    kt = idx / BH;
    bh = idx - kt * BH;
  }
  return true;
}

template <bool CAUSAL>
__device__ __forceinline__ void dkdv_w64_item(
    char* smem, const int kt, const int bh, const u16* __restrict__ Q, const u16* __restrict__ K,
    const u16* __restrict__ V, const u16* __restrict__ dO, const float* __restrict__ L2,
    const float* __restrict__ NDelta, u16* __restrict__ dK, u16* __restrict__ dV, int Lq, int Lk, float sl2,
    float scale) {
  constexpr int D = 128, NW = 4, BN = DKW_BN, BQ = DKW_BQ, S = DKW_STAGES, NC = D / 16, ND = D / 32;
  using Tile = SwzTile<D>;
  constexpr int TE = Tile::kElems(BQ);  // elements of one Q or dO tile
  constexpr int TB = 2 * TE;            // bytes of one Q or dO tile
  constexpr int VS = 64;                // stride (floats) of the LSE / -D row buffers
  using Dma = TileDma<D, BQ, NW>;
  constexpr int IPT = 2 * Dma::kLoads;  // Q + dO loads per wave per tile
  // One LDS block at fixed byte offsets (operand reads are a per-lane address
  // plus an immediate): the Q ring, the dO ring, the LSE / -D rows, then the
  // workgroup's V rows (half h of wave w at rows 32 w + 128 h).
  constexpr int kOQ = 0, kOdO = kOQ + S * TB, kOL = kOdO + S * TB, kOD = kOL + 4 * S * VS, kOV = kOD + 4 * S * VS,
                kLds = kOV + 2 * Tile::kElems(BN);
  constexpr int kVHalf = 2 * 128 * D;  // bytes between a wave's two V halves
  static_assert(kOdO - kOQ + (S - 1) * TB + TB <= 65536, "ring offsets exceed the LDS immediate");
  static_assert(kLds <= kDkwLds, "LDS block");
  u16* const sQ = reinterpret_cast<u16*>(smem + kOQ);
  u16* const sdO = reinterpret_cast<u16*>(smem + kOdO);
  float* const sL = reinterpret_cast<float*>(smem + kOL);
  float* const sDl = reinterpret_cast<float*>(smem + kOD);
  u16* const sV = reinterpret_cast<u16*>(smem + kOV);
  // The lane's LDS addresses are recomputed for every item (from opaque
  // copies of the base and the lane id): hoisted out of the persistent loop,
  // they would stay live across the epilogue and prologue and spill.
  uint32_t a0 = lds_addr(smem), tid = threadIdx.x;
  opaque(a0);
  opaque(tid);
  const int l = tid & 63, g = l >> 5, r32 = l & 31;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int k0 = kt * BN;
  const int key0 = k0 + 32 * w + r32, key1 = key0 + 128;
  const int64_t qbase = (int64_t)bh * Lq * D;
  const int64_t kbase = (int64_t)bh * Lk * D;
  const int64_t lbase = (int64_t)bh * Lq;

  // Query tiles [qstart, Lq); tile n lives in ring buffer n % S.  Query rows
  // past Lq read row Lq - 1 and are masked (P = 0).
  const int qstart = CAUSAL ? k0 : 0;  // k0 is a multiple of BQ
  const int ntiles = Lq > qstart ? (Lq - qstart + BQ - 1) / BQ : 0;
  Dma dma;
  dma.init();
  // Tile t's loads: the Q and dO tiles (kLoads instructions each) and the
  // LSE / -D rows, issued by every wave (the row loads write the same bytes
  // from each wave).  Instruction i < PER alone, always in bounds: a tile past
  // the last one re-reads row Lq - 1 into a buffer nobody reads, so that
  // every iteration issues exactly PER loads per wave and the waits are
  // constant.
  constexpr int PER = IPT + 2;
  auto load_part = [&](int t, int i) __attribute__((always_inline)) {
    const int b = t & (S - 1), qb = min(qstart + t * BQ, Lq - 1);
    if (i < Dma::kLoads)
      dma.issue_part_clamped(Q + qbase, qb, Lq, sQ + b * TE, i);
    else if (i < 2 * Dma::kLoads)
      dma.issue_part_clamped(dO + qbase, qb, Lq, sdO + b * TE, i - Dma::kLoads);
    else
      load_vec_lds((i == IPT ? L2 : NDelta) + lbase + qb, Lq - qb, (i == IPT ? sL : sDl) + b * VS);
  };
  // V rows first (the prologue's wait covers them), then tiles 0 .. S - 2.
  {
    TileDma<D, BN, NW> vdma;
    vdma.init();
    vdma.issue(V + kbase, k0, Lk, sV);
  }
  for (int t = 0; t < S - 1; ++t)
#pragma unroll
    for (int i = 0; i < PER; ++i) load_part(t, i);

  bf16x8 kf[2][NC];
  {
    const int kr0 = min(key0, Lk - 1), kr1 = min(key1, Lk - 1);  // rows past Lk are never stored
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      kf[0][c] = __builtin_bit_cast(bf16x8, ldg16(K + kbase + (int64_t)kr0 * D + 16 * c + 8 * g));
      kf[1][c] = __builtin_bit_cast(bf16x8, ldg16(K + kbase + (int64_t)kr1 * D + 16 * c + 8 * g));
    }
  }
  f32x16 adk[2][ND], adv[2][ND];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) adk[h][dt] = adv[h][dt] = f32x16{};

  // Loop-invariant LDS byte addresses of this lane in ring buffer 0: Q row
  // chunk 2c + g of row r32 (dO, other buffers: immediates away), the V rows
  // of half 0 (half 1: kVHalf away), the transpose reads at rows trow /
  // trow + 8 of column 32 dt + tcol (query chunk qc adds 16 rows), and the
  // LSE / -D rows.
  const int t16 = l & 15;
  const int trow = 4 * g + (t16 >> 2);
  const int tcol = 16 * ((l >> 4) & 1) + 4 * (t16 & 3);
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

  // Scores and MFMA operands.  s[h] holds S_n of the current tile (its
  // rows r < 8 already exponentiated, see below), dp[h] the dP accumulator.
  f32x16 s[2], dp[2];
  f32x16 nd;    // -D rows of the current tile (the dP accumulator's start)
  f32x4 la[2];  // LSE log2(e) rows j = 2, 3 of the current tile (registers r = 8..15)
  constexpr int A = DKW_READ_AHEAD;  // LDS reads run A slots ahead of their MFMA
  constexpr int KB = 32 - A;         // slot of barrier n + 1 (before the first read of tile n + 1)
  // Tile n + 3's PER loads go at slots KB + 5, KB + 11, ...: all of them must
  // fall inside the 64 slots, or barrier_next's constant vmcnt would count a
  // load that was never issued.
  static_assert(KB + 5 + 6 * (PER - 1) <= 63, "tile loads past the last slot of an iteration");
  bf16x8 dac[A / 2], vvc[2][A / 2];  // operands of the current tile's first dP slots, read ahead

  // Barrier n + 1: this wave's loads of tile n + 1 have landed (loads retire
  // in issue order; only tile n + 2's PER loads may still be in flight), then
  // every wave's are visible.  Every read of tile n - 1 has returned before
  // (the MFMAs of iteration n - 1 consumed them), so tile n + 3 may go into its
  // buffer after the barrier: one load instruction every 6 slots from slot
  // KB + 5, clear of the burst of LDS reads that follows the barrier (issued
  // back to back, the four waves' direct-to-LDS loads queue at the CU's
  // address unit and stall every wave; starting at KB + 1 measured 0.4 %
  // slower, KB + 2 every 5 slots 1.3 %).
  auto barrier_next = [&]() __attribute__((always_inline)) {
    wait_vmem_le<PER>();
    __builtin_amdgcn_s_barrier();
  };
  auto pexp = [&](int h, int r, float lse2) __attribute__((always_inline)) {
    float p = fast_exp2(fmaf(s[h][r], sl2, -lse2));
    pin(p);
    s[h][r] = p;
  };
  auto lane4 = [](const f32x4& v, int u) { return u == 0 ? v.x : u == 1 ? v.y : u == 2 ? v.z : v.w; };

  // Iteration n: tile n (query rows qb) in ring buffer B, tile n + 1 in
  // (B + 1) % S (B < 0: n % S at run time).  64 slots, one MFMA each, in the
  // order dP_n (slots 0-15), dV_n (16-31), S_{n+1} (32-47), dK_n (48-63);
  // slot k issues the LDS reads of slot k + 4 and a share of the VALU work:
  //   slots  0-15  P_n rows r = 8..15 (exponentials), the causal / ragged
  //                mask of all 32 rows, and their bf16 conversion
  //   slots 16-31  dS_n = P_n o (dP_n - D) and its bf16 conversion
  //   slots 48-63  P_{n+1} rows r = 0..7 (exponentials only)
  // A scheduling barrier closes every slot, so the compiler keeps this
  // order.  Barrier n + 1 sits at slot KB = 32 - A, before the first read of tile n + 1.
  auto iter = [&](int n, int qb, auto b_tag, auto mask_tag) __attribute__((always_inline)) {
    constexpr int BC = decltype(b_tag)::value;
    constexpr bool MASK = decltype(mask_tag)::value;
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
    const int b = BC >= 0 ? BC : (n & (S - 1));
    const int b1 = BC >= 0 ? ((BC + 1) & (S - 1)) : ((n + 1) & (S - 1));
    const int bq = b * TB, bq1 = b1 * TB, bl1 = b1 * 4 * VS;
    bf16x8 DA[NC], VV[2][NC], OV[2 * ND], QA[NC], OQ[2 * ND];
#pragma unroll
    for (int c = 0; c < A / 2; ++c) {
      DA[c] = dac[c];
      VV[0][c] = vvc[0][c];
      VV[1][c] = vvc[1][c];
    }
    bf16x8 pb[2][2], db[2][2];
    // Under the causal mask a key half can lie wholly after a diagonal tile's
    // queries (every P = 0): its MFMAs are skipped (a wave-uniform branch),
    // those of tile n (dP, dV, dK) by live(h) and those of tile n + 1 (S) by
    // live1(h).  A skipped half's scores and dP hold stale values that the
    // mask zeroes or nothing reads.
    const int klo = k0 + 32 * w;
    auto live = [&](int h) __attribute__((always_inline)) { return !MASK || !CAUSAL || qb + BQ - 1 >= klo + 128 * h; };
    auto live1 = [&](int h) __attribute__((always_inline)) {
      return !MASK || !CAUSAL || qb + 2 * BQ - 1 >= klo + 128 * h;
    };
    f32x4 lan[4];  // LSE rows of tile n + 1
    f32x16 ndn;    // -D rows of tile n + 1
    float prod[2];

    auto tr = [&](int tile_off, int i) __attribute__((always_inline)) {  // transposed operand i = qc * ND + dt
      const uint32_t o = tile_off + 2 * 16 * (i / ND) * D;
      return lds_tr16x2_at(troff[0][i % ND] + o, troff[1][i % ND] + o);
    };
    auto reads = [&](auto tt) __attribute__((always_inline)) {  // operands of slot t
      constexpr int t = decltype(tt)::value;
      if constexpr (t < 16) {
        constexpr int c = t / 2, h = t % 2;
        if constexpr (h == 0) DA[c] = lds_ld<bf16x8>(roff[c] + bq + (kOdO - kOQ));
        VV[h][c] = lds_ld<bf16x8>(voff[c] + h * kVHalf);
      } else if constexpr (t < 32) {
        if constexpr (t % 2 == 0) OV[(t - 16) / 2] = tr(bq + (kOdO - kOQ), (t - 16) / 2);
      } else if constexpr (t < 48) {
        if constexpr (t % 2 == 0) QA[(t - 32) / 2] = lds_ld<bf16x8>(roff[(t - 32) / 2] + bq1);
      } else if constexpr (t < 64) {
        if constexpr (t % 2 == 0) OQ[(t - 48) / 2] = tr(bq, (t - 48) / 2);
      } else {  // the next iteration's first dP slots (tile n + 1)
        constexpr int c = (t - 64) / 2, h = (t - 64) % 2;
        if constexpr (h == 0) dac[c] = lds_ld<bf16x8>(roff[c] + bq1 + (kOdO - kOQ));
        vvc[h][c] = lds_ld<bf16x8>(voff[c] + h * kVHalf);
      }
    };
    auto masked = [&](int h, int r) __attribute__((always_inline)) {
      if constexpr (MASK) {
        const int q = qb + acc_row(r, g);
        float p = (q >= Lq || (CAUSAL && (h == 0 ? key0 : key1) > q)) ? 0.f : s[h][r];
        pin(p);
        s[h][r] = p;
      }
    };
    auto slot = [&](auto kk) __attribute__((always_inline)) {
      constexpr int k = decltype(kk)::value;
      if constexpr (k == KB) barrier_next();
      if constexpr (k >= KB + 5 && (k - KB - 5) % 6 == 0 && (k - KB - 5) / 6 < PER) load_part(n + 3, (k - KB - 5) / 6);
      reads(std::integral_constant<int, k + A>{});
      // rows of tile n + 1 (after barrier n + 1)
      if constexpr (k >= 40 && k < 44) lan[k - 40] = lds_ld<f32x4>(lofs + bl1 + 32 * (k - 40));
      if constexpr (k >= 44 && k < 48) {
        const f32x4 v = lds_ld<f32x4>(lofs + (kOD - kOL) + bl1 + 32 * (k - 44));
        ndn[4 * (k - 44)] = v.x;
        ndn[4 * (k - 44) + 1] = v.y;
        ndn[4 * (k - 44) + 2] = v.z;
        ndn[4 * (k - 44) + 3] = v.w;
      }
      // VALU
      if constexpr (k < 16) {
        constexpr int r = 8 + k / 2, h = k % 2;
        pexp(h, r, lane4(la[(r - 8) / 4], r % 4));
        masked(h, r);
        if constexpr (r % 2 == 1) {
          pb[h][1][(r & 7) - 1] = (__bf16)s[h][r - 1];
          pb[h][1][r & 7] = (__bf16)s[h][r];
          pin(pb[h][1]);
        }
        if constexpr (k < 8) {
          masked(0, k);
          masked(1, k);
          if constexpr (k % 2 == 1) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              pb[hh][0][k - 1] = (__bf16)s[hh][k - 1];
              pb[hh][0][k] = (__bf16)s[hh][k];
              pin(pb[hh][0]);
            }
          }
        }
      } else if constexpr (k < 32) {
        constexpr int r = k - 16;
        if constexpr (r % 2 == 0) {
          prod[0] = s[0][r] * dp[0][r];
          prod[1] = s[1][r] * dp[1][r];
          pin(prod[0]);
          pin(prod[1]);
        } else {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            db[hh][r >> 3][(r & 7) - 1] = (__bf16)prod[hh];
            db[hh][r >> 3][r & 7] = (__bf16)(s[hh][r] * dp[hh][r]);
            pin(db[hh][r >> 3]);
          }
        }
      } else if constexpr (k >= 48) {
        constexpr int r = (k - 48) / 2, h = (k - 48) % 2;
        pexp(h, r, lane4(lan[r / 4], r % 4));
      }
      // MFMA
      if constexpr (k < 16) {
        constexpr int c = k / 2, h = k % 2;
        if (live(h)) dp[h] = mfma_bf16_32x32x16(DA[c], VV[h][c], c == 0 ? nd : dp[h]);
      } else if constexpr (k < 32) {
        constexpr int i = (k - 16) / 2, h = k % 2;
        if (live(h)) mfma_acc_agpr(adv[h][i % ND], OV[i], pb[h][i / ND]);
      } else if constexpr (k < 48) {
        constexpr int c = (k - 32) / 2, h = k % 2;
        if (live1(h)) s[h] = mfma_bf16_32x32x16(QA[c], kf[h][c], c == 0 ? f32x16{} : s[h]);
      } else {
        constexpr int i = (k - 48) / 2, h = k % 2;
        if (live(h)) mfma_acc_agpr(adk[h][i % ND], OQ[i], db[h][i / ND]);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    static_for<0, 64>(slot);
    nd = ndn;
    la[0] = lan[2];
    la[1] = lan[3];
  };
  using AnyBuf = std::integral_constant<int, -1>;
  int n = 0;
  auto run = [&](int hi_tile, auto mask_tag) __attribute__((always_inline)) {
    for (; n < hi_tile; ++n) iter(n, qstart + n * BQ, AnyBuf{}, mask_tag);
  };
  // Unmasked iterations, unrolled by ring buffer so that every LDS address
  // is a loop-invariant lane offset plus an immediate.
  auto run_full = [&](int hi_tile) __attribute__((always_inline)) {
    for (; n < hi_tile && (n & (S - 1)) != 0; ++n) iter(n, qstart + n * BQ, AnyBuf{}, std::false_type{});
    for (; n + S <= hi_tile; n += S) {
      iter(n, qstart + n * BQ, std::integral_constant<int, 0>{}, std::false_type{});
      iter(n + 1, qstart + (n + 1) * BQ, std::integral_constant<int, 1>{}, std::false_type{});
      iter(n + 2, qstart + (n + 2) * BQ, std::integral_constant<int, 2>{}, std::false_type{});
      iter(n + 3, qstart + (n + 3) * BQ, std::integral_constant<int, 3>{}, std::false_type{});
    }
    for (; n < hi_tile; ++n) iter(n, qstart + n * BQ, AnyBuf{}, std::false_type{});
  };
  static_assert(S == 4, "run_full unrolls by four ring buffers");

  // Prologue: retire the K row loads (and the V rows and first tiles with
  // them) here, so the compiler does not keep the K loads pending around the
  // loop; then S_0 with its rows r < 8 exponentiated, tile 0's rows and the
  // operands of its first dP slots.
  wait_vmem_le<0>();
  __syncthreads();
  if (ntiles > 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const bf16x8 qa = lds_ld<bf16x8>(roff[c]);
#pragma unroll
      for (int h = 0; h < 2; ++h) s[h] = mfma_bf16_32x32x16(qa, kf[h][c], c == 0 ? f32x16{} : s[h]);
    }
    f32x4 l0[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      l0[j] = lds_ld<f32x4>(lofs + 32 * j);
      const f32x4 v = lds_ld<f32x4>(lofs + (kOD - kOL) + 32 * j);
      nd[4 * j] = v.x;
      nd[4 * j + 1] = v.y;
      nd[4 * j + 2] = v.z;
      nd[4 * j + 3] = v.w;
    }
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
      for (int h = 0; h < 2; ++h) pexp(h, r, lane4(l0[r / 4], r % 4));
    la[0] = l0[2];
    la[1] = l0[3];
#pragma unroll
    for (int c = 0; c < A / 2; ++c) {
      dac[c] = lds_ld<bf16x8>(roff[c] + (kOdO - kOQ));
      vvc[0][c] = lds_ld<bf16x8>(voff[c]);
      vvc[1][c] = lds_ld<bf16x8>(voff[c] + kVHalf);
    }
    // tiles [0, ndiag) cross the causal diagonal; [nfull, ntiles) is the ragged tail
    const int ndiag = CAUSAL ? min(ntiles, BN / BQ) : 0;
    const int nfull = max(ndiag, (Lq - qstart) / BQ);
    run(ndiag, std::true_type{});
    run_full(nfull);
    run(ntiles, std::true_type{});
  }
  wait_vmem_le<0>();  // nothing may be in flight into LDS when the workgroup exits
  agpr_drain(adk, adv);

  // Epilogue through LDS: the rows dK (scaled) and dV of the workgroup's 256
  // keys go to LDS as bf16 (SwzTile layout, dK rows 0-255 then dV rows
  // 256-511), then every lane stores whole 16-byte chunks, so one store
  // instruction writes four contiguous 256-byte rows.  Stored straight from
  // the accumulators (8 bytes per lane into 32 different rows) the epilogue
  // took about 10 us per workgroup at c5.
  static_assert(kLds >= 2 * 2 * Tile::kElems(BN), "LDS block too small for the staged epilogue");
  __syncthreads();  // every wave is done with the ring and the V rows
  u16* const stage = reinterpret_cast<u16*>(smem);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = 32 * w + 128 * h + r32;
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        const int d0 = 32 * dt + acc_row(r, g);
        uint2 a, bb;
        a.x = pack_bf16x2(adk[h][dt][r] * scale, adk[h][dt][r + 1] * scale);
        a.y = pack_bf16x2(adk[h][dt][r + 2] * scale, adk[h][dt][r + 3] * scale);
        bb.x = pack_bf16x2(adv[h][dt][r], adv[h][dt][r + 1]);
        bb.y = pack_bf16x2(adv[h][dt][r + 2], adv[h][dt][r + 3]);
        *reinterpret_cast<uint2*>(&stage[Tile::at4(row, d0)]) = a;
        *reinterpret_cast<uint2*>(&stage[Tile::at4(BN + row, d0)]) = bb;
      }
  }
  __syncthreads();
  constexpr int CPR = D / 8;  // 16-byte chunks per row
#pragma unroll 4
  for (int c = threadIdx.x; c < 2 * BN * CPR; c += 64 * NW) {
    const int row = c / CPR, ch = c % CPR;
    const int key = k0 + (row & (BN - 1));
    if (key < Lk) {
      const uint4 v = *reinterpret_cast<const uint4*>(&stage[Tile::chunk(row, ch)]);
      *reinterpret_cast<uint4*>((row < BN ? dK : dV) + kbase + (int64_t)key * D + 8 * ch) = v;
    }
  }
}

// Persistent kernel: G workgroups (at most one per CU, so all run at once),
// each working through its items of sched_item.
template <bool CAUSAL>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_w64_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V,
    const u16* __restrict__ dO, const float* __restrict__ L2, const float* __restrict__ NDelta,
    u16* __restrict__ dK, u16* __restrict__ dV, int Lq, int Lk, int BH, int nkt, int P, float sl2,
    float scale) {
  __shared__ __align__(16) char smem[kDkwLds];
  int kt, bh;
  for (int round = 0; sched_item(blockIdx.x, gridDim.x, round, nkt, BH, P, kt, bh); ++round) {
    if (round > 0) __syncthreads();  // the previous item's epilogue reads of LDS are done
    dkdv_w64_item<CAUSAL>(smem, kt, bh, Q, K, V, dO, L2, NDelta, dK, dV, Lq, Lk, sl2, scale);
  }
}

}  // namespace

// Launches the kernel above on `st` (dK, dV of every key of BH heads; L2 /
// ND: the rows LSE log2(e) and -D the dQ kernel wrote).
int launch_dkdv_w64(const u16* q, const u16* k, const u16* v, const u16* dout, const float* l2, const float* nd,
                    u16* dk, u16* dv, int64_t BH, int64_t Lq, int64_t Lk, float sl2, float scale, bool causal,
                    hipStream_t st) {
  const int64_t nkt = (Lk + DKW_BN - 1) / DKW_BN;
  if (!grid_fits(nkt * BH, 256)) return fail(TT_ERR_ARG, "attention backward: grid too large");
  // one workgroup per CU (the LDS block allows no second), each through its share of the items
  const int64_t cus = device_cu_count(), items = nkt * BH;
  const int G = (int)(items < cus ? items : cus);
  const int P = (G % 8 == 0 && G >= 64) ? pick_group(BH, nkt, G / 8) : 0;
  if (causal)
    hipLaunchKernelGGL((attn_bwd_dkdv_w64_kernel<true>), dim3((unsigned)G), dim3(256), 0, st, q, k, v, dout, l2,
                       nd, dk, dv, (int)Lq, (int)Lk, (int)BH, (int)nkt, P, sl2, scale);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_w64_kernel<false>), dim3((unsigned)G), dim3(256), 0, st, q, k, v, dout, l2,
                       nd, dk, dv, (int)Lq, (int)Lk, (int)BH, (int)nkt, P, sl2, scale);
  TT_LAUNCHED("attention backward dK/dV launch", st);
  return ok();
}

}  // namespace tt
