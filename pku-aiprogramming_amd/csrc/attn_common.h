// Device-side building blocks of the gfx950 attention kernels.
//
// MFMA operand layouts used throughout (checked on the MI355X by an in-bounds
// probe of each builtin):
//   v_mfma_f32_32x32x16_bf16  A[32 x 16], B[16 x 32], C[32 x 32]
//     lane l holds A[m = l%32][k = 8*(l/32) + e], e = 0..7 (one bf16x8)
//               B[k = 8*(l/32) + e][n = l%32]
//     accumulator register r (0..15) of lane l is C[8*(r/4) + 4*(l/32) + r%4][l%32]
//   v_mfma_f32_32x32x2f32     lane l holds A[l%32][l/32], B[l/32][l%32];
//     same accumulator layout.
//
// All kernels compute the transposed score tile S^T = K Q^T (M = keys,
// N = queries) so that every lane owns one query column: the row softmax then
// needs one cross-lane step (lanes l and l^32 share a query) instead of a
// 32-lane reduction.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace tt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bf16_to_f32(u16 b) { return __uint_as_float(uint32_t(b) << 16); }

// Round-to-nearest-even float -> bf16 bits (v_cvt_pk_bf16_f32 on gfx950;
// NaN stays NaN).
__device__ __forceinline__ u16 f32_to_bf16(float f) { return __builtin_bit_cast(u16, (__bf16)f); }

// Two floats -> packed bf16x2 (low half = a), RNE.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ f32x16 mfma_bf16_32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row of the 32x32 accumulator tile held in register r by a lane in half g.
__device__ __forceinline__ constexpr int acc_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

__device__ __forceinline__ float wave_xor32(float x) { return __shfl_xor(x, 32, 64); }

// Reductions over lanes l and l ^ 32 in two VALU ops, with no LDS round
// trip: v_permlane32_swap of x with a copy of itself returns r[0] = lanes
// 0..31 of x in both halves and r[1] = lanes 32..63 in both halves (checked
// on the MI355X).  Both halves compute the same expression, so they agree
// bit for bit.
// Maximum of two floats that propagates NaN (IEEE 754-2019 maximum): on gfx950
// v_maximum_f32 / v_maximum3_f32.  fmaxf (maxNum) in the kernels' IEEE mode
// quiets each operand the compiler cannot prove canonical first, one
// v_max_f32 x, x, x per MFMA result or cross-lane value it reads (11 extra VALU
// operations per tile in the forward's row max); a NaN score gives a NaN row
// either way.
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float vmax3(float a, float b, float c) { return vmax(vmax(a, b), c); }

__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}


// acc + the two bf16 halves of element e (a bf16 pair) of v, by one
// v_dot2_f32_bf16 against (1, 1).
__device__ __forceinline__ float sum_bf16x2(const bf16x8& v, int e, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 pair = {v[2 * e], v[2 * e + 1]};
  const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
  return __builtin_amdgcn_fdot2_f32_bf16(pair, one, acc, false);
}

// Exact power-of-two exponent: v_exp_f32 computes 2^x.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// 16-byte load marked non-temporal (global_load_dwordx4 ... nt): for data
// streamed once, such as the decode's K/V cache.  On the MI355X a streaming
// read of an 8 GiB buffer runs at 7.1-7.2 TB/s with these loads against
// 6.2-6.4 TB/s with ordinary ones.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return uint4{v.x, v.y, v.z, v.w};
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// ds_read_b64_tr_b16 (gfx950).  Within each 16-lane group, lane t receives
// element t%4 of the 8-byte chunks addressed by lanes 4e + t/4, e = 0..3.
// So if lane s of the group points at row (r0 + s/4), column (c0 + 4*(s%4))
// of a row-major b16 matrix, lane t gets rows r0..r0+3 of column c0 + t:
// four consecutive k-values of one column, the MFMA operand layout.
__device__ __forceinline__ s16x4 lds_read_tr16(const u16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

// Two transpose reads (rows r0..r0+3 and r1..r1+3 of one column) as one
// bf16x8 MFMA operand.
__device__ __forceinline__ bf16x8 lds_read_tr16x2(const u16* p0, const u16* p1) {
  s16x4 a = lds_read_tr16(p0), b = lds_read_tr16(p1);
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  s16x8 v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ bool wave_any(bool p) { return __any(p); }

// __builtin_amdgcn_iglp_opt with a template-chosen strategy (the builtin takes
// a constant).
template <int K>
__device__ __forceinline__ void iglp() {
  __builtin_amdgcn_iglp_opt(K);
}

// Redefines x in place with no instruction, so loop-invariant code motion
// cannot hoist (x + constant) out of a loop into a second register: the
// constant then folds into the memory instruction's offset field.
__device__ __forceinline__ void opaque(uint32_t& x) { asm volatile("" : "+v"(x)); }

// LDS reads at a byte address (as lds_addr returns).
template <typename V>
__device__ __forceinline__ V lds_ld(uint32_t a) {
  return *(const __attribute__((address_space(3))) V*)(uintptr_t)a;
}
__device__ __forceinline__ bf16x8 lds_tr16x2_at(uint32_t a0, uint32_t a1) {
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)a0);
  s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)a1);
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  s16x8 v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// Dense row-major bf16 tile of D columns in LDS, addressed by 16-byte
// chunks, that serves two read patterns without bank conflicts:
//   * 16-byte row reads: 16 lanes read one chunk of 16 consecutive rows;
//   * transpose reads: 32 lanes read 4 consecutive 8-byte pieces of each of
//     4 consecutive rows (rows r0..r0+3 with r0 % 4 == 0).
// Chunk c of row r is stored at chunk c ^ sw(r) of that row.  With 256-byte
// bank lines (64 banks x 4 bytes) the swizzle spreads both patterns over 16
// distinct 16-byte bank groups:
//   D = 128 (one row per line):    sw = ((r & 3) << 2) | ((r >> 2) & 3)
//   D = 64  (two rows per line):   sw = (((r >> 1) & 1) << 2) | ((r >> 2) & 3)
//   D = 32  (four rows per line):  sw = (r >> 2) & 3
// The tile has no padding, so a wave's 64 consecutive 16-byte slots can be
// filled by one direct global->LDS load (see TileDma).
template <int D>
struct SwzTile {
  static constexpr int kCPR = D / 8;  // chunks per row
  static constexpr int kElems(int rows) { return rows * D; }
  __device__ static __forceinline__ constexpr int sw(int r) {
    if constexpr (D == 128) return ((r & 3) << 2) | ((r >> 2) & 3);
    if constexpr (D == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    return (r >> 2) & 3;
  }
  // element offset of chunk `ch` (8 elements) of row `row`
  __device__ static __forceinline__ int chunk(int row, int ch) { return row * D + 8 * (ch ^ sw(row)); }
  // element offset of column `col` (a multiple of 4) of row `row`
  __device__ static __forceinline__ int at4(int row, int col) { return chunk(row, col >> 3) + (col & 4); }
};

// Output epilogue through LDS.  An MFMA kernel whose lane (r32, g) holds, in
// accumulator tile dt, columns 32 dt + acc_row(r, g) (r = 0..15) of output
// row `row` writes those values to LDS as bf16 (scaled by `mul`), four
// columns per 8-byte write, in the SwzTile layout; after a barrier every
// thread copies whole 16-byte chunks to global memory, so one store
// instruction writes 1 KB of contiguous rows.  Written straight from the
// accumulators, each 8-byte store instruction touches 32 rows, and the
// epilogue of a workgroup took 1-2.5 us on the MI355X.
template <int D, int ND>
__device__ __forceinline__ void stage_rows_bf16(u16* stage, int row, int g, const f32x16 (&acc)[ND], float mul) {
  using Tile = SwzTile<D>;
#pragma unroll
  for (int dt = 0; dt < ND; ++dt)
#pragma unroll
    for (int r = 0; r < 16; r += 4) {
      uint2 v;
      v.x = pack_bf16x2(acc[dt][r] * mul, acc[dt][r + 1] * mul);
      v.y = pack_bf16x2(acc[dt][r + 2] * mul, acc[dt][r + 3] * mul);
      *reinterpret_cast<uint2*>(&stage[Tile::at4(row, 32 * dt + acc_row(r, g))]) = v;
    }
}
// Rows [0, nrows) of `stage` to rows row0 + i of the row-major [., D] matrix
// at `dst`, skipping rows >= rmax; `nthreads` threads of the workgroup.
template <int D>
__device__ __forceinline__ void store_staged_rows(const u16* stage, int nrows, u16* dst, int row0, int rmax,
                                                  int nthreads) {
  using Tile = SwzTile<D>;
  constexpr int CPR = D / 8;
#pragma unroll 4
  for (int c = threadIdx.x; c < nrows * CPR; c += nthreads) {
    const int row = c / CPR, ch = c - row * CPR;
    if (row0 + row < rmax)
      *reinterpret_cast<uint4*>(dst + (int64_t)(row0 + row) * D + 8 * ch) =
          *reinterpret_cast<const uint4*>(&stage[Tile::chunk(row, ch)]);
  }
}

typedef __attribute__((address_space(3))) void lds_void;

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void*)p;
}

// Direct global->LDS loads.  Lane l copies `bytes` bytes from
// sbase + voff (sbase wave-uniform, voff per lane) to LDS byte address
// lds + bytes * l; M0 carries the LDS base.
//
// They are written as inline asm on purpose.  The compiler's wait-count pass
// does model the LDS write of the builtin form, but it cannot tell the
// buffers of a tile ring apart (dynamic offsets into one array), so it puts
// an s_waitcnt vmcnt(0) in front of the first LDS read of every tile, which
// waits for the tile being prefetched and serialises the ring.  Here the
// kernels order these loads themselves: a vmcnt wait for the tile (loads
// retire in order) followed by a workgroup barrier, before any LDS read of
// that buffer.  M0 is a reserved register that the compiler only sets right
// before the instructions that read it; each statement sets it itself.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void glds16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void glds4(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// Direct global->LDS loader of [ROWS x D] bf16 tiles of a row-major [*, D]
// matrix into SwzTile<D> buffers, shared by the loading waves (kWaves: all NW
// of the workgroup, or fewer for tiles smaller than one instruction per
// wave).  Load instruction i of wave w fills the 64 consecutive 16-byte LDS
// slots starting at slot 64 (i kWaves + w); each lane fetches the global
// chunk that belongs in its slot.  One instruction covers 64 / kCPR rows, so
// step i moves kStep = kWaves * 64 / kCPR rows on.  Every swizzle has a period
// dividing 16 rows, so the lane's chunk column repeats every kPh = 16 /
// gcd(kStep, 16) instructions: instruction i reads at byte offset
// voff[i % kPh] + 2 D kStep (i - i % kPh), with the kPh offsets computed
// once.
template <int D, int ROWS, int NW>
struct TileDma {
  static constexpr int kCPR = D / 8;
  // waves that load: all NW, or the first ones when the tile holds fewer
  // 16-byte chunks than one instruction of every wave (32-row tiles at d = 32)
  static constexpr int kWaves = ROWS * kCPR >= 64 * NW ? NW : ROWS * kCPR / 64;
  static_assert(kWaves >= 1 && ROWS * kCPR % (64 * kWaves) == 0, "tile must split evenly over the waves");
  static constexpr int kStep = kWaves * 64 / kCPR;  // rows per load instruction of the workgroup
  static_assert(kStep % 16 == 0 || 16 % kStep == 0, "row step must divide or be a multiple of 16");
  static constexpr int kPh = kStep % 16 == 0 ? 1 : 16 / kStep;
  static constexpr int kLoads = ROWS * kCPR / (64 * kWaves);  // load instructions per loading wave per tile
  // waves w >= kWaves issue nothing (w is wave-uniform)
  __device__ __forceinline__ bool idle() const { return kWaves < NW && w >= kWaves; }
  static_assert(kLoads % kPh == 0 || kLoads < kPh, "loads must cover whole swizzle periods");
  uint32_t voff[kPh];  // this lane's byte offsets for instructions 0..kPh-1, from the tile's first row
  int w;

  __device__ __forceinline__ void init() {
    w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p = w * 64 + (threadIdx.x & 63);
#pragma unroll
    for (int ph = 0; ph < kPh; ++ph) {
      const int row = p / kCPR + ph * kStep, ch = (p % kCPR) ^ SwzTile<D>::sw(row);
      voff[ph] = 2u * (uint32_t)(row * D + 8 * ch);
    }
  }
  // Issue load instruction i (0 <= i < kLoads) of the tile of rows
  // [row0, row0 + ROWS) of `src`, which must lie inside the matrix.  Kernels
  // spread a tile's instructions over their compute: issued back to back
  // right after a barrier, the loads of every wave queue at the CU's texture
  // address unit and each wave stalls until its own are accepted.
  __device__ __forceinline__ void issue_one(const u16* src, int row0, const u16* dst, int i) const {
    if (idle()) return;
    glds16(src + (int64_t)row0 * D + (int64_t)D * kStep * (i - i % kPh), voff[i % kPh],
           lds_addr(dst) + 1024u * (uint32_t)(w + kWaves * i));
  }
  // Load instruction i (0 <= i < kLoads) alone of issue(src, row0, rmax,
  // dst), always by the clamped form (no branch), for kernels that spread a
  // tile's loads over their compute.  Requires 0 <= row0 < rmax.
  __device__ __forceinline__ void issue_part_clamped(const u16* src, int row0, int rmax, const u16* dst, int i) const {
    if (idle()) return;
    const int p0 = w * 64 + (threadIdx.x & 63);
    const int r0 = p0 / kCPR;
    const int ch = (p0 % kCPR) ^ SwzTile<D>::sw(r0 + i * kStep);
    const int row = min(r0 + i * kStep, rmax - 1 - row0);
    glds16(src + (int64_t)row0 * D, 2u * (uint32_t)(row * D + 8 * ch), lds_addr(dst) + 1024u * (uint32_t)(w + kWaves * i));
  }
  // Issue the loads of rows [row0, row0 + ROWS) of `src`, all of which lie
  // inside the matrix, into the tile at `dst` (no bounds test).
  __device__ __forceinline__ void issue_full(const u16* src, int row0, const u16* dst) const {
    if (idle()) return;
    const u16* base = src + (int64_t)row0 * D;
    const uint32_t lds = lds_addr(dst) + 1024u * (uint32_t)w;
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      glds16(base + (int64_t)D * kStep * (i - i % kPh), voff[i % kPh], lds + 1024u * kWaves * i);
  }
  // Issue the loads of rows [row0, row0 + ROWS) of `src` into the tile at
  // `dst`.  Requires 0 <= row0 < rmax; rows >= rmax read row rmax - 1 instead
  // (callers mask them).  Completion: a vmcnt wait, then a barrier.
  __device__ __forceinline__ void issue(const u16* src, int row0, int rmax, const u16* dst) const {
    if (idle()) return;
    const u16* base = src + (int64_t)row0 * D;
    const uint32_t lds = lds_addr(dst) + 1024u * (uint32_t)w;
    if (row0 + ROWS <= rmax) {
#pragma unroll
      for (int i = 0; i < kLoads; ++i)
        glds16(base + (int64_t)D * kStep * (i - i % kPh), voff[i % kPh], lds + 1024u * kWaves * i);
    } else {
      const int p0 = w * 64 + (threadIdx.x & 63);
      const int r0 = p0 / kCPR;
#pragma unroll
      for (int i = 0; i < kLoads; ++i) {
        // the slot's chunk column follows the swizzle of its own (unclamped) row
        const int ch = (p0 % kCPR) ^ SwzTile<D>::sw(r0 + i * kStep);
        const int row = min(r0 + i * kStep, rmax - 1 - row0);
        glds16(base, 2u * (uint32_t)(row * D + 8 * ch), lds + 1024u * kWaves * i);
      }
    }
  }
};

// s_waitcnt vmcnt(N): wait until at most N of this wave's global loads are
// outstanding (loads retire in order), LDS / export counters untouched.
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Runtime count n in [0, MAXN] (MAXN <= 3): wait until at most n * PER
// loads remain.
template <int PER, int MAXN = 3>
__device__ __forceinline__ void wait_vmem_tiles(int n) {
  static_assert(MAXN >= 0 && MAXN <= 3, "at most 3 tiles in flight");
  if (MAXN >= 3 && n >= 3) wait_vmem_le<(MAXN >= 3 ? 3 : 0) * PER>();
  else if (MAXN >= 2 && n == 2) wait_vmem_le<(MAXN >= 2 ? 2 : 0) * PER>();
  else if (MAXN >= 1 && n == 1) wait_vmem_le<(MAXN >= 1 ? 1 : 0) * PER>();
  else wait_vmem_le<0>();
}

// Direct global->LDS load of 64 floats by one wave: dst[i] = src[min(i, nmax - 1)]
// (src wave-uniform, nmax >= 1).
__device__ __forceinline__ void load_vec_lds(const float* src, int nmax, const float* dst) {
  // The lane index is recomputed here (volatile, so it is not hoisted out of
  // the caller's loop): a register-starved kernel would otherwise keep it in
  // a scratch slot, and the reload's vmcnt wait would drain the tile loads
  // issued just before.
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  glds4(src, 4u * (uint32_t)min(l, nmax - 1), lds_addr(dst));
}

}  // namespace tt
