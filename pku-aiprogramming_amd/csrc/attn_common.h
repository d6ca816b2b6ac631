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

// Round-to-nearest-even float -> bf16 bits (NaN kept quiet).
__device__ __forceinline__ u16 f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return u16((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u16(u >> 16);
}

// Two floats -> packed bf16x2 (low half = a), RNE.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return uint32_t(f32_to_bf16(a)) | (uint32_t(f32_to_bf16(b)) << 16);
}

__device__ __forceinline__ f32x16 mfma_bf16_32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_f32_32x32x2(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Row of the 32x32 accumulator tile held in register r by a lane in half g.
__device__ __forceinline__ constexpr int acc_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// Key order inside a 16-key k-chunk of the P^T operand.  Accumulator
// registers 8h..8h+7 of lane half g hold keys 16h' + 8*(e/4) + 4*g + e%4, so
// a [d][key] LDS tile stores key j at position perm16(j) (bits 2 and 3 of j
// swapped); a lane then reads its 8 keys as one 16-byte vector.
__device__ __forceinline__ constexpr int perm16(int j) {
  return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
}

__device__ __forceinline__ float wave_xor32(float x) { return __shfl_xor(x, 32, 64); }

// Exact power-of-two exponent: v_exp_f32 computes 2^x.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

}  // namespace tt
