// Host copy / conversion loops of the staged transfers (x86-64, SSE2 only).
// Each routine writes a scalar head until the destination is 16-byte
// aligned, streams 64 destination bytes per step with movntdq, finishes with
// a scalar tail and fences the streamed stores before it returns.
#include "host_copy.h"

#include <emmintrin.h>

#include <cstring>

namespace tt {
namespace {

uint16_t f32_to_bf16_scalar(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Four float32 bit patterns -> four bf16 patterns, sign-extended to 32 bits
// so that _mm_packs_epi32 passes them through unchanged.
inline __m128i bf16x4(__m128i u) {
  const __m128i mag = _mm_and_si128(u, _mm_set1_epi32(0x7fffffff));
  const __m128i nan = _mm_cmpgt_epi32(mag, _mm_set1_epi32(0x7f800000));
  const __m128i hi = _mm_srli_epi32(u, 16);
  // u + 0x7fff + lsb wraps only for u >= 0xffff8001, which are NaNs
  const __m128i rne =
      _mm_srli_epi32(_mm_add_epi32(_mm_add_epi32(u, _mm_set1_epi32(0x7fff)), _mm_and_si128(hi, _mm_set1_epi32(1))), 16);
  const __m128i qnan = _mm_or_si128(hi, _mm_set1_epi32(0x40));
  const __m128i r = _mm_or_si128(_mm_and_si128(nan, qnan), _mm_andnot_si128(nan, rne));
  return _mm_srai_epi32(_mm_slli_epi32(r, 16), 16);
}

// Elements to write one by one before dst reaches a 16-byte boundary; all of
// them when dst is not even aligned to its element size (streaming then
// never reaches an aligned address).
size_t head_elems(const void* dst, size_t elem, size_t n) {
  const size_t mis = reinterpret_cast<uintptr_t>(dst) & 15;
  if (mis % elem) return n;
  const size_t h = ((16 - mis) & 15) / elem;
  return h < n ? h : n;
}

}  // namespace

void copy_stream(void* dst, const void* src, size_t n) {
  char* d = static_cast<char*>(dst);
  const char* s = static_cast<const char*>(src);
  const size_t h = head_elems(d, 1, n);
  std::memcpy(d, s, h);
  d += h, s += h, n -= h;
  size_t i = 0;
  for (; i + 64 <= n; i += 64) {
    const __m128i a = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i));
    const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 16));
    const __m128i c = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 32));
    const __m128i e = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 48));
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i), a);
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 16), b);
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 32), c);
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 48), e);
  }
  std::memcpy(d + i, s + i, n - i);
  _mm_sfence();
}

void f32_to_bf16_stream(uint16_t* d, const float* s, size_t n) {
  const size_t h = head_elems(d, 2, n);
  for (size_t i = 0; i < h; ++i) {
    const uint16_t b = f32_to_bf16_scalar(s[i]);
    std::memcpy(d + i, &b, 2);
  }
  d += h, s += h, n -= h;
  size_t i = 0;
  for (; i + 32 <= n; i += 32) {
    for (int j = 0; j < 4; ++j) {
      const __m128i a = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 8 * j));
      const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 8 * j + 4));
      _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 8 * j), _mm_packs_epi32(bf16x4(a), bf16x4(b)));
    }
  }
  for (; i < n; ++i) {
    const uint16_t b = f32_to_bf16_scalar(s[i]);
    std::memcpy(d + i, &b, 2);
  }
  _mm_sfence();
}

void bf16_to_f32_stream(float* d, const uint16_t* s, size_t n) {
  const size_t h = head_elems(d, 4, n);
  for (size_t i = 0; i < h; ++i) {
    const uint32_t u = uint32_t(s[i]) << 16;
    std::memcpy(d + i, &u, 4);
  }
  d += h, s += h, n -= h;
  const __m128i z = _mm_setzero_si128();
  size_t i = 0;
  for (; i + 16 <= n; i += 16) {
    const __m128i a = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i));
    const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(s + i + 8));
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i), _mm_unpacklo_epi16(z, a));
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 4), _mm_unpackhi_epi16(z, a));
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 8), _mm_unpacklo_epi16(z, b));
    _mm_stream_si128(reinterpret_cast<__m128i*>(d + i + 12), _mm_unpackhi_epi16(z, b));
  }
  for (; i < n; ++i) {
    const uint32_t u = uint32_t(s[i]) << 16;
    std::memcpy(d + i, &u, 4);
  }
  _mm_sfence();
}

}  // namespace tt
