// Host-side copy and conversion loops for the staged transfers: SSE2 with
// non-temporal stores, so that filling a staging buffer (or a caller's
// array) does not first read the destination lines into the cache.
#pragma once

#include <cstddef>
#include <cstdint>

namespace tt {

// n bytes; any alignment.
void copy_stream(void* dst, const void* src, size_t n);
// n float32 -> n bf16 bit patterns, round to nearest even; NaN stays a quiet
// NaN of the same sign.
void f32_to_bf16_stream(uint16_t* dst, const float* src, size_t n);
// n bf16 bit patterns -> n float32 (exact).
void bf16_to_f32_stream(float* dst, const uint16_t* src, size_t n);

}  // namespace tt
