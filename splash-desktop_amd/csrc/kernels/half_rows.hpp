// The prefill tile's prepared input ("half rows"): each row of bf16 activations scaled by a power of two that
// brings its largest magnitude below 2^16 and converted to fp16, which is exact for every bf16 value in half's
// normal range, stored group by group in the tile's read order, with the power of two kept per row for the
// epilogue. The prefill's own prepare dispatch and the RMS norm producer both write it, from the same bf16 values
// and with these same helpers, so the table is the same bits whichever wrote it.
#pragma once
#include "device.hpp"

namespace sq::kern {

// Chunk v (8 fp16 values, 16 bytes) of a row's table holds inputs 32 g + 4 c .. +3 and 32 g + 16 + 4 c .. +3
// (g = v / 4, c = v % 4): the row's 4-input units half_rows_unit(v) and half_rows_unit(v) + 4.
__device__ __forceinline__ uint32_t half_rows_unit(uint32_t v) { return 8 * (v >> 2) + (v & 3); }

// The largest magnitude among eight bf16 values, as bits (bf16 bit patterns order like their magnitudes).
__device__ __forceinline__ uint32_t bf16_largest(u32x4 w) {
  uint32_t m = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) m = max(m, max(w[e] & 0x7FFFu, (w[e] >> 16) & 0x7FFFu));
  return m;
}

// The row's shift: the table holds x 2^-shift, so that the largest magnitude ends below 2^16 (shift 0 when it is
// already).
__device__ __forceinline__ int half_rows_shift(uint32_t largest) {
  const int exponent = (int)(min(largest, 0x7F80u) >> 7) - 127;
  return exponent >= 16 ? exponent - 15 : 0;
}

// Eight bf16 values times `down` (a power of two) as fp16, in the same order.
__device__ __forceinline__ u32x4 half_rows_chunk(u32x4 w, float down) {
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = (uint32_t)f32_to_f16(bf16_to_f32(w[e] & 0xFFFFu) * down) |
           ((uint32_t)f32_to_f16(bf16_to_f32(w[e] >> 16) * down) << 16);
  return o;
}

}  // namespace sq::kern
