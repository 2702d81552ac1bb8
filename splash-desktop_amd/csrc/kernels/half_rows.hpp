// The prefill tile's prepared input ("half rows"): each row of bf16 activations scaled by the power of two that
// puts its largest magnitude in [2^15, 2^16) and converted to fp16, stored group by group in the tile's read order,
// with the power of two kept per row for the epilogue. Scaling up as well as down keeps a row of any magnitude
// exact: every value of the row within 2^29 of its largest is a normal half after the scale (bf16's 8 significant
// bits fit half's 11), so only values below 2^-29 of the row's largest round, by at most 2^-25 of a half unit, that
// is 2^-40 of the largest, far below the fp32 accumulation's own error. The prefill's own prepare dispatch and the
// RMS norm producer both write it, from the same bf16 values and with these same helpers, so the table is the same
// bits whichever wrote it.
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

// The row's shift: the table holds x 2^-shift, the largest magnitude in [2^15, 2^16). The shift stays at -126 or
// above so that 2^shift and 2^-shift are both normal floats: a row whose largest magnitude is below 2^-111 (a zero
// row, or bf16 subnormals) takes -126, where every nonzero bf16 value times 2^126 is at least 2^-7, a normal half.
// Infinities and NaNs count as 2^128 (shift 113), as before.
__device__ __forceinline__ int half_rows_shift(uint32_t largest) {
  const int exponent = (int)(min(largest, 0x7F80u) >> 7) - 127;
  return max(exponent - 15, -126);
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
