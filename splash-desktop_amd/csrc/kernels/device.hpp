// Device helpers shared by the gfx950 kernels: vector types, the bf16 MFMA, the exact code operands, bf16/fp16
// conversions and the per-format coefficient decode.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../abi.h"

namespace sq::kern {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
typedef __attribute__((__vector_size__(4 * sizeof(short)))) short i16x4;

// D = A B + C on a 16x16x32 bf16 tile. Lane l holds A[l % 16][8 (l / 16) + i], B[8 (l / 16) + i][l % 16] and
// D[4 (l / 16) + i][l % 16] (i = 0..7, 0..7, 0..3).
__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}
// D = A B + C on a 16x16x16 bf16 tile: lane l holds A[l % 16][4 (l / 16) + i], B[4 (l / 16) + i][l % 16] (i = 0..3)
// and D as mfma_bf16 does.
__device__ __forceinline__ f32x4 mfma_bf16_k16(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a), __builtin_bit_cast(i16x4, b), c, 0,
                                                    0, 0);
}
__device__ __forceinline__ f32x4 mfma_f16(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                 0);
}

// D = A B + C on sixteen 4x4x4 bf16 blocks with block `abid`'s A broadcast to all sixteen (cbsz 4). Lane 4b + i holds
// A[b][i][0..3] and B[b][0..3][i] (block b = lane / 4) and D[b][0..3][i]: with the broadcast, lane l's D is the four
// A rows of block abid against the lane's own four B values. abid folds to a constant once the caller's loop is
// unrolled (the instruction takes it as an immediate).
__device__ __forceinline__ f32x4 mfma_bcast(int abid, u32x2 a, u32x2 b, f32x4 c) {
  const i16x4 av = __builtin_bit_cast(i16x4, a), bv = __builtin_bit_cast(i16x4, b);
#define SQ_MFMA_BCAST(k) \
  case k: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(av, bv, c, 4, k, 0);
  switch (abid) {
    SQ_MFMA_BCAST(0) SQ_MFMA_BCAST(1) SQ_MFMA_BCAST(2) SQ_MFMA_BCAST(3)
    SQ_MFMA_BCAST(4) SQ_MFMA_BCAST(5) SQ_MFMA_BCAST(6) SQ_MFMA_BCAST(7)
    SQ_MFMA_BCAST(8) SQ_MFMA_BCAST(9) SQ_MFMA_BCAST(10) SQ_MFMA_BCAST(11)
    SQ_MFMA_BCAST(12) SQ_MFMA_BCAST(13) SQ_MFMA_BCAST(14) default: break;
  }
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(av, bv, c, 4, 15, 0);
#undef SQ_MFMA_BCAST
}
// The same blocks with the A of block `abid` of each quarter broadcast within its quarter (cbsz 2: blocks 4q..4q + 3,
// lanes 16q..16q + 15, take block 4q + abid's A): each 16-lane quarter multiplies its own activations.
__device__ __forceinline__ f32x4 mfma_bcast_quarter(int abid, u32x2 a, u32x2 b, f32x4 c) {
  const i16x4 av = __builtin_bit_cast(i16x4, a), bv = __builtin_bit_cast(i16x4, b);
  switch (abid) {
    case 0: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(av, bv, c, 2, 0, 0);
    case 1: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(av, bv, c, 2, 1, 0);
    case 2: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(av, bv, c, 2, 2, 0);
    default: return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(av, bv, c, 2, 3, 0);
  }
}

// The eight codes of plane word w as exact bf16 operands 128 + q, in chunk-element order: pair p (bits 4p and
// 16 + 4p) gives operands 2p and 2p + 1. bf16 0x4300 is 128 with unit spacing, so or-ing a code into its mantissa
// makes 128 + code exactly.
__device__ __forceinline__ u32x4 code_operands(uint32_t w) {
  const uint32_t m = 0x000F000Fu, o = 0x43004300u;
  return u32x4{(w & m) | o, ((w >> 4) & m) | o, ((w >> 8) & m) | o, ((w >> 12) & m) | o};
}
// code_operands with each operand pair formed by one v_and_or_b32: the mask arrives in a scalar register and the
// exponent 0x43004300 in a vector register (make_code_constants pins them there), so the compiler selects the
// three-operand form itself; with literal constants gfx9 spends two instructions per pair (its three-operand
// encoding takes no literal).
struct CodeConstants {
  uint32_t mask, exponent;
};
__device__ __forceinline__ CodeConstants make_code_constants() {
  uint32_t mask = 0x000F000Fu, exponent = 0x43004300u;
  asm volatile("" : "+s"(mask));
  asm volatile("" : "+v"(exponent));
  return {mask, exponent};
}
__device__ __forceinline__ u32x4 code_pairs(uint32_t w, CodeConstants c) {
  return u32x4{(w & c.mask) | c.exponent, ((w >> 4) & c.mask) | c.exponent, ((w >> 8) & c.mask) | c.exponent,
               ((w >> 12) & c.mask) | c.exponent};
}
// bf16 1.0 in every operand.
__device__ __forceinline__ u32x4 ones_operand() { return u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u}; }

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}
__device__ __forceinline__ uint16_t f32_to_f16(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }

// silu(g) = g / (1 + 2^(-g log2 e)) and sigmoid(x) = 1 / (1 + 2^(-x log2 e)), the reference's forms of them
// (activation.h:8-16).
__device__ __forceinline__ float silu(float g) { return g / (1.0f + exp2f(-1.44269504089f * g)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + exp2f(-1.44269504089f * x)); }

// Epilogue of one output before its bf16 rounding, given the bf16 bits of its aux element: Residual adds it,
// UpWithGate rounds the up value to bf16 and multiplies by silu of the gate (gguf_tile.h:6-14).
template <uint32_t EP>
__device__ __forceinline__ float epilogue_bits(float v, uint32_t aux_bits) {
  if constexpr (EP == 1) v += bf16_to_f32(aux_bits);
  if constexpr (EP == 2) v = bf16_to_f32(f32_to_bf16(v)) * silu(bf16_to_f32(aux_bits));
  return v;
}
template <uint32_t EP>
__device__ __forceinline__ float epilogue(float v, const uint16_t *aux, size_t at) {
  if constexpr (EP == 0) return v;
  else return epilogue_bits<EP>(v, aux[at]);
}

// Per-format traits (QuantFormat.h:147-216). SG: groups of 32 one scale covers; UNIT: groups of 32 per meta unit;
// META: meta unit bytes; P0, P1: plane0 and plane1 bytes per group of 32; ZERO: the code offset of a format whose
// value is s (q - ZERO) (quant_formats.h QUANT_FORMAT); HALVES: one scale per 16 elements (Q6_K).
template <uint32_t FMT> struct Fmt;
template <> struct Fmt<SQ_FMT_AF4G32> { static constexpr int SG = 1, UNIT = 1, META = 4, P0 = 16, P1 = 0, ZERO = 0, HALVES = 0; };
template <> struct Fmt<SQ_FMT_AF4G64> { static constexpr int SG = 2, UNIT = 2, META = 4, P0 = 16, P1 = 0, ZERO = 0, HALVES = 0; };
template <> struct Fmt<SQ_FMT_AF4G128> { static constexpr int SG = 4, UNIT = 4, META = 4, P0 = 16, P1 = 0, ZERO = 0, HALVES = 0; };
template <> struct Fmt<SQ_FMT_AF8G64> { static constexpr int SG = 2, UNIT = 2, META = 4, P0 = 32, P1 = 0, ZERO = 0, HALVES = 0; };
template <> struct Fmt<SQ_FMT_Q4K> { static constexpr int SG = 1, UNIT = 8, META = 16, P0 = 16, P1 = 0, ZERO = 0, HALVES = 0; };
template <> struct Fmt<SQ_FMT_Q5K> { static constexpr int SG = 1, UNIT = 8, META = 16, P0 = 16, P1 = 4, ZERO = 0, HALVES = 0; };
template <> struct Fmt<SQ_FMT_Q6K> { static constexpr int SG = 1, UNIT = 8, META = 20, P0 = 16, P1 = 8, ZERO = 32, HALVES = 1; };
template <> struct Fmt<SQ_FMT_Q80> { static constexpr int SG = 1, UNIT = 1, META = 2, P0 = 32, P1 = 0, ZERO = 0, HALVES = 0; };

// fn(std::integral_constant<uint32_t, f>{}) for a format id f this build takes (a wave-uniform branch): how a
// dispatch of segments in different formats runs each workgroup's own.
template <class Fn>
__device__ __forceinline__ void with_format(uint32_t f, Fn &&fn) {
  switch (f) {
    case SQ_FMT_AF4G32: fn(std::integral_constant<uint32_t, SQ_FMT_AF4G32>{}); break;
    case SQ_FMT_AF4G64: fn(std::integral_constant<uint32_t, SQ_FMT_AF4G64>{}); break;
    case SQ_FMT_AF4G128: fn(std::integral_constant<uint32_t, SQ_FMT_AF4G128>{}); break;
    case SQ_FMT_AF8G64: fn(std::integral_constant<uint32_t, SQ_FMT_AF8G64>{}); break;
    case SQ_FMT_Q4K: fn(std::integral_constant<uint32_t, SQ_FMT_Q4K>{}); break;
    case SQ_FMT_Q5K: fn(std::integral_constant<uint32_t, SQ_FMT_Q5K>{}); break;
    case SQ_FMT_Q6K: fn(std::integral_constant<uint32_t, SQ_FMT_Q6K>{}); break;
    case SQ_FMT_Q80: fn(std::integral_constant<uint32_t, SQ_FMT_Q80>{}); break;
    default: break;   // the host passes only the formats above
  }
}

// The meta words one column needs for scale group `sg` (the meta unit that holds it): affine the (s, z) word,
// Q4_K and Q5_K the 16-byte super-block header, Q6_K its 16 int8 scales and d, Q8_0 its half d.
struct MetaWords {
  uint32_t w[5];
};
template <uint32_t FMT>
__device__ __forceinline__ MetaWords load_meta(const uint8_t *unit_row) {
  MetaWords m{};
  if constexpr (Fmt<FMT>::META == 4) {
    m.w[0] = __builtin_nontemporal_load((const uint32_t *)unit_row);
  } else if constexpr (Fmt<FMT>::META == 2) {
    m.w[0] = __builtin_nontemporal_load((const uint16_t *)unit_row);
  } else if constexpr (Fmt<FMT>::META == 20) {   // 4-byte aligned only
#pragma unroll
    for (int i = 0; i < 5; ++i) m.w[i] = __builtin_nontemporal_load((const uint32_t *)unit_row + i);
  } else {
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)unit_row);
    m.w[0] = v[0]; m.w[1] = v[1]; m.w[2] = v[2]; m.w[3] = v[3];
  }
  return m;
}

// Raw buffer loads: a resource (base and byte range, in scalar registers) over a wave-uniform base, a 32-bit vector
// offset a lane and a scalar offset, so a walk's per-group addresses cost no vector instructions; a load past the
// range reads zero. kStream marks a load as streamed once (nontemporal).
constexpr int kStream = 2;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
template <int POLICY = kStream>
__device__ __forceinline__ u32x4 buffer_b128(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, POLICY));
}
template <int POLICY = kStream>
__device__ __forceinline__ u32x2 buffer_b64(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voffset, soffset, POLICY));
}
template <int POLICY = kStream>
__device__ __forceinline__ uint32_t buffer_b32(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voffset, soffset, POLICY);
}
// load_meta through a buffer resource: the meta unit at voffset + soffset.
template <uint32_t FMT>
__device__ __forceinline__ MetaWords buffer_meta(__amdgpu_buffer_rsrc_t r, uint32_t voffset, uint32_t soffset) {
  MetaWords m{};
  if constexpr (Fmt<FMT>::META == 4) {
    m.w[0] = buffer_b32(r, voffset, soffset);
  } else if constexpr (Fmt<FMT>::META == 2) {
    m.w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, voffset, soffset, kStream);
  } else if constexpr (Fmt<FMT>::META == 20) {   // 4-byte aligned only
#pragma unroll
    for (int i = 0; i < 5; ++i) m.w[i] = buffer_b32(r, voffset, soffset + 4 * i);
  } else {
    const u32x4 v = buffer_b128(r, voffset, soffset);
    m.w[0] = v[0]; m.w[1] = v[1]; m.w[2] = v[2]; m.w[3] = v[3];
  }
  return m;
}

// The scale s and offset z of scale group `sg` of a column: value = fma(q, s, z). Affine: the group's bf16 s and z
// (quant_formats.h:614-616). Q4_K: s = d * sc and z = -(dmin * mn) of sub-block sg % 8 with the 6-bit sc, mn of
// the header's 12 scale bytes (quant_formats.h:105-118; llama.cpp's get_scale_min_k4), both products exact.
struct Coef {
  float s, z;
};
template <uint32_t FMT>
__device__ __forceinline__ Coef coef(const MetaWords &m, uint32_t sg) {
  if constexpr (FMT == SQ_FMT_Q80) {
    return {f16_to_f32(m.w[0] & 0xFFFFu), 0.0f};
  } else if constexpr (FMT == SQ_FMT_Q6K) {
    // Scale 2 (sg % 8) of the super-block's 16 (the group's first half; coef_half gives either).
    const uint32_t i = 2 * (sg & 7u);
    const float d = f16_to_f32(m.w[4] & 0xFFFFu);
    return {d * (float)(int8_t)(m.w[i >> 2] >> (8 * (i & 3))), 0.0f};
  } else if constexpr (FMT != SQ_FMT_Q4K && FMT != SQ_FMT_Q5K) {
    return {bf16_to_f32(m.w[0] & 0xFFFFu), __uint_as_float(m.w[0] & 0xFFFF0000u)};
  } else {
    const uint32_t j = sg & 7u;
    uint32_t sc, mn;
    if (j < 4) {
      const uint32_t sh = 8u * j;
      sc = (m.w[1] >> sh) & 63u;
      mn = (m.w[2] >> sh) & 63u;
    } else {
      const uint32_t sh = 8u * (j - 4), w = m.w[3] >> sh;
      sc = (w & 0xFu) | ((((m.w[1] >> sh) >> 6) & 3u) << 4);
      mn = ((w >> 4) & 0xFu) | ((((m.w[2] >> sh) >> 6) & 3u) << 4);
    }
    const float d = f16_to_f32(m.w[0] & 0xFFFFu), dmin = f16_to_f32(m.w[0] >> 16);
    return {d * (float)sc, -(dmin * (float)mn)};
  }
}
// Q6_K's scale of half h (elements 16 h .. 16 h + 15) of group sg: d * int8 scale 2 (sg % 8) + h, exact in fp32.
__device__ __forceinline__ float q6k_scale(const MetaWords &m, uint32_t sg, uint32_t h) {
  const uint32_t i = 2 * (sg & 7u) + h, k = i >> 2;
  // The word by selects, not by index: a run-time index into the words puts them in scratch memory.
  const uint32_t word = k == 0 ? m.w[0] : k == 1 ? m.w[1] : k == 2 ? m.w[2] : m.w[3];
  return f16_to_f32(m.w[4] & 0xFFFFu) * (float)(int8_t)(word >> (8 * (i & 3)));
}

// The exact bf16 operands of chunk c of a group (elements 4c..4c+3 and 16+4c..19+4c, pairs 0..3), for every
// format: `w0` the chunk's plane0 word (8-bit formats: its first word, pairs 0 and 1, and `w1` its second, pairs 2
// and 3), `high` the chunk's plane1 bits (Q5_K: byte c, bit 2p + i for element i of pair p; Q6_K: halfword c, bits
// 4p + 2i). Codes of at most 7 bits make one operand 128 + q each, in `lo`; 8-bit codes u (Q8_0's signed byte
// + 128) make two, 128 + (u & 15) in `lo` and 128 + (u >> 4) in `hi`, so sum x u = C_lo + 16 C_hi - 2176 sum x.
// With HI16 the `hi` operands are 16 (128 + (u >> 4)) = 2048 + 16 (u >> 4) instead (bf16 exponent byte 0x45, still
// exact), so that both sets can add into one accumulator: sum x u = C - 2176 sum x.
template <uint32_t FMT, bool HI16 = false>
__device__ __forceinline__ void chunk_operands(uint32_t w0, uint32_t w1, uint32_t high, CodeConstants cc, u32x4 &lo,
                                               u32x4 &hi) {
  if constexpr (Fmt<FMT>::P0 == 32) {
    const uint32_t flip = FMT == SQ_FMT_Q80 ? 0x80808080u : 0u;   // the signed byte v as u = v + 128
    const uint32_t a = w0 ^ flip, b = w1 ^ flip, nib = 0x0F0F0F0Fu, e = 0x43434343u;
    const uint32_t eh = HI16 ? 0x45454545u : e;
    const uint32_t al = a & nib, bl = b & nib, ah = (a >> 4) & nib, bh = (b >> 4) & nib;
    // Byte pair (2p', 2p' + 1) of a word into the two halves of an operand, exponent byte 0x43 above each.
    lo = u32x4{__builtin_amdgcn_perm(e, al, 0x04010400u), __builtin_amdgcn_perm(e, al, 0x04030402u),
               __builtin_amdgcn_perm(e, bl, 0x04010400u), __builtin_amdgcn_perm(e, bl, 0x04030402u)};
    hi = u32x4{__builtin_amdgcn_perm(eh, ah, 0x04010400u), __builtin_amdgcn_perm(eh, ah, 0x04030402u),
               __builtin_amdgcn_perm(eh, bh, 0x04010400u), __builtin_amdgcn_perm(eh, bh, 0x04030402u)};
  } else {
    lo = code_pairs(w0, cc);
    if constexpr (Fmt<FMT>::P1 == 4) {
      // Fifth bits: bit 2p + i of the byte to bit 4 of half i of operand p.
      const uint32_t s = ((high & 0x55u) | ((high & 0xAAu) << 15)) << 4;
#pragma unroll
      for (int p = 0; p < 4; ++p) lo[p] |= (s >> (2 * p)) & 0x00100010u;
    } else if constexpr (Fmt<FMT>::P1 == 8) {
      // High two bits: bits 4p + 2i of the halfword to bits 4..5 of half i of operand p. The spread word holds
      // half i of pair p at bits 16 i + 4p (pair 3's second half at 28..29, so it is moved into place per pair).
      const uint32_t s = (high & 0x3333u) | ((high & 0xCCCCu) << 14);
#pragma unroll
      for (int p = 0; p < 4; ++p) lo[p] |= ((s >> (4 * p)) & 0x00030003u) << 4;
    }
    (void)w1;
    (void)hi;
  }
}

}  // namespace sq::kern
