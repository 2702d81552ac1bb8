/*
 * CPU oracle for the 4-bit quantized matmul path — TEST INFRASTRUCTURE ONLY (see sq_oracle.h).
 * Every function cites the reference file:line whose semantics it restates.
 */
#define _GNU_SOURCE
#include "sq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------ formats (QuantFormat.h:147-216) */

int sqo_format_info(uint32_t fmt, sqo_format *out) {
  /* {ggml_type, block_elements, block_bytes, plane0_bytes, plane1_bytes, meta_bytes, meta_groups}:
   * q4k QuantFormat.h:159, q5k :162, q6k :163, q80 :165; af4g32/64/128 :185-187 and af8g64 :192 (ggml_type
   * QUANT_AFFINE_TYPE(bits, g)). */
  switch (fmt) {
    case SQO_FMT_Q4K: *out = (sqo_format){12, 256, 144, 16, 0, 16, 8}; return 0;
    case SQO_FMT_Q5K: *out = (sqo_format){13, 256, 176, 16, 4, 16, 8}; return 0;
    case SQO_FMT_Q6K: *out = (sqo_format){14, 256, 210, 16, 8, 20, 8}; return 0;
    case SQO_FMT_Q80: *out = (sqo_format){8, 32, 34, 32, 0, 2, 1}; return 0;
    case SQO_FMT_AF4G32: *out = (sqo_format){0x4D4C0000u | (4u << 8) | 32u, 32, 20, 16, 0, 4, 1}; return 0;
    case SQO_FMT_AF4G64: *out = (sqo_format){0x4D4C0000u | (4u << 8) | 64u, 64, 36, 16, 0, 4, 2}; return 0;
    case SQO_FMT_AF4G128: *out = (sqo_format){0x4D4C0000u | (4u << 8) | 128u, 128, 68, 16, 0, 4, 4}; return 0;
    case SQO_FMT_AF8G64: *out = (sqo_format){0x4D4C0000u | (8u << 8) | 64u, 64, 68, 32, 0, 4, 2}; return 0;
    default: return -1;
  }
}

static int affine(uint32_t fmt) {
  return fmt == SQO_FMT_AF4G32 || fmt == SQO_FMT_AF4G64 || fmt == SQO_FMT_AF4G128 || fmt == SQO_FMT_AF8G64;
}
static uint32_t affine_bits(uint32_t fmt) { return fmt == SQO_FMT_AF8G64 ? 8 : 4; }
/* Byte offsets in block_q6_K (GgufFormatReference.hpp kQ6KScales, kQ6KD; llama.cpp's ql[128] qh[64] scales[16] d). */
#define SQO_Q6K_SCALES 192u
#define SQO_Q6K_D 208u

/* quant_slot (QuantFormat.h:254): element e of a group of 32 sits at slot 8c + 2p + (e & 1). */
uint32_t sqo_quant_slot(uint32_t e) { return 8 * ((e >> 2) & 3) + 4 * (e >> 4) + (e & 3); }

/* quant_tile_index (QuantFormat.h:292-294), tiles of 64 rows. */
uint64_t sqo_tile_index(uint32_t row, uint32_t block, uint32_t blocks) {
  return ((uint64_t)(row / 64) * blocks + block) * 64 + row % 64;
}

/* ------------------------------------------------------------------ IEEE helpers */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary32 -> binary16, round to nearest even, subnormals kept (IEEE 754-2008 conversion). */
uint16_t sqo_f32_to_f16(float f) {
  const uint32_t x = f2u(f), sign = (x >> 16) & 0x8000u, exp = (x >> 23) & 0xFFu, man = x & 0x7FFFFFu;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0));
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7C00u);
  if (e <= 0) {
    const int shift = 14 - e;            /* half subnormal unit 2^-24 */
    if (shift > 24 || exp == 0) return (uint16_t)sign;
    const uint32_t full = man | 0x800000u;
    uint32_t h = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
  return (uint16_t)(sign | h);
}

float sqo_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  if (exp == 0x1F) return u2f(sign | 0x7F800000u | (man << 13));
  if (exp == 0) {
    const float v = ldexpf((float)man, -24);
    return sign ? -v : v;
  }
  return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

/* The reference's f2bf (GgufFormatReference.hpp:220-223): nearest, ties to even. */
uint16_t sqo_f32_to_bf16(float f) {
  const uint32_t v = f2u(f);
  return (uint16_t)((v + 0x7FFFu + ((v >> 16) & 1u)) >> 16);
}
float sqo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ------------------------------------------------------------------ native blocks and planes */

/* mlxNative affine branch (GgufFormatReference.hpp:236-270; loader GgufPreparation.cpp:141-193): per group of
 * `group` elements the block {bf16 s, bf16 z, the group's codes as MLX packs them}. */
int sqo_mlx_native(uint32_t fmt, uint32_t rows, uint32_t K, const uint8_t *weight, const uint16_t *scales,
                   const uint16_t *biases, uint8_t *native) {
  sqo_format f;
  if (!affine(fmt) || sqo_format_info(fmt, &f) || K % f.block_elements) return -1;
  const uint32_t bits = affine_bits(fmt), group = f.block_elements, group_bytes = group * bits / 8, groups = K / group,
                 row_codes = K * bits / 8;
  uint8_t *out = native;
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t g = 0; g < groups; ++g) {
      const size_t parameter = (size_t)r * groups + g;
      memcpy(out, &scales[parameter], 2);
      memcpy(out + 2, &biases[parameter], 2);
      memcpy(out + 4, weight + (size_t)r * row_codes + (size_t)g * group_bytes, group_bytes);
      out += f.block_bytes;
    }
  return 0;
}

/* packPairs (GgufFormatReference.hpp:332-338) / gguf_store_pairs (gguf_repack.metal:25-31): word c holds slots
 * 8c..8c+7, slot 8c + i at bit (i & 1) * 16 + 4 (i >> 1). */
static void pack_pairs(const uint8_t slots[32], uint8_t dst[16]) {
  for (uint32_t c = 0; c < 4; ++c) {
    uint32_t v = 0;
    for (uint32_t i = 0; i < 8; ++i) v |= (uint32_t)slots[8 * c + i] << ((i & 1) * 16 + 4 * (i >> 1));
    memcpy(dst + 4 * c, &v, 4);
  }
}
static void unpack_pairs(const uint8_t src[16], uint8_t slots[32]) {
  for (uint32_t c = 0; c < 4; ++c) {
    uint32_t v;
    memcpy(&v, src + 4 * c, 4);
    for (uint32_t i = 0; i < 8; ++i) slots[8 * c + i] = (uint8_t)((v >> ((i & 1) * 16 + 4 * (i >> 1))) & 15u);
  }
}

/* packBits (GgufFormatReference.hpp:331-337): the slots as a little-endian string of `bits`-bit fields. */
static void pack_bits(const uint8_t slots[32], uint32_t bits, uint8_t *dst) {
  const uint32_t per = 32 / bits;
  for (uint32_t w = 0; w < bits; ++w) {
    uint32_t v = 0;
    for (uint32_t i = 0; i < per; ++i) v |= (uint32_t)slots[w * per + i] << (bits * i);
    memcpy(dst + 4 * w, &v, 4);
  }
}
static void unpack_bits(const uint8_t *src, uint32_t bits, uint8_t slots[32]) {
  const uint32_t per = 32 / bits, mask = bits == 8 ? 0xFFu : (1u << bits) - 1;
  for (uint32_t w = 0; w < bits; ++w) {
    uint32_t v;
    memcpy(&v, src + 4 * w, 4);
    for (uint32_t i = 0; i < per; ++i) slots[w * per + i] = (uint8_t)((v >> (bits * i)) & mask);
  }
}
/* The widths of a format's low codes (plane0) and high bits (plane1). */
static uint32_t low_bits(uint32_t fmt) { return fmt == SQO_FMT_Q80 || fmt == SQO_FMT_AF8G64 ? 8 : 4; }
static uint32_t high_bits(uint32_t fmt) { return fmt == SQO_FMT_Q5K ? 1 : fmt == SQO_FMT_Q6K ? 2 : 0; }

/* scale_min_k4 (GgufFormatReference.hpp:323-326), llama.cpp's get_scale_min_k4. */
static void scale_min_k4(const uint8_t *sc, uint32_t j, uint8_t *s, uint8_t *m) {
  if (j < 4) {
    *s = sc[j] & 63;
    *m = sc[j + 4] & 63;
  } else {
    *s = (uint8_t)((sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4));
    *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
  }
}

/* The low codes, high bits (by element) and fp32 values of group g of a native row: groupPack
 * (GgufFormatReference.hpp:349-440), llama.cpp's dequantize_row_* for the GGUF formats. Affine value =
 * fma(code, s, z); Q4_K d*sc*q - dmin*mn; Q5_K the same of the 5-bit q; Q6_K d*sc*(q - 32) with a scale per 16;
 * Q8_0 d*q. Every product before the last rounding is exact in fp32. */
static void group_codes(uint32_t fmt, const sqo_format *f, const uint8_t *row, uint32_t g, uint8_t codes[32],
                        uint8_t highs[32], float vals[32]) {
  const uint8_t *blk = row + (size_t)(g * 32 / f->block_elements) * f->block_bytes;
  const uint32_t j = (g * 32 % f->block_elements) / 32;
  memset(highs, 0, 32);
  if (affine(fmt)) {
    uint16_t sb, zb;
    memcpy(&sb, blk, 2);
    memcpy(&zb, blk + 2, 2);
    const float s = sqo_bf16_to_f32(sb), z = sqo_bf16_to_f32(zb);
    for (uint32_t e = 0; e < 32; ++e) {
      const uint32_t l = 32 * j + e;
      codes[e] = affine_bits(fmt) == 8 ? blk[4 + l] : (uint8_t)((blk[4 + l / 2] >> (4 * (l % 2))) & 15u);
      vals[e] = fmaf((float)codes[e], s, z);
    }
    return;
  }
  if (fmt == SQO_FMT_Q80) {
    uint16_t d16;
    memcpy(&d16, blk, 2);
    for (uint32_t e = 0; e < 32; ++e) {
      codes[e] = blk[2 + e];
      vals[e] = sqo_f16_to_f32(d16) * (float)(int8_t)blk[2 + e];
    }
    return;
  }
  if (fmt == SQO_FMT_Q6K) {
    const uint32_t n = j / 4, r = j % 4;
    const uint8_t *ql = blk + 64 * n, *qh = blk + 128 + 32 * n;
    const int8_t *sc = (const int8_t *)(blk + SQO_Q6K_SCALES) + 8 * n;
    uint16_t d16;
    memcpy(&d16, blk + SQO_Q6K_D, 2);
    const float d = sqo_f16_to_f32(d16);
    for (uint32_t k = 0; k < 32; ++k) {
      codes[k] = (uint8_t)((ql[k + 32 * (r & 1)] >> (4 * (r >> 1))) & 15u);
      highs[k] = (uint8_t)((qh[k] >> (2 * r)) & 3u);
      vals[k] = d * (float)sc[2 * r + k / 16] * (float)((int)(codes[k] | (highs[k] << 4)) - 32);
    }
    return;
  }
  /* Q4_K and Q5_K */
  const uint8_t *q = blk + (fmt == SQO_FMT_Q5K ? 48 : 16) + (j / 2) * 32, *qh = blk + 16;
  const uint32_t sh = (j % 2) * 4;
  uint16_t d16, m16;
  memcpy(&d16, blk, 2);
  memcpy(&m16, blk + 2, 2);
  uint8_t sc, mn;
  scale_min_k4(blk + 4, j, &sc, &mn);
  /* d * sc (17 bits) and dmin * mn are exact in fp32; d * sc * q is too, so only the subtraction rounds. */
  const float s = sqo_f16_to_f32(d16) * (float)sc, m = sqo_f16_to_f32(m16) * (float)mn;
  for (uint32_t k = 0; k < 32; ++k) {
    codes[k] = (uint8_t)((q[k] >> sh) & 15u);
    if (fmt == SQO_FMT_Q5K) highs[k] = (uint8_t)((qh[k] >> j) & 1u);
    vals[k] = s * (float)(codes[k] | (highs[k] << 4)) - m;
  }
}

/* metaPack (GgufFormatReference.hpp:675-690): the block's leading meta_bytes (affine s, z; the K-quant headers;
 * Q8_0's d), but Q6_K's scales, d and two zero bytes. */
static void meta_pack(uint32_t fmt, const sqo_format *f, const uint8_t *blk, uint8_t *dst) {
  if (fmt == SQO_FMT_Q6K) {
    memcpy(dst, blk + SQO_Q6K_SCALES, 16);
    memcpy(dst + 16, blk + SQO_Q6K_D, 2);
    dst[18] = dst[19] = 0;
    return;
  }
  memcpy(dst, blk, f->meta_bytes);
}

/* repack (GgufFormatReference.hpp:701-725) restating gguf_repack_group (gguf_repack.metal:42-74): plane0
 * [N/64][G][64][plane0_bytes] (4-bit low codes pair-interleaved, 8-bit codes as bytes), plane1 [N/64][G][64]
 * [plane1_bytes] (Q5_K's fifth bits, Q6_K's high two, as bit strings over the slots), meta
 * [N/64][units][64][meta_bytes]. plane1 may be NULL for a format without one. */
int sqo_repack(uint32_t fmt, const uint8_t *native, uint32_t N, uint32_t K, uint8_t *plane0, uint8_t *plane1,
               uint8_t *meta, float *values) {
  sqo_format f;
  if (sqo_format_info(fmt, &f) || K % f.block_elements || N % 64 || (f.plane1_bytes && !plane1)) return -1;
  const uint32_t G = K / 32, units = G / f.meta_groups;
  const size_t row_bytes = (size_t)K / f.block_elements * f.block_bytes;
  for (uint32_t n = 0; n < N; ++n) {
    const uint8_t *row = native + (size_t)n * row_bytes;
    for (uint32_t g = 0; g < G; ++g) {
      uint8_t codes[32], highs[32], slots[32], hslots[32];
      float vals[32];
      group_codes(fmt, &f, row, g, codes, highs, vals);
      for (uint32_t e = 0; e < 32; ++e) {
        slots[sqo_quant_slot(e)] = codes[e];
        hslots[sqo_quant_slot(e)] = highs[e];
      }
      if (low_bits(fmt) == 4) pack_pairs(slots, plane0 + sqo_tile_index(n, g, G) * 16);
      else pack_bits(slots, 8, plane0 + sqo_tile_index(n, g, G) * f.plane0_bytes);
      if (f.plane1_bytes) pack_bits(hslots, high_bits(fmt), plane1 + sqo_tile_index(n, g, G) * f.plane1_bytes);
      if (values)
        for (uint32_t e = 0; e < 32; ++e) values[(size_t)n * K + (size_t)g * 32 + e] = vals[e];
    }
    for (uint32_t u = 0; u < units; ++u)
      meta_pack(fmt, &f, row + (size_t)u * f.block_bytes, meta + sqo_tile_index(n, u, units) * f.meta_bytes);
  }
  return 0;
}

/* Inverse of sqo_repack: native rows rebuilt from the planes (for the round-trip invariant). */
int sqo_unpack(uint32_t fmt, const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, uint32_t N,
               uint32_t K, uint8_t *native) {
  sqo_format f;
  if (sqo_format_info(fmt, &f) || K % f.block_elements || N % 64 || (f.plane1_bytes && !plane1)) return -1;
  const uint32_t G = K / 32, units = G / f.meta_groups;
  const size_t row_bytes = (size_t)K / f.block_elements * f.block_bytes;
  memset(native, 0, (size_t)N * row_bytes);
  for (uint32_t n = 0; n < N; ++n) {
    uint8_t *row = native + (size_t)n * row_bytes;
    for (uint32_t u = 0; u < units; ++u) {
      const uint8_t *m = meta + sqo_tile_index(n, u, units) * f.meta_bytes;
      uint8_t *blk = row + (size_t)u * f.block_bytes;
      if (fmt == SQO_FMT_Q6K) {
        memcpy(blk + SQO_Q6K_SCALES, m, 16);
        memcpy(blk + SQO_Q6K_D, m + 16, 2);
      } else {
        memcpy(blk, m, f.meta_bytes);
      }
    }
    for (uint32_t g = 0; g < G; ++g) {
      uint8_t slots[32], hslots[32] = {0};
      if (low_bits(fmt) == 4) unpack_pairs(plane0 + sqo_tile_index(n, g, G) * 16, slots);
      else unpack_bits(plane0 + sqo_tile_index(n, g, G) * f.plane0_bytes, 8, slots);
      if (f.plane1_bytes) unpack_bits(plane1 + sqo_tile_index(n, g, G) * f.plane1_bytes, high_bits(fmt), hslots);
      uint8_t *blk = row + (size_t)(g * 32 / f.block_elements) * f.block_bytes;
      const uint32_t j = (g * 32 % f.block_elements) / 32;
      for (uint32_t e = 0; e < 32; ++e) {
        const uint8_t code = slots[sqo_quant_slot(e)], high = hslots[sqo_quant_slot(e)];
        if (affine(fmt) && affine_bits(fmt) == 8) {
          blk[4 + 32 * j + e] = code;
        } else if (affine(fmt)) {
          const uint32_t l = 32 * j + e;
          uint8_t *byte = blk + 4 + l / 2;
          *byte = (uint8_t)((*byte & ~(0xFu << (4 * (l % 2)))) | (code << (4 * (l % 2))));
        } else if (fmt == SQO_FMT_Q80) {
          blk[2 + e] = code;
        } else if (fmt == SQO_FMT_Q6K) {
          const uint32_t nn = j / 4, r = j % 4;
          uint8_t *ql = blk + 64 * nn + e + 32 * (r & 1), *qh = blk + 128 + 32 * nn + e;
          const uint32_t sh = 4 * (r >> 1);
          *ql = (uint8_t)((*ql & ~(0xFu << sh)) | (code << sh));
          *qh = (uint8_t)((*qh & ~(3u << (2 * r))) | (high << (2 * r)));
        } else {
          uint8_t *byte = blk + (fmt == SQO_FMT_Q5K ? 48 : 16) + (j / 2) * 32 + e;
          const uint32_t sh = (j % 2) * 4;
          *byte = (uint8_t)((*byte & ~(0xFu << sh)) | (code << sh));
          if (fmt == SQO_FMT_Q5K) blk[16 + e] = (uint8_t)((blk[16 + e] & ~(1u << j)) | (high << j));
        }
      }
    }
  }
  return 0;
}

/* Values read from the planes alone: the chunk decode of quant_formats.h (codes by quant_nibble_pairs :94 and the
 * bit strings of FmtQ5K/FmtQ6K/FmtQ80 :138-235, coefficients FmtAffine :614-616, quant_k4_coef :105-118 and the Q6_K
 * and Q8_0 scales) as value = fma(q, s, z), with Q6_K's z = -32 s and Q8_0's q the signed byte; and the staged
 * fp16 rounding of gguf_staged.h:11-16. */
int sqo_plane_values(uint32_t fmt, const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, uint32_t N,
                     uint32_t K, float *values, uint16_t *halves) {
  sqo_format f;
  if (sqo_format_info(fmt, &f) || K % f.block_elements || N % 64 || (f.plane1_bytes && !plane1)) return -1;
  const uint32_t G = K / 32, units = G / f.meta_groups;
  for (uint32_t n = 0; n < N; ++n)
    for (uint32_t g = 0; g < G; ++g) {
      uint8_t slots[32], hslots[32] = {0};
      if (low_bits(fmt) == 4) unpack_pairs(plane0 + sqo_tile_index(n, g, G) * 16, slots);
      else unpack_bits(plane0 + sqo_tile_index(n, g, G) * f.plane0_bytes, 8, slots);
      if (f.plane1_bytes) unpack_bits(plane1 + sqo_tile_index(n, g, G) * f.plane1_bytes, high_bits(fmt), hslots);
      const uint8_t *m = meta + sqo_tile_index(n, g / f.meta_groups, units) * f.meta_bytes;
      for (uint32_t e = 0; e < 32; ++e) {
        const uint32_t slot = sqo_quant_slot(e);
        float s, z, q = (float)(slots[slot] | (hslots[slot] << 4));
        if (affine(fmt)) {
          uint16_t sb, zb;
          memcpy(&sb, m, 2);
          memcpy(&zb, m + 2, 2);
          s = sqo_bf16_to_f32(sb);
          z = sqo_bf16_to_f32(zb);
        } else if (fmt == SQO_FMT_Q80) {
          uint16_t d16;
          memcpy(&d16, m, 2);
          s = sqo_f16_to_f32(d16);
          z = 0.0f;
          q = (float)(int8_t)slots[slot];
        } else if (fmt == SQO_FMT_Q6K) {
          uint16_t d16;
          memcpy(&d16, m + 16, 2);
          s = sqo_f16_to_f32(d16) * (float)(int8_t)m[2 * (g % 8) + e / 16];
          z = -32.0f * s;
        } else {
          uint16_t d16, m16;
          memcpy(&d16, m, 2);
          memcpy(&m16, m + 2, 2);
          uint8_t sc, mn;
          scale_min_k4(m + 4, g % 8, &sc, &mn);
          s = sqo_f16_to_f32(d16) * (float)sc;
          z = -(sqo_f16_to_f32(m16) * (float)mn);
        }
        /* staged_linear (gguf_staged.h:11-16): a format with a code offset multiplies the exact q - Zero by s
         * (so -0.0 where q = Zero and s < 0, as GGML's d * sc * (q - 32)); the rest take fma(q, s, z). Q8_0
         * multiplies its signed value by d (QuantInt8, :40-44). */
        const float v = fmt == SQO_FMT_Q6K ? (q - 32.0f) * s : fmt == SQO_FMT_Q80 ? q * s : fmaf(q, s, z);
        const size_t at = (size_t)n * K + (size_t)g * 32 + e;
        if (values) values[at] = v;
        if (halves) halves[at] = sqo_f32_to_f16(v);
      }
    }
  return 0;
}

/* ------------------------------------------------------------------ the reference fixture */

/* MT19937 (Matsumoto & Nishimura 1998), as std::mt19937 defines it: seed by the linear recurrence with 1812433253,
 * temper with (11, 7 0x9d2c5680, 15 0xefc60000, 18). */
typedef struct {
  uint32_t mt[624];
  uint32_t idx;
} mt19937;
static void mt_seed(mt19937 *s, uint32_t seed) {
  s->mt[0] = seed;
  for (uint32_t i = 1; i < 624; ++i) s->mt[i] = 1812433253u * (s->mt[i - 1] ^ (s->mt[i - 1] >> 30)) + i;
  s->idx = 624;
}
static uint32_t mt_next(mt19937 *s) {
  if (s->idx >= 624) {
    for (uint32_t i = 0; i < 624; ++i) {
      const uint32_t y = (s->mt[i] & 0x80000000u) | (s->mt[(i + 1) % 624] & 0x7FFFFFFFu);
      s->mt[i] = s->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
    }
    s->idx = 0;
  }
  uint32_t y = s->mt[s->idx++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9D2C5680u;
  y ^= (y << 15) & 0xEFC60000u;
  y ^= y >> 18;
  return y;
}
/* A finite random half: draws until the exponent is not all ones (GgufFixtures.hpp:159-163). */
static uint16_t finite_half(mt19937 *rng) {
  uint16_t h;
  do h = (uint16_t)mt_next(rng);
  while ((h & 0x7C00u) == 0x7C00u);
  return h;
}

/* fixture (GgufFixtures.hpp:148-165) for Q4_K (through makeNative, GgufFormatReference.hpp:187-216) and the affine
 * formats: every byte one draw, then per block the half scale d and dmin (Q4_K), or the bf16 s, z made finite. */
int sqo_fixture(uint32_t fmt, uint32_t rows, uint32_t K, uint32_t seed, uint8_t *native) {
  sqo_format f;
  if (sqo_format_info(fmt, &f) || K % f.block_elements) return -1;
  mt19937 rng;
  mt_seed(&rng, seed);
  const size_t bytes = (size_t)rows * (K / f.block_elements) * f.block_bytes;
  for (size_t i = 0; i < bytes; ++i) native[i] = (uint8_t)mt_next(&rng);
  for (size_t at = 0; at < bytes; at += f.block_bytes) {
    uint8_t *blk = native + at;
    if (affine(fmt)) {
      for (uint32_t field = 0; field < 4; field += 2)
        if ((blk[field + 1] & 0x7F) == 0x7F && (blk[field] & 0x80)) blk[field + 1] ^= 1;
    } else {
      /* makeNative: the half d (Q6_K's at its end), and Q4_K's and Q5_K's dmin after it. */
      const uint16_t d = finite_half(&rng);
      memcpy(blk + (fmt == SQO_FMT_Q6K ? SQO_Q6K_D : 0), &d, 2);
      if (fmt == SQO_FMT_Q4K || fmt == SQO_FMT_Q5K) {
        const uint16_t m = finite_half(&rng);
        memcpy(blk + 2, &m, 2);
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ fp64 projection and bounds */

typedef struct {
  uint32_t M, N, K;
  const uint16_t *x;
  const float *w;
  const uint16_t *halves;
  double *value, *magnitude, *inputs, *largest;
  float *out32;
  uint32_t n_begin, n_end;
} project_job;

/* dot (GgufFormatReference.hpp:758-769): the fp64 value, sum |x w|, sum |x| and max |w|. */
static void *project_f64_worker(void *arg) {
  const project_job *j = (const project_job *)arg;
  double *xf = (double *)malloc(sizeof(double) * j->K);
  for (uint32_t m = 0; m < j->M; ++m) {
    for (uint32_t k = 0; k < j->K; ++k) xf[k] = sqo_bf16_to_f32(j->x[(size_t)m * j->K + k]);
    for (uint32_t n = j->n_begin; n < j->n_end; ++n) {
      const float *w = j->w + (size_t)n * j->K;
      double v = 0, mag = 0, in = 0, big = 0;
      for (uint32_t k = 0; k < j->K; ++k) {
        v += xf[k] * w[k];
        mag += fabs(xf[k] * w[k]);
        in += fabs(xf[k]);
        if (fabs((double)w[k]) > big) big = fabs((double)w[k]);
      }
      const size_t at = (size_t)m * j->N + n;
      j->value[at] = v;
      if (j->magnitude) j->magnitude[at] = mag;
      if (j->inputs) j->inputs[at] = in;
      if (j->largest) j->largest[at] = big;
    }
  }
  free(xf);
  return NULL;
}

static void *project_staged_worker(void *arg) {
  const project_job *j = (const project_job *)arg;
  float *xf = (float *)malloc(sizeof(float) * j->K);
  for (uint32_t m = 0; m < j->M; ++m) {
    for (uint32_t k = 0; k < j->K; ++k) xf[k] = sqo_bf16_to_f32(j->x[(size_t)m * j->K + k]);
    for (uint32_t n = j->n_begin; n < j->n_end; ++n) {
      const uint16_t *h = j->halves + (size_t)n * j->K;
      float acc = 0.0f;
      /* Each product of a bf16 input and a half weight is exact in fp32; only the additions round. */
      for (uint32_t k = 0; k < j->K; ++k) acc = acc + xf[k] * sqo_f16_to_f32(h[k]);
      j->out32[(size_t)m * j->N + n] = acc;
    }
  }
  free(xf);
  return NULL;
}

static void run_jobs(project_job *base, uint32_t N, int threads, void *(*fn)(void *)) {
  if (threads < 1) threads = 1;
  if ((uint32_t)threads > N) threads = (int)N;
  pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  project_job *jobs = (project_job *)malloc(sizeof(project_job) * (size_t)threads);
  for (int t = 0; t < threads; ++t) {
    jobs[t] = *base;
    jobs[t].n_begin = (uint32_t)((uint64_t)N * t / threads);
    jobs[t].n_end = (uint32_t)((uint64_t)N * (t + 1) / threads);
    pthread_create(&tid[t], NULL, fn, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
}

void sqo_project_f64(uint32_t M, uint32_t N, uint32_t K, const uint16_t *x, const float *w, double *value,
                     double *magnitude, double *inputs, double *largest, int threads) {
  project_job job = {M, N, K, x, w, NULL, value, magnitude, inputs, largest, NULL, 0, N};
  run_jobs(&job, N, threads, project_f64_worker);
}

/* projectionBound (GgufFormatReference.hpp:794-797). */
double sqo_projection_bound(double magnitude, double inputs, double largest, int staged) {
  const double accumulation = ldexp(inputs * largest, -16);
  return staged ? accumulation + ldexp(magnitude, -11) + ldexp(inputs, -25) : accumulation;
}

void sqo_project_staged_f32(uint32_t M, uint32_t N, uint32_t K, const uint16_t *x, const uint16_t *halves,
                            float *out, int threads) {
  project_job job = {M, N, K, x, NULL, halves, NULL, NULL, NULL, NULL, out, 0, N};
  run_jobs(&job, N, threads, project_staged_worker);
}

/* ------------------------------------------------------------------ CPU baseline */

typedef struct {
  uint32_t fmt, M, N, K;
  const float *xf;
  const uint8_t *plane0, *meta;
  uint16_t *out;
  uint32_t n_begin, n_end;
} cpu_job;

/* The 32 fp32 values of group g of column n straight from the planes, as sqo_plane_values decodes them. */
static inline void cpu_group(uint32_t fmt, const uint8_t *plane0, const uint8_t *meta, uint32_t G, uint32_t units,
                             uint32_t meta_groups, uint32_t meta_bytes, uint32_t n, uint32_t g, float w[32]) {
  const uint8_t *p = plane0 + sqo_tile_index(n, g, G) * 16;
  const uint8_t *m = meta + sqo_tile_index(n, g / meta_groups, units) * meta_bytes;
  float s, z;
  if (fmt != SQO_FMT_Q4K) {
    uint16_t sb, zb;
    memcpy(&sb, m, 2);
    memcpy(&zb, m + 2, 2);
    s = sqo_bf16_to_f32(sb);
    z = sqo_bf16_to_f32(zb);
  } else {
    uint16_t d16, m16;
    memcpy(&d16, m, 2);
    memcpy(&m16, m + 2, 2);
    uint8_t sc, mn;
    scale_min_k4(m + 4, g % 8, &sc, &mn);
    s = sqo_f16_to_f32(d16) * (float)sc;
    z = -(sqo_f16_to_f32(m16) * (float)mn);
  }
  /* Word c, pair p: element 16(p >> 1) + 4c + 2(p & 1) at bits 4p, its neighbour at 16 + 4p. */
  for (uint32_t c = 0; c < 4; ++c) {
    uint32_t v;
    memcpy(&v, p + 4 * c, 4);
    for (uint32_t pr = 0; pr < 4; ++pr) {
      const uint32_t e0 = 16 * (pr >> 1) + 4 * c + 2 * (pr & 1);
      w[e0] = fmaf((float)((v >> (4 * pr)) & 15u), s, z);
      w[e0 + 1] = fmaf((float)((v >> (16 + 4 * pr)) & 15u), s, z);
    }
  }
}

static void *cpu_worker(void *arg) {
  const cpu_job *j = (const cpu_job *)arg;
  sqo_format f;
  sqo_format_info(j->fmt, &f);
  const uint32_t G = j->K / 32, units = G / f.meta_groups;
  float *acc = (float *)malloc(sizeof(float) * j->M);
  float w[32];
  for (uint32_t n = j->n_begin; n < j->n_end; ++n) {
    for (uint32_t m = 0; m < j->M; ++m) acc[m] = 0.0f;
    for (uint32_t g = 0; g < G; ++g) {
      cpu_group(j->fmt, j->plane0, j->meta, G, units, f.meta_groups, f.meta_bytes, n, g, w);
      for (uint32_t m = 0; m < j->M; ++m) {
        const float *x = j->xf + (size_t)m * j->K + (size_t)g * 32;
        float s = 0.0f;
        for (uint32_t e = 0; e < 32; ++e) s += x[e] * w[e];
        acc[m] += s;
      }
    }
    for (uint32_t m = 0; m < j->M; ++m) j->out[(size_t)m * j->N + n] = sqo_f32_to_bf16(acc[m]);
  }
  free(acc);
  return NULL;
}

double sqo_cpu_matmul(uint32_t fmt, uint32_t M, uint32_t N, uint32_t K, const uint16_t *x, const uint8_t *plane0,
                      const uint8_t *meta, uint16_t *out, int threads) {
  /* The CPU baseline runs the 4-bit formats of the headline workloads. */
  if (fmt != SQO_FMT_Q4K && fmt != SQO_FMT_AF4G32 && fmt != SQO_FMT_AF4G64 && fmt != SQO_FMT_AF4G128) return -1.0;
  struct timespec t0, t1;
  clock_gettime(CLOCK_MONOTONIC, &t0);
  float *xf = (float *)malloc(sizeof(float) * (size_t)M * K);
  for (size_t i = 0; i < (size_t)M * K; ++i) xf[i] = sqo_bf16_to_f32(x[i]);
  if (threads < 1) threads = 1;
  if ((uint32_t)threads > N) threads = (int)N;
  pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  cpu_job *jobs = (cpu_job *)malloc(sizeof(cpu_job) * (size_t)threads);
  for (int t = 0; t < threads; ++t) {
    jobs[t] = (cpu_job){fmt, M, N, K, xf, plane0, meta, out,
                        (uint32_t)((uint64_t)N * t / threads), (uint32_t)((uint64_t)N * (t + 1) / threads)};
    pthread_create(&tid[t], NULL, cpu_worker, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
  free(xf);
  clock_gettime(CLOCK_MONOTONIC, &t1);
  return (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
}

/* ------------------------------------------------------------------ MoE */

static double sqo_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

/* moe_route_select (moe.metal:23-104): rank by rank, the highest remaining score wins and the lower expert id among
 * equal scores. A selected expert's score becomes -inf. Scores compare as the kernel's strict `score > best` from a
 * best of -inf does: a NaN never wins, and when no score above -inf is left expert 0 wins (moe.metal:77-93, where
 * every lane then offers its first slot and the lowest lane is expert 0), so an all-NaN row selects expert 0 k
 * times. Softmax (router 0): weight of rank r = exp(s_r - s_0) / sum_j exp(s_j - s_0) over the selected k, the s the
 * ranks' winning scores; SigmoidNormalized (router 1): sigmoid(s_r) / (sum_j sigmoid(s_j) + 1e-20). In fp64. Rows
 * of `per_row` routes, the routed top_k first (the caller fills the shared slices' routes after them). */
void sqo_route_select(uint32_t rows, uint32_t experts, uint32_t top_k, uint32_t router, uint32_t per_row,
                      const float *scores, uint32_t *selected, double *weights) {
  float *left = (float *)malloc(sizeof(float) * experts);
  double *ordered = (double *)malloc(sizeof(double) * (top_k ? top_k : 1));
  for (uint32_t r = 0; r < rows; ++r) {
    uint32_t *sel = selected + (size_t)r * per_row;
    double *w = weights + (size_t)r * per_row;
    memcpy(left, scores + (size_t)r * experts, sizeof(float) * experts);
    for (uint32_t rank = 0; rank < top_k; ++rank) {
      float top = -INFINITY;
      uint32_t best = 0;
      for (uint32_t e = 0; e < experts; ++e)
        if (left[e] > top) top = left[e], best = e;   /* strict: the first (lowest) id of the top score */
      left[best] = -INFINITY;
      sel[rank] = best;
      ordered[rank] = top;
    }
    double denominator = 0;
    for (uint32_t rank = 0; rank < top_k; ++rank)
      denominator += router ? sqo_sigmoid(ordered[rank]) : exp(ordered[rank] - ordered[0]);
    if (router) denominator += 1e-20;
    for (uint32_t rank = 0; rank < top_k; ++rank)
      w[rank] = (router ? sqo_sigmoid(ordered[rank]) : exp(ordered[rank] - ordered[0])) / denominator;
  }
  free(ordered);
  free(left);
}

/* moe_group_routes_phase (moe.metal:184-278): count per expert, exclusive prefix of the experts' tiles in expert
 * order, then each expert's routes in route order over its tiles; the `shared` slices' tiles follow, slice after
 * slice, each holding every row in order. Rows hold top_k + shared routes, the routed ones first. With verify_rows
 * (the verified grouping, moe.metal:164-173 moe_unverified_route): a routed route of row r is left out when
 * r % lane_rows >= verify_rows[r / lane_rows]; it takes no grouped row and its route row is ~0u. The shared slices
 * route every row either way. */
uint32_t sqo_group_routes(uint32_t rows, uint32_t top_k, uint32_t shared, uint32_t experts, uint32_t tile_rows,
                          const uint32_t *selected, const uint32_t *verify_rows, uint32_t lane_rows, uint32_t *tiles,
                          uint32_t *grouped_routes, uint32_t *route_rows) {
  const uint32_t per_row = top_k + shared, routes = rows * per_row;
  uint32_t *count = (uint32_t *)calloc(experts, sizeof(uint32_t));
  uint32_t *offset = (uint32_t *)calloc(experts, sizeof(uint32_t));
  uint32_t *cursor = (uint32_t *)calloc(experts, sizeof(uint32_t));
#define SQO_UNVERIFIED(r) (verify_rows && ((r) / per_row) % lane_rows >= verify_rows[((r) / per_row) / lane_rows])
  for (uint32_t r = 0; r < routes; ++r)
    if (r % per_row < top_k && !SQO_UNVERIFIED(r)) ++count[selected[r]];
  uint32_t total = 0;
  for (uint32_t e = 0; e < experts; ++e) {
    offset[e] = total;
    const uint32_t t = (count[e] + tile_rows - 1) / tile_rows;
    for (uint32_t i = 0; i < t; ++i) {
      tiles[2 * (total + i)] = e;
      tiles[2 * (total + i) + 1] = count[e] - i * tile_rows < tile_rows ? count[e] - i * tile_rows : tile_rows;
    }
    total += t;
  }
  const uint32_t shared_tiles = (rows + tile_rows - 1) / tile_rows;
  for (uint32_t i = 0; i < (total + shared * shared_tiles) * tile_rows; ++i) grouped_routes[i] = ~0u;
  for (uint32_t r = 0; r < routes; ++r) {
    if (r % per_row >= top_k) continue;
    if (SQO_UNVERIFIED(r)) {
      route_rows[r] = ~0u;
      continue;
    }
    const uint32_t e = selected[r], row = offset[e] * tile_rows + cursor[e]++;
    grouped_routes[row] = r;
    route_rows[r] = row;
  }
  for (uint32_t slice = 0; slice < shared; ++slice) {
    for (uint32_t t = 0; t < shared_tiles; ++t) {
      const uint32_t at = total + slice * shared_tiles + t;
      tiles[2 * at] = experts + slice;
      tiles[2 * at + 1] = rows - t * tile_rows < tile_rows ? rows - t * tile_rows : tile_rows;
    }
    for (uint32_t row = 0; row < rows; ++row) {
      const uint32_t r = row * per_row + top_k + slice, g = (total + slice * shared_tiles) * tile_rows + row;
      grouped_routes[g] = r;
      route_rows[r] = g;
    }
  }
#undef SQO_UNVERIFIED
  total += shared * shared_tiles;
  free(count);
  free(offset);
  free(cursor);
  return total;
}
