// Load-time repack into the plane layout and the dequantisation kernel the tests read the weights through.
//
// Repack (reference: gguf_repack_group's affine, Q4_K, Q5_K, Q6_K and Q8_0 branches, kernels/shared/gguf_repack.metal
// :24-74, and kernel gguf_repack :232-238): one thread per (row, group of 32) writes the group's plane units, element
// e's code at slot quant_slot(e), and the first group of each meta unit copies the unit's meta bytes. The MLX repack
// reads MLX's own tensors (uint32 codes, bf16 scales and biases, model/GgufPreparation.cpp:141-193 builds the native
// block from them) and writes the same planes without the staging copy.
//
// Dequant (reference: gguf_test_dequant_<fmt>, dev/tests/engine/gguf_dequant_test.metal:5-21): every weight's fp32
// value fma(q, s, z) and its fp16 rounding, the staged tile's weight (kernels/common/gguf_staged.h:11-16).
#include "device.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

// Word c of a 4-bit plane unit holds slots 8c..8c+7, slot 8c + i at bit (i & 1) * 16 + 4 (i >> 1).
__device__ __forceinline__ void store_pairs(const uint8_t codes[32], uint8_t *dst) {
  uint32_t word[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (uint32_t e = 0; e < 32; ++e) {
    const uint32_t slot = sq_quant_slot(e), c = slot >> 3, i = slot & 7u;
    word[c] |= (uint32_t)codes[e] << ((i & 1u) * 16u + 4u * (i >> 1));
  }
  *(u32x4 *)dst = u32x4{word[0], word[1], word[2], word[3]};
}
// Every other field is a little-endian string of BITS-bit fields over the slots (QuantFormat.h:27-31): 8-bit codes
// one byte a slot, Q5_K's fifth bits one bit a slot, Q6_K's high bits two bits a slot.
template <uint32_t BITS>
__device__ __forceinline__ void store_bits(const uint8_t codes[32], uint8_t *dst) {
  uint32_t word[BITS] = {};
#pragma unroll
  for (uint32_t e = 0; e < 32; ++e) {
    const uint32_t slot = sq_quant_slot(e);
    word[slot * BITS / 32] |= (uint32_t)codes[e] << ((slot * BITS) % 32);
  }
#pragma unroll
  for (uint32_t w = 0; w < BITS; ++w) ((uint32_t *)dst)[w] = word[w];
}

// Group g of row n (native row `row`, G groups a row) of format fmt: the group's low codes into its plane0 unit, its
// high bits into its plane1 unit, and the first group of each meta unit copies the unit's meta (gguf_repack_group,
// gguf_repack.metal:42-74, and metaPack's Q6_K arrangement: its 16 int8 scales, d and two zero bytes). plane0,
// plane1 and meta point at the tensor's planes.
__device__ void repack_group(const uint8_t *row, uint32_t fmt, uint32_t G, uint32_t n, uint32_t g, uint8_t *plane0,
                             uint8_t *plane1, uint8_t *meta_plane) {
  const SqQuantFormat f = sq_format(fmt);
  const uint32_t b = g / f.meta_groups, jj = g % f.meta_groups;
  const uint8_t *blk = row + (size_t)b * f.block_bytes;
  uint8_t codes[32], highs[32];
  uint8_t *unit0 = plane0 + sq_tile_index(n, g, G) * f.plane0_bytes;
  uint8_t *unit1 = plane1 + sq_tile_index(n, g, G) * f.plane1_bytes;
  if (fmt == SQ_FMT_AF8G64) {
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) codes[e] = blk[4 + 32u * jj + e];
    store_bits<8>(codes, unit0);
  } else if (sq_affine_format(fmt)) {
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) {
      const uint32_t l = 32u * jj + e;
      codes[e] = (blk[4 + l / 2] >> (4u * (l & 1u))) & 15u;
    }
    store_pairs(codes, unit0);
  } else if (fmt == SQ_FMT_Q80) {
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) codes[e] = blk[2 + e];
    store_bits<8>(codes, unit0);
  } else if (fmt == SQ_FMT_Q6K) {
    const uint32_t h = jj / 4, r = jj % 4;
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) {
      codes[e] = (blk[64 * h + e + 32 * (r & 1u)] >> (4u * (r >> 1))) & 15u;
      highs[e] = (blk[128 + 32 * h + e] >> (2u * r)) & 3u;
    }
    store_pairs(codes, unit0);
    store_bits<2>(highs, unit1);
  } else {   // Q4_K, Q5_K
    const uint32_t q = fmt == SQ_FMT_Q5K ? 48u : 16u;
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) codes[e] = (blk[q + (jj / 2) * 32 + e] >> (4u * (jj & 1u))) & 15u;
    store_pairs(codes, unit0);
    if (fmt == SQ_FMT_Q5K) {
#pragma unroll
      for (uint32_t e = 0; e < 32; ++e) highs[e] = (blk[16 + e] >> jj) & 1u;
      store_bits<1>(highs, unit1);
    }
  }
  if (jj == 0) {
    uint8_t *meta = meta_plane + sq_tile_index(n, b, G / f.meta_groups) * f.meta_bytes;
    if (fmt == SQ_FMT_Q6K) {
      for (uint32_t i = 0; i < 16; ++i) meta[i] = blk[SQ_Q6K_SCALES + i];
      meta[16] = blk[SQ_Q6K_D];
      meta[17] = blk[SQ_Q6K_D + 1];
      meta[18] = meta[19] = 0;
    } else {
      for (uint32_t i = 0; i < f.meta_bytes; ++i) meta[i] = blk[i];
    }
  }
}

// One thread a (row, group of 32) of one tensor (kernel gguf_repack, gguf_repack.metal:232-238).
__global__ void repack_kernel(const uint8_t *src, uint8_t *dst, SqGgufRepackParams p) {
  const uint32_t G = p.input_size / 32;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)p.rows * G) return;
  const uint32_t n = (uint32_t)(t / G), g = (uint32_t)(t % G);
  repack_group(src + (size_t)n * p.src_row_bytes, p.fmt, G, n, g, dst, dst + p.dst_plane1, dst + p.dst_meta);
}

// Streamed experts into their slots (moe_expert_load, gguf_repack.metal:239-257): workgroup (x, y, z) repacks 256
// (row, group of 32) pairs of projection z of job y from staging + sources[3 y + z] on into the planes of slot
// slots[y] of the arena, projection z's plane i at planes[i] + slot * slot_bytes[i]. `grid` holds the three
// workgroup counts the dispatch runs (the reference's indirect grid, written by an earlier dispatch): the launch
// covers the largest grid and workgroups past grid's return. A job whose source rows or slot planes would fall
// outside the staging or the arena writes nothing.
__global__ __launch_bounds__(SQ_MOE_EXPERT_LOAD_THREADS) void expert_load_kernel(
    const uint8_t *staging, uint64_t staging_bytes, uint8_t *arena, uint64_t arena_bytes, const uint32_t *slots,
    const uint64_t *sources, SqMoeExpertLoadParams p, const uint32_t *grid) {
  if (blockIdx.x >= grid[0] || blockIdx.y >= grid[1] || blockIdx.z >= grid[2]) return;
  const SqMoeExpertLoadProjection &q = p.projections[blockIdx.z];
  const uint32_t G = q.columns / 32;
  const uint64_t t = (uint64_t)blockIdx.x * SQ_MOE_EXPERT_LOAD_THREADS + threadIdx.x;
  if (!q.rows || t >= (uint64_t)q.rows * G) return;
  const uint32_t n = (uint32_t)(t / G), g = (uint32_t)(t % G);
  const uint64_t slot = slots[blockIdx.y], source = sources[3 * (uint64_t)blockIdx.y + blockIdx.z];
  const SqQuantFormat f = sq_format(q.format);
  const uint64_t row_blocks = (uint64_t)q.columns / f.block_elements * f.block_bytes;
  const uint64_t need[3] = {(uint64_t)q.rows * G * f.plane0_bytes, (uint64_t)q.rows * G * f.plane1_bytes,
                            (uint64_t)q.rows * (G / f.meta_groups) * f.meta_bytes};
  if (source > staging_bytes || (uint64_t)(q.rows - 1) * q.row_bytes + row_blocks > staging_bytes - source) return;
#pragma unroll
  for (int i = 0; i < 3; ++i)
    if (need[i] && (q.planes[i] > arena_bytes || slot > (arena_bytes - q.planes[i]) / max(q.slot_bytes[i], (uint64_t)1) ||
                    q.planes[i] + slot * q.slot_bytes[i] + need[i] > arena_bytes))
      return;
  repack_group(staging + source + (uint64_t)n * q.row_bytes, q.format, G, n, g, arena + q.planes[0] + slot * q.slot_bytes[0],
               arena + q.planes[1] + slot * q.slot_bytes[1], arena + q.planes[2] + slot * q.slot_bytes[2]);
}

// MLX's own tensors: row n's codes a little-endian string of BITS-bit codes (group g of 32 is BITS words of the
// row), bf16 scales and biases per group of the format.
__global__ void mlx_repack_kernel(uint32_t fmt, const uint32_t *weight, const uint16_t *scales,
                                  const uint16_t *biases, uint32_t rows, uint32_t K, uint8_t *plane0, uint8_t *meta) {
  const uint32_t G = K / 32;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)rows * G) return;
  const uint32_t n = (uint32_t)(t / G), g = (uint32_t)(t % G);
  const SqQuantFormat f = sq_format(fmt);
  uint8_t codes[32];
  if (fmt == SQ_FMT_AF8G64) {
    const u32x4 *w = (const u32x4 *)(weight + (size_t)n * (K / 4) + (size_t)g * 8);
    const u32x4 lo = w[0], hi = w[1];
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) codes[e] = ((e < 16 ? lo[e >> 2] : hi[(e - 16) >> 2]) >> (8u * (e & 3u))) & 0xFFu;
    store_bits<8>(codes, plane0 + sq_tile_index(n, g, G) * 32);
  } else {
    const u32x4 w = *(const u32x4 *)(weight + (size_t)n * (K / 8) + (size_t)g * 4);
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) codes[e] = (w[e >> 3] >> (4u * (e & 7u))) & 15u;
    store_pairs(codes, plane0 + sq_tile_index(n, g, G) * 16);
  }
  if (g % f.meta_groups == 0) {
    const uint32_t groups = K / f.block_elements, b = g / f.meta_groups;
    const size_t parameter = (size_t)n * groups + b;
    *(uint32_t *)(meta + sq_tile_index(n, b, groups) * 4) = (uint32_t)scales[parameter] |
                                                            ((uint32_t)biases[parameter] << 16);
  }
}

// Element e's code (low bits from plane0, high bits from plane1) of a group's units.
template <uint32_t FMT>
__device__ __forceinline__ uint32_t group_code(const uint8_t *unit0, const uint8_t *unit1, uint32_t e) {
  using F = Fmt<FMT>;
  const uint32_t slot = sq_quant_slot(e);
  uint32_t q;
  if constexpr (F::P0 == 32) {
    q = unit0[slot];
  } else {
    const uint32_t word = ((const uint32_t *)unit0)[slot >> 3], i = slot & 7u;
    q = (word >> ((i & 1u) * 16u + 4u * (i >> 1))) & 15u;
  }
  if constexpr (F::P1 == 4) q |= ((((const uint32_t *)unit1)[0] >> slot) & 1u) << 4;
  if constexpr (F::P1 == 8) q |= ((((const uint32_t *)unit1)[slot >> 4] >> (2 * (slot & 15u))) & 3u) << 4;
  return q;
}

// Every weight's fp32 value and its fp16 rounding, as the staged tile decodes it (staged_linear,
// gguf_staged.h:11-16, and QuantInt8 :40-44): fma(q, s, z), but s (q - 32) for Q6_K and s q of the signed byte for
// Q8_0, so signed zeros come out as the reference's.
template <uint32_t FMT>
__global__ void dequant_kernel(const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, uint32_t N,
                               uint32_t K, float *values, uint16_t *halves) {
  using F = Fmt<FMT>;
  const uint32_t G = K / 32, units = G / F::UNIT;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)N * G) return;
  const uint32_t n = (uint32_t)(t / G), g = (uint32_t)(t % G);
  const uint8_t *unit0 = plane0 + sq_tile_index(n, g, G) * F::P0;
  const uint8_t *unit1 = F::P1 ? plane1 + sq_tile_index(n, g, G) * F::P1 : nullptr;
  const MetaWords m = load_meta<FMT>(meta + sq_tile_index(n, g / F::UNIT, units) * F::META);
  const Coef k = coef<FMT>(m, g / F::SG);
  const size_t base = (size_t)n * K + (size_t)g * 32;
#pragma unroll 4
  for (uint32_t e = 0; e < 32; ++e) {
    const uint32_t q = group_code<FMT>(unit0, unit1, e);
    float v;
    if constexpr (FMT == SQ_FMT_Q6K) v = ((float)q - 32.0f) * q6k_scale(m, g, e >> 4);
    else if constexpr (FMT == SQ_FMT_Q80) v = (float)(int8_t)q * k.s;
    else v = fmaf((float)q, k.s, k.z);
    if (values) values[base + e] = v;
    if (halves) halves[base + e] = f32_to_f16(v);
  }
}

}  // namespace

hipError_t launch_expert_load(const uint8_t *staging, uint64_t staging_bytes, uint8_t *arena, uint64_t arena_bytes,
                              const uint32_t *slots, const uint64_t *sources, const SqMoeExpertLoadParams &p,
                              uint32_t groups, uint32_t jobs, const uint32_t *grid, hipStream_t stream) {
  if (!groups || !jobs) return hipSuccess;
  hipLaunchKernelGGL(expert_load_kernel, dim3(groups, jobs, 3), dim3(SQ_MOE_EXPERT_LOAD_THREADS), 0, stream, staging,
                     staging_bytes, arena, arena_bytes, slots, sources, p, grid);
  return hipGetLastError();
}

hipError_t launch_repack(const uint8_t *src, uint8_t *dst, const SqGgufRepackParams &p, hipStream_t stream) {
  const uint64_t threads = (uint64_t)p.rows * (p.input_size / 32);
  hipLaunchKernelGGL(repack_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, stream, src, dst, p);
  return hipGetLastError();
}

hipError_t launch_mlx_repack(uint32_t fmt, const uint32_t *weight, const uint16_t *scales, const uint16_t *biases,
                             uint32_t rows, uint32_t K, uint8_t *plane0, uint8_t *meta, hipStream_t stream) {
  const uint64_t threads = (uint64_t)rows * (K / 32);
  hipLaunchKernelGGL(mlx_repack_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, stream, fmt, weight,
                     scales, biases, rows, K, plane0, meta);
  return hipGetLastError();
}

hipError_t launch_dequant(uint32_t fmt, const uint8_t *plane0, const uint8_t *plane1, const uint8_t *meta, uint32_t N,
                          uint32_t K, float *values, uint16_t *halves, hipStream_t stream) {
  const uint64_t threads = (uint64_t)N * (K / 32);
  const dim3 grid((uint32_t)((threads + 255) / 256)), block(256);
#define SQ_DEQUANT(F) \
  case F: hipLaunchKernelGGL(dequant_kernel<F>, grid, block, 0, stream, plane0, plane1, meta, N, K, values, halves); break;
  switch (fmt) {
    SQ_DEQUANT(SQ_FMT_AF4G32) SQ_DEQUANT(SQ_FMT_AF4G64) SQ_DEQUANT(SQ_FMT_AF4G128) SQ_DEQUANT(SQ_FMT_AF8G64)
    SQ_DEQUANT(SQ_FMT_Q4K) SQ_DEQUANT(SQ_FMT_Q5K) SQ_DEQUANT(SQ_FMT_Q6K) SQ_DEQUANT(SQ_FMT_Q80)
    default: return hipErrorInvalidValue;
  }
#undef SQ_DEQUANT
  return hipGetLastError();
}

}  // namespace sq::kern
