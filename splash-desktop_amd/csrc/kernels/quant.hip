// Load-time repack into the plane layout and the dequantisation kernel the tests read the weights through.
//
// Repack (reference: gguf_repack_group's affine and Q4_K branches, kernels/shared/gguf_repack.metal:24-74, and
// kernel gguf_repack :232-238): one thread per (row, group of 32) writes the group's 16-byte plane unit, element e's
// code at slot quant_slot(e), and the first group of each meta unit copies the unit's meta bytes. The MLX repack
// reads MLX's own tensors (uint32 codes, bf16 scales and biases, model/GgufPreparation.cpp:141-193 builds the native
// block from them) and writes the same planes without the staging copy.
//
// Dequant (reference: gguf_test_dequant_<fmt>, dev/tests/engine/gguf_dequant_test.metal:5-21): every weight's fp32
// value fma(q, s, z) and its fp16 rounding, the staged tile's weight (kernels/common/gguf_staged.h:11-16).
#include "device.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

// Word c of a plane unit holds slots 8c..8c+7, slot 8c + i at bit (i & 1) * 16 + 4 (i >> 1).
__device__ __forceinline__ void store_pairs(const uint8_t codes[32], uint8_t *dst) {
  uint32_t word[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (uint32_t e = 0; e < 32; ++e) {
    const uint32_t slot = sq_quant_slot(e), c = slot >> 3, i = slot & 7u;
    word[c] |= (uint32_t)codes[e] << ((i & 1u) * 16u + 4u * (i >> 1));
  }
  *(u32x4 *)dst = u32x4{word[0], word[1], word[2], word[3]};
}

__global__ void repack_kernel(const uint8_t *src, uint8_t *dst, SqGgufRepackParams p) {
  const uint32_t G = p.input_size / 32;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)p.rows * G) return;
  const uint32_t n = (uint32_t)(t / G), g = (uint32_t)(t % G);
  const SqQuantFormat f = sq_format(p.fmt);
  const uint32_t b = g / f.meta_groups, jj = g % f.meta_groups;
  const uint8_t *blk = src + (size_t)n * p.src_row_bytes + (size_t)b * f.block_bytes;
  uint8_t codes[32];
  if (sq_affine_format(p.fmt)) {
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) {
      const uint32_t l = 32u * jj + e;
      codes[e] = (blk[4 + l / 2] >> (4u * (l & 1u))) & 15u;
    }
  } else {
#pragma unroll
    for (uint32_t e = 0; e < 32; ++e) codes[e] = (blk[16 + (jj / 2) * 32 + e] >> (4u * (jj & 1u))) & 15u;
  }
  store_pairs(codes, dst + sq_tile_index(n, g, G) * 16);
  if (jj == 0) {
    uint8_t *meta = dst + p.dst_meta + sq_tile_index(n, b, G / f.meta_groups) * f.meta_bytes;
    for (uint32_t i = 0; i < f.meta_bytes; ++i) meta[i] = blk[i];
  }
}

__global__ void mlx_repack_kernel(uint32_t fmt, const uint32_t *weight, const uint16_t *scales,
                                  const uint16_t *biases, uint32_t rows, uint32_t K, uint8_t *plane0, uint8_t *meta) {
  const uint32_t G = K / 32;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)rows * G) return;
  const uint32_t n = (uint32_t)(t / G), g = (uint32_t)(t % G);
  const SqQuantFormat f = sq_format(fmt);
  // Row n's codes are a little-endian string of 4-bit codes: group g is words 4g..4g+3 of the row.
  const u32x4 w = *(const u32x4 *)(weight + (size_t)n * (K / 8) + (size_t)g * 4);
  uint8_t codes[32];
#pragma unroll
  for (uint32_t e = 0; e < 32; ++e) codes[e] = (w[e >> 3] >> (4u * (e & 7u))) & 15u;
  store_pairs(codes, plane0 + sq_tile_index(n, g, G) * 16);
  if (g % f.meta_groups == 0) {
    const uint32_t groups = K / f.block_elements, b = g / f.meta_groups;
    const size_t parameter = (size_t)n * groups + b;
    *(uint32_t *)(meta + sq_tile_index(n, b, groups) * 4) = (uint32_t)scales[parameter] |
                                                            ((uint32_t)biases[parameter] << 16);
  }
}

template <uint32_t FMT>
__global__ void dequant_kernel(const uint8_t *plane0, const uint8_t *meta, uint32_t N, uint32_t K, float *values,
                               uint16_t *halves) {
  using F = Fmt<FMT>;
  const uint32_t G = K / 32, units = G / F::UNIT;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)N * G) return;
  const uint32_t n = (uint32_t)(t / G), g = (uint32_t)(t % G);
  const u32x4 w = *(const u32x4 *)(plane0 + sq_tile_index(n, g, G) * 16);
  const MetaWords m = load_meta<FMT>(meta + sq_tile_index(n, g / F::UNIT, units) * F::META);
  const Coef k = coef<FMT>(m, g / F::SG);
  const size_t base = (size_t)n * K + (size_t)g * 32;
#pragma unroll
  for (uint32_t c = 0; c < 4; ++c)
#pragma unroll
    for (uint32_t p = 0; p < 4; ++p) {
      const uint32_t e0 = 16u * (p >> 1) + 4u * c + 2u * (p & 1u);
      const float v0 = fmaf((float)((w[c] >> (4u * p)) & 15u), k.s, k.z);
      const float v1 = fmaf((float)((w[c] >> (16u + 4u * p)) & 15u), k.s, k.z);
      if (values) {
        values[base + e0] = v0;
        values[base + e0 + 1] = v1;
      }
      if (halves) {
        halves[base + e0] = f32_to_f16(v0);
        halves[base + e0 + 1] = f32_to_f16(v1);
      }
    }
}

}  // namespace

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

hipError_t launch_dequant(uint32_t fmt, const uint8_t *plane0, const uint8_t *meta, uint32_t N, uint32_t K,
                          float *values, uint16_t *halves, hipStream_t stream) {
  const uint64_t threads = (uint64_t)N * (K / 32);
  const dim3 grid((uint32_t)((threads + 255) / 256)), block(256);
  switch (fmt) {
    case SQ_FMT_AF4G32: hipLaunchKernelGGL(dequant_kernel<SQ_FMT_AF4G32>, grid, block, 0, stream, plane0, meta, N, K, values, halves); break;
    case SQ_FMT_AF4G64: hipLaunchKernelGGL(dequant_kernel<SQ_FMT_AF4G64>, grid, block, 0, stream, plane0, meta, N, K, values, halves); break;
    case SQ_FMT_AF4G128: hipLaunchKernelGGL(dequant_kernel<SQ_FMT_AF4G128>, grid, block, 0, stream, plane0, meta, N, K, values, halves); break;
    case SQ_FMT_Q4K: hipLaunchKernelGGL(dequant_kernel<SQ_FMT_Q4K>, grid, block, 0, stream, plane0, meta, N, K, values, halves); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace sq::kern
