// The producers either side of the projections: the RMS norm that feeds them (reference: Normalization::addRms,
// runtime/ops/Normalization.cpp:16-38; kernels/shared/normalization.metal:60-103,150-221 and
// kernels/common/rms_inverse.h:14-31), optionally writing the prefill tile's prepared input in the same pass, and
// the float projection of rows kept unquantized, the MoE router's among them (reference: addGgufFloat,
// runtime/ops/LinearGguf.cpp:806-818 and kernels/shared/gguf_float.metal).
//
// CDNA4 mapping. The norm is HBM-bound at 4 bytes a value in and out (plus 4 for the table): one workgroup a row,
// every value read once into registers in the prefill table's chunk order, so the table costs no extra read. The
// float projection is a few hundred MFLOP at the router's sizes: a wave computes 4 rows x 4 columns, its lanes
// splitting K (coalesced 16-byte weight loads), and a butterfly sums the lanes in a fixed order.
#include "device.hpp"
#include "half_rows.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

// SPLASH_RMS_EPSILON (metal/abi/ExecutionGeometry.h:59).
constexpr float kRmsEpsilon = 1e-6f;

// The norm weights of one 4-input unit, widened to fp32: bf16 or F32 as stored (Normalization.hpp:14-23).
template <bool F32W>
__device__ __forceinline__ f32x4 unit_weights(const void *weight, uint32_t unit) {
  if constexpr (F32W) {
    return ((const f32x4 *)weight)[unit];
  } else {
    const u32x2 v = ((const u32x2 *)weight)[unit];
    return f32x4{bf16_to_f32(v[0] & 0xFFFFu), bf16_to_f32(v[0] >> 16), bf16_to_f32(v[1] & 0xFFFFu),
                 bf16_to_f32(v[1] >> 16)};
  }
}

// out[r][c] = bf16((x[r][c] * inv) * w[c]), inv = rsqrt(sum_c x[r][c]^2 / width + eps) in fp32, one workgroup a row.
// Thread t holds the row's chunks t + 256 i of the prefill table's order (8 values each, half_rows.hpp), held in
// registers for rows of at most 256 NV chunks (NV > 0) and read twice otherwise. With TABLE the pass also writes
// the half rows table of the normalised bf16 row and its scale, the same bits the prefill's prepare dispatch
// would write from `output`.
template <bool F32W, bool TABLE, int NV>
__global__ __launch_bounds__(256) void rms_kernel(const uint16_t *input, const void *weight, uint16_t *output,
                                                  uint32_t width, uint16_t *half_input, float *row_scale) {
  const uint32_t r = blockIdx.x, vectors = width / 8;
  const u32x2 *units = (const u32x2 *)(input + (size_t)r * width);
  u32x2 *out = (u32x2 *)(output + (size_t)r * width);
  const auto chunk = [&](uint32_t v) __attribute__((always_inline)) {
    const uint32_t u = half_rows_unit(v);
    const u32x2 lo = units[u], hi = units[u + 4];
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  const auto squares = [](u32x4 w, float s) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x0 = bf16_to_f32(w[e] & 0xFFFFu), x1 = bf16_to_f32(w[e] >> 16);
      s = fmaf(x0, x0, s);
      s = fmaf(x1, x1, s);
    }
    return s;
  };
  float sum = 0.0f;
  u32x4 held[NV > 0 ? NV : 1];
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t v = threadIdx.x + 256u * i;
      held[i] = v < vectors ? chunk(v) : u32x4{0u, 0u, 0u, 0u};
      sum = squares(held[i], sum);
    }
  } else {
    for (uint32_t v = threadIdx.x; v < vectors; v += 256) sum = squares(chunk(v), sum);
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) sum += __shfl_xor(sum, d);
  __shared__ float part[4];
  __shared__ uint32_t largest_part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sum;
  __syncthreads();
  const float total = ((part[0] + part[1]) + part[2]) + part[3];
  const float inverse = rsqrtf(total / (float)width + kRmsEpsilon);

  const auto normalise = [&](u32x4 x, uint32_t v) __attribute__((always_inline)) {
    const uint32_t u = half_rows_unit(v);
    const f32x4 w0 = unit_weights<F32W>(weight, u), w1 = unit_weights<F32W>(weight, u + 4);
    u32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f32x4 &w = e < 2 ? w0 : w1;
      const float a = (bf16_to_f32(x[e] & 0xFFFFu) * inverse) * w[2 * (e & 1)];
      const float b = (bf16_to_f32(x[e] >> 16) * inverse) * w[2 * (e & 1) + 1];
      y[e] = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
    }
    out[u] = u32x2{y[0], y[1]};
    out[u + 4] = u32x2{y[2], y[3]};
    return y;
  };
  uint32_t largest = 0;
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t v = threadIdx.x + 256u * i;
      if (v < vectors) {
        held[i] = normalise(held[i], v);
        largest = max(largest, bf16_largest(held[i]));
      }
    }
  } else {
    for (uint32_t v = threadIdx.x; v < vectors; v += 256) largest = max(largest, bf16_largest(normalise(chunk(v), v)));
  }
  if constexpr (TABLE) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) largest = max(largest, (uint32_t)__shfl_xor((int)largest, d));
    if ((threadIdx.x & 63) == 0) largest_part[threadIdx.x >> 6] = largest;
    __syncthreads();
    largest = max(max(largest_part[0], largest_part[1]), max(largest_part[2], largest_part[3]));
    const int shift = half_rows_shift(largest);
    const float down = ldexpf(1.0f, -shift);
    if (threadIdx.x == 0) row_scale[r] = ldexpf(1.0f, shift);
    u32x4 *h = (u32x4 *)(half_input + (size_t)r * width);
    if constexpr (NV > 0) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const uint32_t v = threadIdx.x + 256u * i;
        if (v < vectors) h[v] = half_rows_chunk(held[i], down);
      }
    } else {
      // The thread reads back the chunks it wrote itself.
      const u32x2 *written = (const u32x2 *)out;
      for (uint32_t v = threadIdx.x; v < vectors; v += 256) {
        const uint32_t u = half_rows_unit(v);
        const u32x2 lo = written[u], hi = written[u + 4];
        h[v] = half_rows_chunk(u32x4{lo[0], lo[1], hi[0], hi[1]}, down);
      }
    }
  }
}

template <bool F32W, bool TABLE>
hipError_t launch_rms_rows(const uint16_t *input, const void *weight, uint16_t *output, uint32_t width,
                           uint32_t rows, uint16_t *half_input, float *row_scale, hipStream_t stream) {
  const uint32_t chunks = width / 8;
  const dim3 grid(rows), block(256);
#define SQ_RMS(NV) \
  hipLaunchKernelGGL((rms_kernel<F32W, TABLE, NV>), grid, block, 0, stream, input, weight, output, width, half_input, \
                     row_scale)
  if (chunks <= 256) SQ_RMS(1);
  else if (chunks <= 512) SQ_RMS(2);
  else if (chunks <= 1024) SQ_RMS(4);
  else if (chunks <= 2048) SQ_RMS(8);
  else SQ_RMS(0);
#undef SQ_RMS
  return hipGetLastError();
}

// out[r][offset + n] = sum_k x[r][k] W[n][k], W's rows fp32 or bf16 as stored, products and sums in fp32. A wave
// computes rows 4 blockIdx.y .. +3 against columns 4 (4 blockIdx.x + w) .. +3: lane l takes inputs 4 l + 256 i
// .. +3 of each, and the lanes' sums meet in a butterfly (the same order for every output).
template <bool F32W, bool F32OUT>
__global__ __launch_bounds__(256) void float_rows_kernel(const uint16_t *input, const void *weights, void *output,
                                                         uint32_t rows, uint32_t N, uint32_t K, uint32_t out_stride,
                                                         uint32_t out_offset) {
  const uint32_t lane = threadIdx.x & 63, n0 = 4 * (4 * blockIdx.x + (threadIdx.x >> 6)), r0 = 4 * blockIdx.y;
  if (n0 >= N) return;
  float acc[4][4] = {};
  const uint16_t *xr[4];
  const uint8_t *wr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xr[i] = input + (size_t)min(r0 + i, rows - 1) * K;
    wr[i] = (const uint8_t *)weights + (size_t)min(n0 + i, N - 1) * K * (F32W ? 4 : 2);
  }
  for (uint32_t k = 4 * lane; k < K; k += 256) {
    f32x4 w[4], x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (F32W) {
        w[i] = *(const f32x4 *)(wr[i] + (size_t)k * 4);
      } else {
        const u32x2 v = *(const u32x2 *)(wr[i] + (size_t)k * 2);
        w[i] = f32x4{bf16_to_f32(v[0] & 0xFFFFu), bf16_to_f32(v[0] >> 16), bf16_to_f32(v[1] & 0xFFFFu),
                     bf16_to_f32(v[1] >> 16)};
      }
      const u32x2 v = *(const u32x2 *)(xr[i] + k);
      x[i] = f32x4{bf16_to_f32(v[0] & 0xFFFFu), bf16_to_f32(v[0] >> 16), bf16_to_f32(v[1] & 0xFFFFu),
                   bf16_to_f32(v[1] >> 16)};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][n] = fmaf(x[i][e], w[n][e], acc[i][n]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int n = 0; n < 4; ++n)
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) acc[i][n] += __shfl_xor(acc[i][n], d);
  if (lane >= 16) return;
  const uint32_t i = lane >> 2, n = lane & 3;
  if (r0 + i >= rows || n0 + n >= N) return;
  float v = 0.0f;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
      if ((uint32_t)a == i && (uint32_t)b == n) v = acc[a][b];
  const size_t at = (size_t)(r0 + i) * out_stride + out_offset + n0 + n;
  if constexpr (F32OUT) ((float *)output)[at] = v;
  else ((uint16_t *)output)[at] = f32_to_bf16(v);
}

// The same projection for rows in the prefill's numbers, on the fp32 MFMA (16x16x4): a workgroup of kFloatSlices
// waves computes 32 rows x 32 columns, wave s over K slice s (K / kFloatSlices inputs). Per 16 inputs lane (kq, r)
// (l = 16 kq + r) loads inputs 4 kq..4 kq + 3 of row r of each row block and of column r of each column block, and
// MFMA e (0..3) takes input 4 kq + e of them, into accumulator chain e: four chains of K / (16 kFloatSlices) MFMAs,
// added ((0 + 1) + (2 + 3)), then the slices in a fixed pairwise tree through LDS. An output's longest path is at most
// 4 K / (16 kFloatSlices) + 2 + log2 kFloatSlices + 1 roundings (an MFMA's four products summed in at most four),
// K / 64 + 7 for sixteen slices: within the lane-chain kernel's K / 64 + 8.
constexpr int kFloatSlices = 16;
static_assert(kFloatMfmaInputs == 16 * kFloatSlices, "every slice takes whole 16-input steps");
template <bool F32W, bool F32OUT>
__global__ __launch_bounds__(64 * kFloatSlices) void float_rows_mfma_kernel(const uint16_t *input, const void *weights,
                                                                            void *output, uint32_t rows, uint32_t N,
                                                                            uint32_t K, uint32_t out_stride,
                                                                            uint32_t out_offset) {
  const uint32_t lane = threadIdx.x & 63, slice = threadIdx.x >> 6, r = lane & 15, kq = lane >> 4;
  const uint32_t r0 = 32 * blockIdx.y, n0 = 32 * blockIdx.x, span = K / kFloatSlices, k0 = slice * span + 4 * kq;
  const uint16_t *xr[2];
  const uint8_t *wr[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    xr[b] = input + (size_t)min(r0 + 16 * b + r, rows - 1) * K + k0;
    wr[b] = (const uint8_t *)weights + ((size_t)min(n0 + 16 * b + r, N - 1) * K + k0) * (F32W ? 4 : 2);
  }
  const auto widen = [](u32x2 v) __attribute__((always_inline)) {
    return f32x4{bf16_to_f32(v[0] & 0xFFFFu), bf16_to_f32(v[0] >> 16), bf16_to_f32(v[1] & 0xFFFFu),
                 bf16_to_f32(v[1] >> 16)};
  };
  f32x4 acc[4][2][2];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) acc[e][a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (uint32_t k = 0; k < span; k += 16) {
    f32x4 x[2], w[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      x[b] = widen(*(const u32x2 *)(xr[b] + k));
      if constexpr (F32W) w[b] = *(const f32x4 *)(wr[b] + (size_t)k * 4);
      else w[b] = widen(*(const u32x2 *)(wr[b] + (size_t)k * 2));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[e][a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[a][e], w[b][e], acc[e][a][b], 0, 0, 0);
  }
  // Lane (kq, c) holds rows 4 kq + i of each row block at column c of each column block.
  __shared__ float red[kFloatSlices][2][2][4][64];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[slice][a][b][i][lane] = (acc[0][a][b][i] + acc[1][a][b][i]) + (acc[2][a][b][i] + acc[3][a][b][i]);
  __syncthreads();
  // Output o = ((a 2 + b) 4 + i) 64 + lane, 1024 of them: one a thread, the slices added pairwise in a fixed tree.
  const uint32_t o = threadIdx.x, a = o >> 9, b = (o >> 8) & 1, i = (o >> 6) & 3, l = o & 63;
  float v[kFloatSlices];
#pragma unroll
  for (int s = 0; s < kFloatSlices; ++s) v[s] = red[s][a][b][i][l];
#pragma unroll
  for (int w = 1; w < kFloatSlices; w <<= 1)
#pragma unroll
    for (int s = 0; s < kFloatSlices; s += 2 * w) v[s] += v[s + w];
  const uint32_t row = r0 + 16 * a + 4 * (l >> 4) + i, col = n0 + 16 * b + (l & 15);
  if (row >= rows || col >= N) return;
  const size_t at = (size_t)row * out_stride + out_offset + col;
  if constexpr (F32OUT) ((float *)output)[at] = v[0];
  else ((uint16_t *)output)[at] = f32_to_bf16(v[0]);
}

}  // namespace

hipError_t launch_rms_norm(const uint16_t *input, const void *weight, bool f32_weights, uint16_t *output,
                           uint32_t width, uint32_t rows, uint16_t *half_input, float *row_scale,
                           hipStream_t stream) {
  if (!rows || width % 64) return hipErrorInvalidValue;
  const bool table = half_input != nullptr;
  if (f32_weights)
    return table ? launch_rms_rows<true, true>(input, weight, output, width, rows, half_input, row_scale, stream)
                 : launch_rms_rows<true, false>(input, weight, output, width, rows, half_input, row_scale, stream);
  return table ? launch_rms_rows<false, true>(input, weight, output, width, rows, half_input, row_scale, stream)
               : launch_rms_rows<false, false>(input, weight, output, width, rows, half_input, row_scale, stream);
}

hipError_t launch_float_rows(const uint16_t *input, const void *weights, bool f32_weights, void *output,
                             bool f32_output, uint32_t rows, uint32_t N, uint32_t K, uint32_t out_stride,
                             uint32_t out_offset, bool mfma, hipStream_t stream) {
  if (!rows || !N || K % 4 || (mfma && K % kFloatMfmaInputs)) return hipErrorInvalidValue;
  const dim3 grid = mfma ? dim3((N + 31) / 32, (rows + 31) / 32) : dim3((N + 15) / 16, (rows + 3) / 4);
  const dim3 block = mfma ? dim3(64 * kFloatSlices) : dim3(256);
#define SQ_FLOAT(W, O)                                                                                                \
  if (mfma)                                                                                                          \
    hipLaunchKernelGGL((float_rows_mfma_kernel<W, O>), grid, block, 0, stream, input, weights, output, rows, N, K,   \
                       out_stride, out_offset);                                                                      \
  else                                                                                                               \
    hipLaunchKernelGGL((float_rows_kernel<W, O>), grid, block, 0, stream, input, weights, output, rows, N, K,         \
                       out_stride, out_offset)
  if (f32_weights) {
    if (f32_output) SQ_FLOAT(true, true);
    else SQ_FLOAT(true, false);
  } else {
    if (f32_output) SQ_FLOAT(false, true);
    else SQ_FLOAT(false, false);
  }
#undef SQ_FLOAT
  return hipGetLastError();
}

}  // namespace sq::kern
