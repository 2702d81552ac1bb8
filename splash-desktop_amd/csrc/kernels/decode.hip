// The decode tile: y[r][c] = sum_k x[r][k] w[c][k] for up to 32 rows of bf16 activations against 4-bit plane
// weights, fp32 accumulation (reference: gguf_decode / gguf_decode_tile and gguf_decode_gate_up,
// kernels/shared/gguf_linear.metal:71-192, and the exact-operand register tile of
// kernels/decode/linear_gguf_sgmatrix.metal).
//
// CDNA4 mapping. A 256-thread workgroup owns one 64-column plane tile and one K partition; each of its four waves
// walks a contiguous quarter of the partition's scale groups (walk.hpp) and the waves meet in LDS in wave order.
// K partitions reduce as the reference's split_reduce.h:14-45 does: fp32 partials [split][rows][stride], and the last
// workgroup to arrive at the tile's counter adds them in split order and returns the counter to zero, so results do
// not depend on scheduling.
#include "kernels.hpp"
#include "walk.hpp"

namespace sq::kern {
namespace {

// Adds this split's totals to the others' in split order when this workgroup arrives last; returns false when
// another workgroup still has to arrive. `index(b, i)` is the partial's offset within a split (row-major, stride
// elements per row), `stride_rows` the rows of a split.
template <int NB, int R>
__device__ __forceinline__ bool split_reduce(float (&total)[NB][R], const bool (&live)[NB][R],
                                             const size_t (&index)[NB][R], float *partials, size_t split_elements,
                                             uint32_t split, uint32_t splits, uint32_t *counter) {
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (live[b][i]) partials[split * split_elements + index[b][i]] = total[b][i];
  __shared__ uint32_t arrival;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) arrival = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (arrival != splits - 1) return false;
  __threadfence();
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (!live[b][i]) continue;
      float v = 0.0f;
      for (uint32_t p = 0; p < splits; ++p)
        v += p == split ? total[b][i]
                        : __hip_atomic_load(&partials[p * split_elements + index[b][i]], __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
      total[b][i] = v;
    }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

template <uint32_t FMT, int MT, uint32_t EP, bool F32OUT>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
  using F = Fmt<FMT>;
  constexpr int MB = MT > 16 ? 2 : 1;   // 16-row A blocks
  constexpr int R = MT >= 4 ? 4 : MT;   // accumulator rows each lane group keeps
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;

  uint32_t tile = blockIdx.x, s = 0;
  while (s + 1 < a.segments && tile >= a.seg[s].tiles) tile -= a.seg[s++].tiles;
  const Segment seg = a.seg[s];
  const uint32_t G = a.K >> 5, units = G / F::UNIT, groups = G / F::SG;
  const uint32_t per = groups / a.splits, split = blockIdx.y;
  const uint32_t g0 = split * per + (uint32_t)wave * per / 4, g1 = split * per + (uint32_t)(wave + 1) * per / 4;
  const uint8_t *plane[1] = {seg.plane0 + (size_t)tile * G * 1024 + (size_t)j * 16 + (size_t)q * 4};
  const uint8_t *meta[1] = {seg.meta + ((size_t)tile * units * 64 + j) * F::META};
  RowPtrs x;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint32_t r = 16u * b + j;
    x.row[b] = b < MB && r < a.rows ? a.input + (size_t)r * a.K : nullptr;
  }

  f32x4 acc[1][4][MB];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[0][t][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  walk<FMT, MB, R, 1>(plane, meta, x, g0, g1, q, acc);

  __shared__ float red[4 * 4 * MB * R * 64];
  float total[1][MB][R];
  reduce_waves<MB, R, 1>(acc, red, wave, lane, total);

  const uint32_t col = seg.out_offset + tile * 64 + 16 * wave + j;
  bool live[MB][R];
  size_t index[MB][R];
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const uint32_t r = 16u * b + 4u * q + i;
      live[b][i] = r < a.rows;
      index[b][i] = (size_t)r * a.out_stride + col;
    }
  if (a.splits > 1 && !split_reduce<MB, R>(total[0], live, index, a.partials, (size_t)a.rows * a.out_stride, split,
                                           a.splits, a.counters + seg.out_offset / 64 + tile))
    return;
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (!live[b][i]) continue;
      const float o = epilogue<EP>(total[0][b][i], a.aux, index[b][i]);
      if constexpr (F32OUT) ((float *)a.output)[index[b][i]] = o;
      else ((uint16_t *)a.output)[index[b][i]] = f32_to_bf16(o);
    }
}

// Gate and up of one format over the same 64 columns in one dispatch: both tensors' walks share the activations'
// loads and input sums, and the output is bf16(bf16(up) * silu(bf16(gate))) as the up pass of two passes writes
// it. Each tensor's sums follow its own single-pass order, so the result is bitwise the two passes' at the same
// split. Partials [split][rows][2 * out_stride] (gate's columns, then up's at out_stride on).
template <uint32_t FMT, int MT>
__global__ __launch_bounds__(256) void gate_up_kernel(GateUpArgs a) {
  using F = Fmt<FMT>;
  constexpr int MB = MT > 16 ? 2 : 1;
  constexpr int R = MT >= 4 ? 4 : MT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;
  const uint32_t tile = blockIdx.x;
  const uint32_t G = a.K >> 5, units = G / F::UNIT, groups = G / F::SG;
  const uint32_t per = groups / a.splits, split = blockIdx.y;
  const uint32_t g0 = split * per + (uint32_t)wave * per / 4, g1 = split * per + (uint32_t)(wave + 1) * per / 4;
  const size_t pbase = (size_t)tile * G * 1024 + (size_t)j * 16 + (size_t)q * 4;
  const size_t mbase = ((size_t)tile * units * 64 + j) * F::META;
  const uint8_t *plane[2] = {a.gate.plane0 + pbase, a.up.plane0 + pbase};
  const uint8_t *meta[2] = {a.gate.meta + mbase, a.up.meta + mbase};
  RowPtrs x;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint32_t r = 16u * b + j;
    x.row[b] = b < MB && r < a.rows ? a.input + (size_t)r * a.K : nullptr;
  }
  f32x4 acc[2][4][MB];
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b) acc[n][t][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  walk<FMT, MB, R, 2>(plane, meta, x, g0, g1, q, acc);
  __shared__ float red[4 * 2 * 4 * MB * R * 64];
  float total[2][MB][R];
  reduce_waves<MB, R, 2>(acc, red, wave, lane, total);

  const uint32_t col = a.up.out_offset + tile * 64 + 16 * wave + j;
  // Both tensors' partials in one array: gate's at column col, up's at out_stride + col of each row of 2 strides.
  float both[2 * MB][R];
  bool live[2 * MB][R];
  size_t index[2 * MB][R];
#pragma unroll
  for (int n = 0; n < 2; ++n)
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const uint32_t r = 16u * b + 4u * q + i;
        both[n * MB + b][i] = total[n][b][i];
        live[n * MB + b][i] = r < a.rows;
        index[n * MB + b][i] = (size_t)r * 2 * a.out_stride + n * a.out_stride + col;
      }
  if (a.splits > 1 && !split_reduce<2 * MB, R>(both, live, index, a.partials, (size_t)a.rows * 2 * a.out_stride,
                                               split, a.splits, a.counters + a.up.out_offset / 64 + tile))
    return;
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (!live[b][i]) continue;
      const uint32_t r = 16u * b + 4u * q + i;
      const float g = bf16_to_f32(f32_to_bf16(both[b][i])), u = bf16_to_f32(f32_to_bf16(both[MB + b][i]));
      a.output[(size_t)r * a.out_stride + col] = f32_to_bf16(u * silu(g));
    }
}

template <uint32_t FMT, int MT, uint32_t EP, bool F32OUT>
hipError_t launch_one(const DecodeArgs &a, hipStream_t stream) {
  uint32_t tiles = 0;
  for (uint32_t s = 0; s < a.segments; ++s) tiles += a.seg[s].tiles;
  hipLaunchKernelGGL((decode_kernel<FMT, MT, EP, F32OUT>), dim3(tiles, a.splits), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <uint32_t FMT, uint32_t EP, bool F32OUT>
hipError_t launch_rows(const DecodeArgs &a, hipStream_t stream) {
  if (a.rows <= 1) return launch_one<FMT, 1, EP, F32OUT>(a, stream);
  if (a.rows <= 2) return launch_one<FMT, 2, EP, F32OUT>(a, stream);
  if (a.rows <= 4) return launch_one<FMT, 4, EP, F32OUT>(a, stream);
  if (a.rows <= 16) return launch_one<FMT, 16, EP, F32OUT>(a, stream);
  return launch_one<FMT, 32, EP, F32OUT>(a, stream);
}

template <uint32_t FMT>
hipError_t launch_format(uint32_t epilogue, bool f32_output, const DecodeArgs &a, hipStream_t stream) {
  if (f32_output) return launch_rows<FMT, EpNone, true>(a, stream);
  switch (epilogue) {
    case EpNone: return launch_rows<FMT, EpNone, false>(a, stream);
    case EpResidual: return launch_rows<FMT, EpResidual, false>(a, stream);
    default: return launch_rows<FMT, EpUpWithGate, false>(a, stream);
  }
}

template <uint32_t FMT, int MT>
hipError_t launch_pair(const GateUpArgs &a, hipStream_t stream) {
  hipLaunchKernelGGL((gate_up_kernel<FMT, MT>), dim3(a.up.tiles, a.splits), dim3(256), 0, stream, a);
  return hipGetLastError();
}
template <uint32_t FMT>
hipError_t launch_pair_rows(const GateUpArgs &a, hipStream_t stream) {
  if (a.rows <= 1) return launch_pair<FMT, 1>(a, stream);
  if (a.rows <= 2) return launch_pair<FMT, 2>(a, stream);
  if (a.rows <= 4) return launch_pair<FMT, 4>(a, stream);
  if (a.rows <= 16) return launch_pair<FMT, 16>(a, stream);
  return launch_pair<FMT, 32>(a, stream);
}

}  // namespace

hipError_t launch_decode(uint32_t fmt, uint32_t epilogue, bool f32_output, const DecodeArgs &a,
                         hipStream_t stream) {
  switch (fmt) {
    case SQ_FMT_AF4G32: return launch_format<SQ_FMT_AF4G32>(epilogue, f32_output, a, stream);
    case SQ_FMT_AF4G64: return launch_format<SQ_FMT_AF4G64>(epilogue, f32_output, a, stream);
    case SQ_FMT_AF4G128: return launch_format<SQ_FMT_AF4G128>(epilogue, f32_output, a, stream);
    case SQ_FMT_Q4K: return launch_format<SQ_FMT_Q4K>(epilogue, f32_output, a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode_gate_up(uint32_t fmt, const GateUpArgs &a, hipStream_t stream) {
  switch (fmt) {
    case SQ_FMT_AF4G32: return launch_pair_rows<SQ_FMT_AF4G32>(a, stream);
    case SQ_FMT_AF4G64: return launch_pair_rows<SQ_FMT_AF4G64>(a, stream);
    case SQ_FMT_AF4G128: return launch_pair_rows<SQ_FMT_AF4G128>(a, stream);
    case SQ_FMT_Q4K: return launch_pair_rows<SQ_FMT_Q4K>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sq::kern
