// The row tile of the decode GEMV: y[r][c] = sum_k x[r][k] w[c][k] for 5 to 32 rows of bf16 activations against
// plane weights of any format this build takes, fp32 accumulation (reference: gguf_decode / gguf_decode_tile and gguf_decode_gate_up,
// kernels/shared/gguf_linear.metal:71-192, and the exact-operand register tile of
// kernels/decode/linear_gguf_sgmatrix.metal), and the decode tiles' layout and dispatch.
//
// CDNA4 mapping. A workgroup of W waves takes a 64-column plane tile and W K slices; each wave streams its slice
// with the row tile's inner loop (rowtile.hpp: exact bf16 operands on the 16x16x32 MFMA, rows on its 16-row side,
// per-group closes in fp32); the slices meet in LDS in slice order, every wave adding a share of the accumulators,
// and K partitions across workgroups reduce through split_reduce. A row's result depends only on its own
// activations and the layout, never on the other rows.
#include "device.hpp"
#include "kernels.hpp"
#include "rowtile.hpp"
#include "split.hpp"

namespace sq::kern {
namespace {

// The most waves a row-tile workgroup holds, so that a wave's registers fit without spilling: 16 (128 registers) for
// one tensor of 16 rows, 4 (512) for a gate/up pair of 32 rows, else 8 (256).
constexpr uint32_t row_max_waves(int mb, int nt) { return mb == 1 && nt == 1 ? 16 : mb == 2 && nt == 2 ? 4 : 8; }

template <uint32_t FMT, int MB, int GW, int NT, uint32_t EP, bool F32OUT>
__global__ __launch_bounds__(64 * row_max_waves(MB, NT)) void row_kernel(DecodeArgs a) {
  using F = Fmt<FMT>;
  constexpr int A = NT * 4 * MB * 4;   // accumulators per lane: tensor n, column block t, row block b, row i
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const uint32_t slice = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), waves = blockDim.x >> 6;
  const uint32_t split = blockIdx.y;
  uint32_t tile = blockIdx.x, s = 0;
  while (s + 1 < a.segments && tile >= a.seg[s].tiles) tile -= a.seg[s++].tiles;
  const Segment seg = a.seg[s];
  const uint32_t G = a.K >> 5, units = G / F::UNIT, gs = G / a.splits;
  const uint32_t gb = split * gs + slice * GW, live = min((uint32_t)GW, gs - min(gs, slice * GW));

  const uint8_t *plane[NT], *high[NT], *meta[NT];
  {
    const size_t pbase = ((size_t)tile * G * 64 + lane) * F::P0 + (size_t)gb * 64 * F::P0;
    const size_t hbase = ((size_t)tile * G * 64 + lane) * F::P1 + (size_t)gb * 64 * F::P1;
    const size_t mbase = ((size_t)tile * units * 64 + j) * F::META + (size_t)(gb / F::UNIT) * 64 * F::META;
    const Segment &first = NT == 2 ? a.gate : seg;
    plane[0] = first.plane0 + pbase;
    high[0] = F::P1 ? first.plane1 + hbase : nullptr;
    meta[0] = first.meta + mbase;
    if constexpr (NT == 2) {
      plane[1] = seg.plane0 + pbase;
      high[1] = F::P1 ? seg.plane1 + hbase : nullptr;
      meta[1] = seg.meta + mbase;
    }
  }
  // Lane (j, q) of row block b reads row 16 b + j's inputs 4q..4q+3 and 16+4q..19+4q of each group (the MFMA's A
  // layout); rows past the live ones read row 0, whose results nothing stores.
  const uint16_t *xrow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const uint32_t r = 16u * b + j;
    xrow[b] = a.input + (size_t)(r < a.rows ? r : 0) * a.K + 4 * q + (size_t)gb * 32;
  }
  float acc[NT][4][MB][4];
  clear(acc);
  row_slice<FMT, MB, GW, NT>(plane, high, meta, xrow, live, acc);

  __shared__ float red[row_max_waves(MB, NT) * A * 64];
  float sum[A];
  bool owned[A];
  row_reduce<MB, NT>(acc, red, slice, waves, lane, sum, owned);
  const uint32_t cstride = NT == 2 ? 2 * a.out_stride : a.out_stride;
  float total[A][1];
  bool rlive[A][1];
  size_t index[A][1];
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = ((n * 4 + t) * MB + b) * 4 + i;
          const uint32_t row = 16u * b + 4u * q + i;
          total[e][0] = sum[e];
          rlive[e][0] = owned[e] && row < a.rows;
          index[e][0] = (size_t)row * cstride + n * a.out_stride + seg.out_offset + tile * 64 + 16 * t + j;
        }
  if (a.splits > 1 && !split_reduce<A, 1>(total, rlive, index, a.partials, (size_t)a.rows * cstride, split, a.splits,
                                          a.counters + blockIdx.x, true))
    return;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = (t * MB + b) * 4 + i;
        if (!rlive[e][0]) continue;
        const size_t o = (size_t)(16u * b + 4u * q + i) * a.out_stride + seg.out_offset + tile * 64 + 16 * t + j;
        if constexpr (NT == 2) {
          const float g = bf16_to_f32(f32_to_bf16(total[e][0])), up = bf16_to_f32(f32_to_bf16(total[4 * MB * 4 + e][0]));
          ((uint16_t *)a.output)[o] = f32_to_bf16(up * silu(g));
        } else {
          const float v = epilogue<EP>(total[e][0], a.aux, o);
          if constexpr (F32OUT) ((float *)a.output)[o] = v;
          else ((uint16_t *)a.output)[o] = f32_to_bf16(v);
        }
      }
}

template <uint32_t FMT, int MB, int NT, uint32_t EP, bool F32OUT>
hipError_t launch_mb(const DecodeArgs &a, uint32_t tiles, DecodeLayout layout, hipStream_t stream) {
  const dim3 grid(tiles, a.splits), block(64 * layout.nb);
  switch (layout.ks) {
    case 8: hipLaunchKernelGGL((row_kernel<FMT, MB, 8, NT, EP, F32OUT>), grid, block, 0, stream, a); break;
    case 16: hipLaunchKernelGGL((row_kernel<FMT, MB, 16, NT, EP, F32OUT>), grid, block, 0, stream, a); break;
    default:
      if constexpr (NT == 1) hipLaunchKernelGGL((row_kernel<FMT, MB, 32, NT, EP, F32OUT>), grid, block, 0, stream, a);
      break;
  }
  return hipGetLastError();
}

template <uint32_t FMT, int NT, uint32_t EP, bool F32OUT>
hipError_t launch_rows(const DecodeArgs &a, uint32_t tiles, DecodeLayout layout, hipStream_t stream) {
  return a.rows <= 16 ? launch_mb<FMT, 1, NT, EP, F32OUT>(a, tiles, layout, stream)
                      : launch_mb<FMT, 2, NT, EP, F32OUT>(a, tiles, layout, stream);
}

template <uint32_t FMT>
hipError_t launch_format(uint32_t epilogue, bool f32_output, bool pair, const DecodeArgs &a, uint32_t tiles,
                         DecodeLayout layout, hipStream_t stream) {
  if (pair) return launch_rows<FMT, 2, EpNone, false>(a, tiles, layout, stream);
  if (f32_output) return launch_rows<FMT, 1, EpNone, true>(a, tiles, layout, stream);
  switch (epilogue) {
    case EpNone: return launch_rows<FMT, 1, EpNone, false>(a, tiles, layout, stream);
    case EpResidual: return launch_rows<FMT, 1, EpResidual, false>(a, tiles, layout, stream);
    default: return launch_rows<FMT, 1, EpUpWithGate, false>(a, tiles, layout, stream);
  }
}

}  // namespace

DecodeLayout decode_layout(uint32_t fmt, uint32_t blocks, uint32_t K, uint32_t splits, bool pair, uint32_t rows) {
  const uint32_t sg = sq_format(fmt).meta_groups;   // groups of 32 per meta unit
  const bool runs = rows <= kColumnTileRows ? column_tile_format(fmt) : row_tile_format(fmt);
  if (!runs || !splits || !rows || rows > SQ_MAXIMUM_DECODE_ROWS || blocks % 4) return {0, 0};
  const uint32_t units = K / 32 / sg;
  if (units % splits || !(units / splits)) return {0, 0};
  // The shortest slices (8, 16 or 32 groups; a gate/up pair streams two tensors, at most 16) whose waves fit one
  // workgroup of the tile the rows run.
  const uint32_t gs = units / splits * sg;
  const uint32_t most = rows <= kColumnTileRows ? kColumnMaxWaves : row_max_waves(rows <= 16 ? 1 : 2, pair ? 2 : 1);
  for (uint32_t ks = 8; ks <= (pair ? kColumnMaxGroups / 2 : kColumnMaxGroups); ks *= 2)
    if ((gs + ks - 1) / ks <= most) return {(gs + ks - 1) / ks, ks};
  return {0, 0};
}

hipError_t launch_decode(uint32_t fmt, uint32_t epilogue, bool f32_output, const DecodeArgs &args,
                         hipStream_t stream) {
  if (args.rows <= kColumnTileRows) return launch_decode_column(fmt, epilogue, f32_output, args, stream);
  uint32_t tiles = 0;
  for (uint32_t s = 0; s < args.segments; ++s) tiles += args.seg[s].tiles;
  const bool pair = args.gate.plane0 != nullptr;
  const DecodeLayout layout = decode_layout(fmt, tiles * 4, args.K, args.splits, pair, args.rows);
  if (!layout.nb) return hipErrorInvalidValue;
  switch (fmt) {
    case SQ_FMT_AF4G32: return launch_format<SQ_FMT_AF4G32>(epilogue, f32_output, pair, args, tiles, layout, stream);
    case SQ_FMT_AF4G64: return launch_format<SQ_FMT_AF4G64>(epilogue, f32_output, pair, args, tiles, layout, stream);
    case SQ_FMT_AF4G128: return launch_format<SQ_FMT_AF4G128>(epilogue, f32_output, pair, args, tiles, layout, stream);
    case SQ_FMT_Q4K: return launch_format<SQ_FMT_Q4K>(epilogue, f32_output, pair, args, tiles, layout, stream);
    case SQ_FMT_Q5K: return launch_format<SQ_FMT_Q5K>(epilogue, f32_output, pair, args, tiles, layout, stream);
    case SQ_FMT_Q6K: return launch_format<SQ_FMT_Q6K>(epilogue, f32_output, pair, args, tiles, layout, stream);
    case SQ_FMT_Q80: return launch_format<SQ_FMT_Q80>(epilogue, f32_output, pair, args, tiles, layout, stream);
    case SQ_FMT_AF8G64: return launch_format<SQ_FMT_AF8G64>(epilogue, f32_output, pair, args, tiles, layout, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sq::kern
