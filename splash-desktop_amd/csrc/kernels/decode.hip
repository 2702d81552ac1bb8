// The row tile of the decode GEMV: y[r][c] = sum_k x[r][k] w[c][k] for 5 to 32 rows of bf16 activations against
// plane weights of any format this build takes, fp32 accumulation (reference: gguf_decode / gguf_decode_tile and
// gguf_decode_gate_up, kernels/shared/gguf_linear.metal:71-192, and the exact-operand register tile of
// kernels/decode/linear_gguf_sgmatrix.metal), and the decode tiles' layout and dispatch.
//
// CDNA4 mapping. A workgroup of W waves takes a 64-column plane tile and W K slices; each wave streams its slice
// with the row tile's inner loop (rowtile.hpp: exact bf16 operands on the 16x16x32 MFMA, rows on its 16-row side,
// per-group closes in fp32); the slices meet in LDS in slice order, every wave adding and storing only the outputs
// it owns, and K partitions across workgroups reduce as the column tile's do (the last workgroup to arrive adds the
// splits in split order). A dispatch of few tiles (column_slices 4) runs four workgroups a tile instead, each wave
// one MFMA column block of its slice (its lanes load their column's chunks and meta directly): the same operands,
// MFMAs and closes, so the same bits. A row's result depends only on its own activations and the layout, never on
// the other rows.
#include "device.hpp"
#include "kernels.hpp"
#include "rowtile.hpp"
#include "split.hpp"

namespace sq::kern {
namespace {

// The most waves a row-tile workgroup holds, so that a wave's registers fit without spilling: 16 (128 registers) for
// one tensor of 16 rows, 4 (512) for a gate/up pair of 32 rows, else 8 (256).
constexpr uint32_t row_max_waves(int mb, int nt) { return mb == 1 && nt == 1 ? 16 : mb == 2 && nt == 2 ? 4 : 8; }

// Wave `slice`'s K slice (groups gb.. of which `live` are in the slice) of plane tile `tile` of segment `seg`, in
// format FMT, into acc. TB 1: column block cs of the tile only, lane (j, q) loading chunk q of column 16 cs + j and
// that column's meta itself.
template <uint32_t FMT, int MB, int GW, int NT, int TB>
__device__ __forceinline__ void row_walk(const DecodeArgs &a, const Segment &seg, uint32_t tile, uint32_t cs,
                                         uint32_t gb, uint32_t live, uint8_t *xlds, float (&acc)[NT][TB][MB][4]) {
  using F = Fmt<FMT>;
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const uint32_t G = a.K >> 5, units = G / F::UNIT, col = TB == 1 ? 16 * cs + j : lane;
  RowBuffers<FMT, NT, MB, TB> src;
  {
    const uint32_t chunk = TB == 1 ? q * (F::P0 / 4) : 0, word = TB == 1 && F::P1 == 8 ? 4 * (q >> 1) : 0;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const Segment &from = NT == 2 && n == 0 ? a.gate : seg;
      src.plane[n] = buffer_rsrc(from.plane0 + (size_t)tile * G * 64 * F::P0, G * 64 * F::P0);
      if constexpr (F::P1) src.high[n] = buffer_rsrc(from.plane1 + (size_t)tile * G * 64 * F::P1, G * 64 * F::P1);
      src.meta[n] = buffer_rsrc(from.meta + (size_t)tile * units * 64 * F::META, units * 64 * F::META);
    }
    src.pv = (gb * 64 + col) * F::P0 + chunk;
    src.hv = (gb * 64 + col) * F::P1 + word;
    src.mv = (gb / F::UNIT * 64 + col) * F::META;
  }
  // Lane (j, q) of row block b reads row 16 b + j's inputs 8q..8q+7 of each group (row_slice puts them into the
  // MFMA's A layout through the wave's LDS slot); rows past the live ones read row 0, whose results nothing stores.
  src.input = buffer_rsrc(a.input, a.rows * a.K * 2);
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const uint32_t r = 16u * b + j;
    src.xv[b] = ((r < a.rows ? r : 0) * a.K + 8 * q + gb * 32) * 2;
  }
  row_slice<FMT, MB, GW, NT, TB>(src, xlds, live, acc);
}

// FMT kSegmentFormats: each workgroup runs its segment's format. TB 1: workgroup x takes column block x % 4 of tile
// x / 4 (16-column workgroups, each wave the same K slice as in the 64-column layout; the same bits).
template <uint32_t FMT, int MB, int GW, int NT, uint32_t EP, bool F32OUT, int TB>
__global__ __launch_bounds__(64 * row_max_waves(MB, NT)) void row_kernel(DecodeArgs a) {
  constexpr int A = NT * TB * MB * 4;   // accumulators per lane: tensor n, column block t, row block b, row i
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const uint32_t slice = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), waves = blockDim.x >> 6;
  const uint32_t split = blockIdx.y, cs = TB == 1 ? blockIdx.x & 3 : 0;
  uint32_t tile = TB == 1 ? blockIdx.x >> 2 : blockIdx.x, s = 0;
  while (s + 1 < a.segments && tile >= a.seg[s].tiles) tile -= a.seg[s++].tiles;
  const Segment seg = a.seg[s];
  const uint32_t G = a.K >> 5, gs = G / a.splits;
  const uint32_t gb = split * gs + slice * GW, live = min((uint32_t)GW, gs - min(gs, slice * GW));

  float acc[NT][TB][MB][4];
  clear(acc);
  // The slices' reduction buffer; during the walk each wave's own part of it (A floats a lane, at least MB KiB) is
  // its activations' LDS slot, which the wave leaves before writing its sums there.
  constexpr uint32_t FO = TB * MB * 4;   // outputs per tensor
  __shared__ float red[row_max_waves(MB, NT) * A * 64];
  static_assert(A * 64 * 4 >= MB * 1024, "a wave's reduction slot holds its activations' slot");
  uint8_t *const xlds = (uint8_t *)(red + slice * A * 64);
  if constexpr (FMT == kSegmentFormats)
    with_format(seg.fmt,
                [&](auto f) { row_walk<decltype(f)::value, MB, GW, NT, TB>(a, seg, tile, cs, gb, live, xlds, acc); });
  else
    row_walk<FMT, MB, GW, NT, TB>(a, seg, tile, cs, gb, live, xlds, acc);

  // The slices meet in LDS: red[slice][n FO + f][lane], f = (t MB + b) 4 + i the accumulator of column block t, row
  // block b, row 4q + i of the block. Output f (of both tensors) belongs to wave f % waves, which adds it over the
  // slices in slice order and stores it; a wave decodes and indexes only the outputs it owns. A K partition across
  // workgroups stores the sums as fp32 partials, and the last workgroup to arrive adds every split's in split order
  // and returns the counter to zero (split_reduce.h:14-45).
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(slice * A + n * FO + (t * MB + b) * 4 + i) * 64 + lane] = acc[n][t][b][i];
  __syncthreads();
  const uint32_t cstride = NT == 2 ? 2 * a.out_stride : a.out_stride;
  const uint32_t column0 = seg.out_offset + tile * 64 + 16 * cs + j;
  const size_t split_elements = (size_t)a.rows * cstride;
  // Output f's row and column.
  const auto place = [&](uint32_t f, uint32_t &row, uint32_t &col) __attribute__((always_inline)) {
    row = 16u * ((f >> 2) % MB) + 4u * q + (f & 3);
    col = column0 + 16u * ((f >> 2) / MB);
  };
  const auto store = [&](const float (&v)[NT], uint32_t row, uint32_t col) __attribute__((always_inline)) {
    const size_t o = (size_t)row * a.out_stride + col;
    if constexpr (NT == 2) {
      const float g = bf16_to_f32(f32_to_bf16(v[0])), up = bf16_to_f32(f32_to_bf16(v[1]));
      ((uint16_t *)a.output)[o] = f32_to_bf16(up * silu(g));
    } else {
      const float y = epilogue<EP>(v[0], a.aux, o);
      if constexpr (F32OUT) ((float *)a.output)[o] = y;
      else ((uint16_t *)a.output)[o] = f32_to_bf16(y);
    }
  };
  const bool splitting = a.splits > 1;
#pragma unroll 1
  for (uint32_t f = slice; f < FO; f += waves) {
    uint32_t row, col;
    place(f, row, col);
    float v[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      // Every wave slot's read goes out at once (slots past the workgroup's waves hold nothing the sum takes), then
      // the adds run in slice order.
      constexpr uint32_t kSlots = row_max_waves(MB, NT);
      float part[kSlots], sum = 0.0f;
#pragma unroll
      for (uint32_t w = 0; w < kSlots; ++w) part[w] = red[(w * A + n * FO + f) * 64 + lane];
#pragma unroll
      for (uint32_t w = 0; w < kSlots; ++w)
        if (w < waves) sum += part[w];
      v[n] = sum;
    }
    if (row >= a.rows) continue;
    if (!splitting) {
      store(v, row, col);
      continue;
    }
#pragma unroll
    for (int n = 0; n < NT; ++n)
      __hip_atomic_store(&a.partials[split * split_elements + (size_t)row * cstride + n * a.out_stride + col], v[n],
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!splitting) return;
  // Every access to the partials and the counter is a device-scope atomic, performed past the per-XCD L2s; each wave
  // waits for its partial stores to complete before thread 0 arrives at the counter.
  __shared__ uint32_t arrival;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t *counter = a.counters + blockIdx.x;
  if (threadIdx.x == 0) arrival = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (arrival != a.splits - 1) return;
  // Four of the wave's outputs at a time: their splits' loads go out together (sum_splits), each output summed in
  // split order as one at a time would be.
  constexpr int kBatch = FO < 4 ? FO : 4;
#pragma unroll 1
  for (uint32_t f0 = slice; f0 < FO; f0 += kBatch * waves) {
    uint32_t row[kBatch], col[kBatch];
    float sum[kBatch * NT], *at[kBatch * NT];
    bool on[kBatch * NT];
#pragma unroll
    for (int d = 0; d < kBatch; ++d) {
      const uint32_t f = f0 + d * waves;
      place(f < FO ? f : f0, row[d], col[d]);
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        on[d * NT + n] = f < FO && row[d] < a.rows;
        at[d * NT + n] = a.partials + (size_t)row[d] * cstride + n * a.out_stride + col[d];
      }
    }
    sum_splits(sum, on, at, split_elements, a.splits);
#pragma unroll
    for (int d = 0; d < kBatch; ++d) {
      if (!on[d * NT]) continue;
      float v[NT];
#pragma unroll
      for (int n = 0; n < NT; ++n) v[n] = sum[d * NT + n];
      store(v, row[d], col[d]);
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// column_slices 4: 16-column workgroups, four a tile (the same bits as the 64-column ones).
template <uint32_t FMT, int MB, int GW, int NT, uint32_t EP, bool F32OUT>
void launch_gw(const DecodeArgs &a, uint32_t tiles, DecodeLayout layout, hipStream_t stream) {
  const dim3 block(64 * layout.nb);
  if (a.column_slices == 4)
    hipLaunchKernelGGL((row_kernel<FMT, MB, GW, NT, EP, F32OUT, 1>), dim3(tiles * 4, a.splits), block, 0, stream, a);
  else
    hipLaunchKernelGGL((row_kernel<FMT, MB, GW, NT, EP, F32OUT, 4>), dim3(tiles, a.splits), block, 0, stream, a);
}

template <uint32_t FMT, int MB, int NT, uint32_t EP, bool F32OUT>
hipError_t launch_mb(const DecodeArgs &a, uint32_t tiles, DecodeLayout layout, hipStream_t stream) {
  switch (layout.ks) {
    case 8: launch_gw<FMT, MB, 8, NT, EP, F32OUT>(a, tiles, layout, stream); break;
    case 16: launch_gw<FMT, MB, 16, NT, EP, F32OUT>(a, tiles, layout, stream); break;
    default:
      if constexpr (NT == 1) launch_gw<FMT, MB, 32, NT, EP, F32OUT>(a, tiles, layout, stream);
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
  // workgroup of the tile the rows run. A row tile of one tensor in 16-byte codes whose 64-column workgroups
  // outnumber the compute units takes 32-group slices instead: half the waves a workgroup, so more workgroups share
  // a compute unit and the grid runs in fewer rounds. Measured (graph-replayed, one box, order alternated; M = 8 /
  // 16): K 5120 x N 27648 Q4_K 23.96 / 28.02 -> 22.85 / 26.36 us, af4g64 22.21 / 25.42 -> 21.03 / 24.63, Q6_K (M =
  // 16) 40.99 -> 38.86, N 17408 af4g64 20.12 / 23.32 -> 18.90 / 22.84; 8-bit codes lost (Q8_0 at M = 16 44.39 ->
  // 45.97), so they keep the shortest slices.
  const uint32_t gs = units / splits * sg;
  const uint32_t most = rows <= kColumnTileRows ? kColumnMaxWaves : row_max_waves(rows <= 16 ? 1 : 2, pair ? 2 : 1);
  const uint32_t tiles = blocks / 4;
  if (rows > kColumnTileRows && !pair && sq_format(fmt).plane0_bytes == 16 && tiles * splits > kDecodeUnits &&
      (gs + kColumnMaxGroups - 1) / kColumnMaxGroups <= most)
    return {(gs + kColumnMaxGroups - 1) / kColumnMaxGroups, kColumnMaxGroups};
  for (uint32_t ks = 8; ks <= (pair ? kColumnMaxGroups / 2 : kColumnMaxGroups); ks *= 2)
    if ((gs + ks - 1) / ks <= most) return {(gs + ks - 1) / ks, ks};
  return {0, 0};
}

uint32_t layout_format(uint32_t fmt, const DecodeArgs &args) {
  if (fmt != kSegmentFormats) return fmt;
  // Slices and splits that take whole meta units of the longest unit take whole units of every shorter one (units
  // of 1, 2, 4 or 8 groups), so that format's layout is every segment's.
  uint32_t widest = args.seg[0].fmt;
  for (uint32_t s = 1; s < args.segments; ++s)
    if (sq_format(args.seg[s].fmt).meta_groups > sq_format(widest).meta_groups) widest = args.seg[s].fmt;
  return widest;
}

hipError_t launch_decode(uint32_t fmt, uint32_t epilogue, bool f32_output, const DecodeArgs &args,
                         hipStream_t stream) {
  if (args.rows <= kColumnTileRows) return launch_decode_column(fmt, epilogue, f32_output, args, stream);
  uint32_t tiles = 0;
  for (uint32_t s = 0; s < args.segments; ++s) tiles += args.seg[s].tiles;
  const bool pair = args.gate.plane0 != nullptr;
  const DecodeLayout layout = decode_layout(layout_format(fmt, args), tiles * 4, args.K, args.splits, pair, args.rows);
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
    case kSegmentFormats:
      if (epilogue != EpNone || f32_output || pair) return hipErrorInvalidValue;
      return launch_rows<kSegmentFormats, 1, EpNone, false>(args, tiles, layout, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sq::kern
