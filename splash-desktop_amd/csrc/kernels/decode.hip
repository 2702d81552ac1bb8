// The decode tile: y[r][c] = sum_k x[r][k] w[c][k] for up to 32 rows of bf16 activations against 4-bit plane
// weights, fp32 accumulation (reference: gguf_decode / gguf_decode_tile and gguf_decode_gate_up,
// kernels/shared/gguf_linear.metal:71-192, and the exact-operand register tile of
// kernels/decode/linear_gguf_sgmatrix.metal).
//
// CDNA4 mapping. The tile is HBM-bound, so the design maximises bytes in flight and minimises serial phases:
//  - a wave owns one 16-column block and one K slice of up to KS groups of 32 inputs, and issues every code and
//    meta load of its slice before its first MFMA (up to 16 KiB of codes per wave in flight);
//  - per group the 16 columns' 256 bytes of codes arrive as one dword per lane (lane (j, q): word q of column j's
//    16-byte unit), become eight exact bf16 operands 128 + q each, and meet the activations in one 16x16x32 bf16
//    MFMA; a second MFMA against bf16 ones gives the rows' input sums. Each scale group closes in fp32:
//      acc += s * sum x (128 + q) + (z - 128 s) * sum x  =  sum x (s q + z);
//  - the activation fragments (L2-resident, shared by every workgroup) stream through a ring of registers kPipe
//    groups ahead of the MFMAs;
//  - a workgroup of four waves holds NB column blocks x (4 / NB) K slices; slices meet in LDS in slice order;
//  - K partitions across workgroups (splits) reduce as the reference's split_reduce.h:14-45 does: fp32 partials
//    [split][rows][stride] and the last workgroup to arrive at the column block's counter adds them in split order
//    and returns the counter to zero, so results do not depend on scheduling. A row's result depends only on its
//    own activations, the split and the layout (NB, KS), which the launcher derives from the shape alone.
#include "kernels.hpp"
#include "device.hpp"
#include "split.hpp"

namespace sq::kern {
namespace {

constexpr int kWaves = 4;
constexpr int kPipe = 8;   // activation fragments in flight ahead of the MFMAs

// Where a 16-column block of the dispatch lies: its segment, plane tile and 16-column sub-block t of the tile.
struct BlockPlace {
  const uint8_t *plane0, *meta;
  uint32_t tile, t, out_offset, live;
};
__device__ __forceinline__ BlockPlace place(const Segment (&seg)[3], uint32_t segments, uint32_t block) {
  uint32_t s = 0;
  while (s + 1 < segments && block >= seg[s].tiles * 4) block -= seg[s++].tiles * 4;
  return {seg[s].plane0, seg[s].meta, block / 4, block % 4, seg[s].out_offset, block < seg[s].tiles * 4 ? 1u : 0u};
}

// One wave's K slice of one 16-column block, NT tensors (gate, up): acc[n][b] over row blocks b.
template <uint32_t FMT, int MB, int R, int KS, int NT>
__device__ __forceinline__ void slice_walk(const uint8_t *const (&plane)[NT], const uint8_t *const (&meta)[NT],
                                           const uint16_t *const (&xrow)[2], uint32_t g_begin, uint32_t count,
                                           int q, f32x4 (&acc)[NT][MB]) {
  using F = Fmt<FMT>;
  constexpr int SG = F::SG;
  constexpr int NU = (KS + F::UNIT - 1) / F::UNIT + 1;   // meta units a slice can touch
  uint32_t codes[NT][KS];
  MetaWords units[NT][NU];
  u32x4 x[kPipe][MB];
  const uint32_t unit0 = g_begin / F::UNIT;
  const auto load_x = [&](int slot, uint32_t u) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      if (xrow[b] && u < count) {
        const uint16_t *p = xrow[b] + (g_begin + u) * 32 + 4 * q;
        const u32x2 lo = *(const u32x2 *)p, hi = *(const u32x2 *)(p + 16);
        x[slot][b] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      } else {
        x[slot][b] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  // The first activation fragments, then every code and meta load of the slice.
#pragma unroll
  for (int u = 0; u < kPipe && u < KS; ++u) load_x(u, u);
#pragma unroll
  for (int u = 0; u < KS; ++u)
#pragma unroll
    for (int n = 0; n < NT; ++n)
      codes[n][u] = (uint32_t)u < count ? __builtin_nontemporal_load((const uint32_t *)(plane[n] + (size_t)(g_begin + u) * 1024))
                                        : 0u;
  const uint32_t last_unit = (g_begin + count - 1) / F::UNIT;
#pragma unroll
  for (int v = 0; v < NU; ++v)
#pragma unroll
    for (int n = 0; n < NT; ++n)
      units[n][v] = unit0 + v <= last_unit ? load_meta<FMT>(meta[n] + (size_t)(unit0 + v) * 64 * F::META)
                                           : MetaWords{{0u, 0u, 0u, 0u}};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 c[NT][MB], sx[MB];
#pragma unroll
  for (int u = 0; u < KS; ++u) {
    if ((uint32_t)u >= count) continue;
    const int slot = u % kPipe;
    const uint32_t g = g_begin + u;
    const bool first = u % SG == 0;   // slices start on meta units, so on scale groups
#pragma unroll
    for (int b = 0; b < MB; ++b) sx[b] = mfma_bf16(x[slot][b], ones_operand(), first ? zero : sx[b]);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      const u32x4 w = code_operands(codes[n][u]);
#pragma unroll
      for (int b = 0; b < MB; ++b) c[n][b] = mfma_bf16(x[slot][b], w, first ? zero : c[n][b]);
    }
    if (u + kPipe < KS) load_x(slot, u + kPipe);
    if ((u + 1) % SG == 0) {
      constexpr int kUnitStride = F::UNIT;
      const int v = u / kUnitStride;   // the slice starts on a meta unit
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const Coef k = coef<FMT>(units[n][v], g / SG);
        const float zc = fmaf(-128.0f, k.s, k.z);
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
          for (int i = 0; i < R; ++i) {
            acc[n][b][i] = fmaf(k.s, c[n][b][i], acc[n][b][i]);
            acc[n][b][i] = fmaf(zc, sx[b][i], acc[n][b][i]);
          }
      }
    }
  }
}

template <uint32_t FMT, int MT, int KS, int NT, uint32_t EP, bool F32OUT>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
  using F = Fmt<FMT>;
  constexpr int MB = MT > 16 ? 2 : 1;   // 16-row A blocks
  constexpr int R = MT >= 4 ? 4 : MT;   // accumulator rows each lane group keeps
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;
  const uint32_t nb = a.nb, slices = kWaves / nb, wnb = (uint32_t)wave % nb, slice = (uint32_t)wave / nb;
  const uint32_t block = blockIdx.x * nb + wnb, split = blockIdx.y;
  const BlockPlace at = place(a.seg, a.segments, block);
  const uint32_t G = a.K >> 5, units = G / F::UNIT;
  // Meta units of this split and this slice of it: slices start on meta units, so a group's unit is at a
  // compile-time offset from the slice's first.
  const uint32_t per = units / a.splits;
  const uint32_t s0 = split * per + slice * per / slices, s1 = split * per + (slice + 1) * per / slices;
  const uint32_t g_begin = s0 * F::UNIT, count = at.live ? (s1 - s0) * F::UNIT : 0;

  const uint8_t *plane[NT], *meta[NT];
  const size_t pbase = ((size_t)at.tile * G * 64 + 16 * at.t + j) * 16 + 4 * q;
  const size_t mbase = ((size_t)at.tile * units * 64 + 16 * at.t + j) * F::META;
  plane[0] = (NT == 2 ? a.gate.plane0 : at.plane0) + pbase;
  meta[0] = (NT == 2 ? a.gate.meta : at.meta) + mbase;
  if constexpr (NT == 2) {
    plane[NT - 1] = at.plane0 + pbase;
    meta[NT - 1] = at.meta + mbase;
  }
  const uint16_t *xrow[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const uint32_t r = 16u * b + j;
    xrow[b] = b < MB && r < a.rows ? a.input + (size_t)r * a.K : nullptr;
  }
  f32x4 acc[NT][MB];
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[n][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  slice_walk<FMT, MB, R, KS, NT>(plane, meta, xrow, g_begin, count, q, acc);

  // Slices meet in LDS; the slice-0 wave of each column block adds them in slice order.
  __shared__ float red[kWaves * NT * MB * R * 64];
  const auto at_red = [&](uint32_t w, int n, int b, int i) { return (((w * NT + n) * MB + b) * R + i) * 64 + lane; };
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i) red[at_red(wave, n, b, i)] = acc[n][b][i];
  __syncthreads();
  const bool owner = slice == 0 && at.live;
  float total[NT * MB][R];
  bool live[NT * MB][R];
  size_t index[NT * MB][R];
  const uint32_t col = at.out_offset + at.tile * 64 + 16 * at.t + j;
  const uint32_t cstride = NT == 2 ? 2 * a.out_stride : a.out_stride;
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i) {
        float v = 0.0f;
        for (uint32_t s = 0; s < slices; ++s) v += red[at_red(s * nb + wnb, n, b, i)];
        const uint32_t r = 16u * b + 4u * q + i;
        total[n * MB + b][i] = v;
        live[n * MB + b][i] = r < a.rows;
        index[n * MB + b][i] = (size_t)r * cstride + n * a.out_stride + col;
      }
  if (a.splits > 1 &&
      !split_reduce<NT * MB, R>(total, live, index, a.partials, (size_t)a.rows * cstride, split, a.splits,
                                a.counters + blockIdx.x, owner))
    return;
  if (!owner) return;
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (!live[b][i]) continue;
      const size_t o = (size_t)(16u * b + 4u * q + i) * a.out_stride + col;
      if constexpr (NT == 2) {
        const float g = bf16_to_f32(f32_to_bf16(total[b][i])), u = bf16_to_f32(f32_to_bf16(total[MB + b][i]));
        ((uint16_t *)a.output)[o] = f32_to_bf16(u * silu(g));
      } else {
        const float v = epilogue<EP>(total[b][i], a.aux, o);
        if constexpr (F32OUT) ((float *)a.output)[o] = v;
        else ((uint16_t *)a.output)[o] = f32_to_bf16(v);
      }
    }
}

template <uint32_t FMT, int MT, int NT, uint32_t EP, bool F32OUT>
hipError_t launch_ks(const DecodeArgs &a, uint32_t blocks, uint32_t ks, hipStream_t stream) {
  const dim3 grid(blocks / a.nb, a.splits), block(256);
  if (NT == 2 || ks <= 32) hipLaunchKernelGGL((decode_kernel<FMT, MT, 32, NT, EP, F32OUT>), grid, block, 0, stream, a);
  else hipLaunchKernelGGL((decode_kernel<FMT, MT, 64, NT, EP, F32OUT>), grid, block, 0, stream, a);
  return hipGetLastError();
}

template <uint32_t FMT, int NT, uint32_t EP, bool F32OUT>
hipError_t launch_rows(const DecodeArgs &a, uint32_t blocks, uint32_t ks, hipStream_t stream) {
  if (a.rows <= 1) return launch_ks<FMT, 1, NT, EP, F32OUT>(a, blocks, ks, stream);
  if (a.rows <= 4) return launch_ks<FMT, 4, NT, EP, F32OUT>(a, blocks, ks, stream);
  if (a.rows <= 16) return launch_ks<FMT, 16, NT, EP, F32OUT>(a, blocks, ks, stream);
  return launch_ks<FMT, 32, NT, EP, F32OUT>(a, blocks, ks, stream);
}

template <uint32_t FMT>
hipError_t launch_format(uint32_t epilogue, bool f32_output, bool pair, const DecodeArgs &a, uint32_t blocks,
                         uint32_t ks, hipStream_t stream) {
  if (pair) return launch_rows<FMT, 2, EpNone, false>(a, blocks, ks, stream);
  if (f32_output) return launch_rows<FMT, 1, EpNone, true>(a, blocks, ks, stream);
  switch (epilogue) {
    case EpNone: return launch_rows<FMT, 1, EpNone, false>(a, blocks, ks, stream);
    case EpResidual: return launch_rows<FMT, 1, EpResidual, false>(a, blocks, ks, stream);
    default: return launch_rows<FMT, 1, EpUpWithGate, false>(a, blocks, ks, stream);
  }
}

}  // namespace

DecodeLayout decode_layout(uint32_t fmt, uint32_t blocks, uint32_t K, uint32_t splits, bool pair, uint32_t rows) {
  const uint32_t sg = sq_format(fmt).meta_groups;   // groups of 32 per meta unit
  const uint32_t per = K / 32 / sg / (splits ? splits : 1);   // meta units per split
  if (!sq_format_supported(fmt) || !splits || (K / 32 / sg) % splits || !per || blocks % 4) return {0, 0};
  if (rows <= kColumnTileRows) {
    // The shortest slices (8, 16 or 32 groups; a gate/up pair streams two tensors, at most 16) whose waves fit one
    // workgroup.
    const uint32_t gs = per * sg;
    for (uint32_t ks = 8; ks <= (pair ? kColumnMaxGroups / 2 : kColumnMaxGroups); ks *= 2)
      if ((gs + ks - 1) / ks <= kColumnMaxWaves) return {(gs + ks - 1) / ks, ks};
    return {0, 0};
  }
  const uint32_t most = pair ? 32 : 64;        // groups of 32 a wave holds in registers
  // The fewest slices per column block whose waves hold their slice (widest column blocks per workgroup), among
  // those whose grid fills the device's 256 compute units.
  DecodeLayout best{0, 0};
  for (uint32_t nb = 4; nb >= 1; nb /= 2) {
    const uint32_t slices = kWaves / nb;
    if (blocks % nb) continue;
    const uint32_t ks = (per + slices - 1) / slices * sg;
    if (ks > most) continue;
    best = {nb, ks};
    if (uint64_t{blocks / nb} * splits >= 256) break;
  }
  return best;
}

hipError_t launch_decode(uint32_t fmt, uint32_t epilogue, bool f32_output, const DecodeArgs &args,
                         hipStream_t stream) {
  if (args.rows <= kColumnTileRows) return launch_decode_column(fmt, epilogue, f32_output, args, stream);
  DecodeArgs a = args;
  uint32_t blocks = 0;
  for (uint32_t s = 0; s < a.segments; ++s) blocks += a.seg[s].tiles * 4;
  const bool pair = a.gate.plane0 != nullptr;
  const DecodeLayout layout = decode_layout(fmt, blocks, a.K, a.splits, pair, a.rows);
  if (!layout.nb) return hipErrorInvalidValue;
  a.nb = layout.nb;
  switch (fmt) {
    case SQ_FMT_AF4G32: return launch_format<SQ_FMT_AF4G32>(epilogue, f32_output, pair, a, blocks, layout.ks, stream);
    case SQ_FMT_AF4G64: return launch_format<SQ_FMT_AF4G64>(epilogue, f32_output, pair, a, blocks, layout.ks, stream);
    case SQ_FMT_AF4G128: return launch_format<SQ_FMT_AF4G128>(epilogue, f32_output, pair, a, blocks, layout.ks, stream);
    case SQ_FMT_Q4K: return launch_format<SQ_FMT_Q4K>(epilogue, f32_output, pair, a, blocks, layout.ks, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sq::kern
