// MoE block: top-k route select and shared-slice weights, grouping of routes into expert tiles, the expert passes
// (gate and up in one pass, then down) and the combine (reference: kernels/shared/moe.metal:23-162,175-331,480-505
// and kernels/shared/moe_gguf.metal:21-206).
//
// CDNA4 mapping. Each expert pass is the decode row tile's exact-operand inner loop (rowtile.hpp) per expert tile:
// a wave streams one 64-column plane tile of its expert over all of K against the tile's (at most 32) grouped
// rows; an expert's other tiles read the same weights while they are still in L2. The passes read their input rows
// in the tile's read order (one 16-byte load per row block and group): the routed work opens by writing the block's
// input rows in that order, and the gate/up pass writes the intermediate rows in it.
#include "kernels.hpp"
#include "rowtile.hpp"

namespace sq::kern {
namespace {

// A 64-lane reduction by DPP row operations (dpp_ctrl quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror,
// row_mirror, then row_bcast15 into rows 1 and 3 and row_bcast31 into rows 2 and 3): after the six steps lane 63
// holds op over all 64 lanes, which readlane gives every lane. op must be associative, commutative and idempotent
// (a row the mask leaves out combines a value with itself).
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_row(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWS, 0xF, false);
}
template <typename Op>
__device__ __forceinline__ uint32_t wave_reduce(uint32_t v, Op op) {
  v = op(v, dpp_row<0xB1, 0xF>(v));
  v = op(v, dpp_row<0x4E, 0xF>(v));
  v = op(v, dpp_row<0x141, 0xF>(v));
  v = op(v, dpp_row<0x140, 0xF>(v));
  v = op(v, dpp_row<0x142, 0xA>(v));
  v = op(v, dpp_row<0x143, 0xC>(v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// One wave per row (moe.metal:23-112). Rank by rank, the highest remaining score wins, the lowest expert id among
// equal scores; the router then weights the top_k routes in rank order: Softmax weight_r =
// 2^((s_r - s_0) log2 e) / sum_o 2^((s_o - s_0) log2 e), SigmoidNormalized weight_r = sigmoid(s_r) /
// (sum_o sigmoid(s_o) + 1e-20). The row's routes top_k .. top_k + shared - 1 are the shared expert's slices (ids
// experts on), each weighted by sigmoid(x . g) of the block's fp32 scalar gate g (gated) or by 1.
__global__ __launch_bounds__(128) void route_select_kernel(const float *scores, uint32_t stride, uint32_t *selected,
                                                          float *weights, SqMoeRouteParams p, const uint16_t *input,
                                                          const float *shared_gate, uint32_t router, uint32_t shared,
                                                          uint16_t *rows_table) {
  constexpr int kPer = SQ_MOE_WIDE_EXPERT_SLOTS / 64;
  const uint32_t row = blockIdx.x, lane = threadIdx.x & 63, per_row = p.top_k + shared;
  const size_t base = (size_t)row * per_row;
  if (threadIdx.x >= 64) {
    // The second wave (launched with rows_table only): the row in the tiles' read order (input_rows_kernel's 16-byte
    // chunks, lane l the row's chunks l, l + 64, ...), beside the first wave's selection.
    const uint16_t *xr = input + (size_t)row * p.input_size;
    uint16_t *out = rows_table + (size_t)row * p.input_size;
    for (uint32_t i = lane; i < p.input_size / 8; i += 64) {
      const uint32_t *in = (const uint32_t *)(xr + 32 * (i / 4)) + 2 * (i % 4);
      const u32x2 lo = *(const u32x2 *)in, hi = *(const u32x2 *)(in + 8);
      *(u32x4 *)(out + 8 * i) = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
    return;
  }
  if (shared) {
    float gate = 1.0f;
    if (shared_gate) {
      float dot = 0.0f;
      const uint16_t *xr = input + (size_t)row * p.input_size;
      if (p.input_size % 512 == 0) {
        // Eight inputs a lane a step (one 16-byte load of the row, two of the gate), four steps' loads in flight.
#pragma unroll 4
        for (uint32_t d = 8 * lane; d < p.input_size; d += 512) {
          const u32x4 x = *(const u32x4 *)(xr + d);
          const f32x4 g0 = *(const f32x4 *)(shared_gate + d), g1 = *(const f32x4 *)(shared_gate + d + 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float ge = e < 2 ? g0[2 * e] : g1[2 * e - 4], go = e < 2 ? g0[2 * e + 1] : g1[2 * e - 3];
            dot = fmaf(bf16_to_f32(x[e] & 0xFFFFu), ge, dot);
            dot = fmaf(bf16_to_f32(x[e] >> 16), go, dot);
          }
        }
      } else {
        for (uint32_t d = lane; d < p.input_size; d += 64) dot = fmaf(bf16_to_f32(xr[d]), shared_gate[d], dot);
      }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) dot += __shfl_xor(dot, m);
      gate = sigmoid(dot);
    }
    if (lane < shared) {
      selected[base + p.top_k + lane] = p.experts + lane;
      weights[base + p.top_k + lane] = gate;
    }
  }
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t e = lane + 64u * i;
    v[i] = e < p.experts ? scores[(size_t)row * stride + e] : -INFINITY;
  }
  __shared__ float ordered[64];
  // A lane's best starts at -inf in its first slot and moves only to a strictly greater score, so a NaN score never
  // becomes a lane's best and the wave maximum sees no NaN; a taken expert's score becomes -inf (moe.metal:77-93).
  // Every lane offers at least its first slot, so the winner is always an expert id below `experts`: when no finite
  // score is left, every lane's best is -inf and lane 0's expert 0 wins (the reference's choice too).
  for (uint32_t rank = 0; rank < p.top_k; ++rank) {
    float best = -INFINITY;
    int at = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (v[i] > best) best = v[i], at = i;
    const float top = __uint_as_float(wave_reduce(__float_as_uint(best), [](uint32_t a, uint32_t b) {
      return __float_as_uint(fmaxf(__uint_as_float(a), __uint_as_float(b)));
    }));
    const uint32_t candidate = best == top ? lane + 64u * at : 0xFFFFFFFFu;
    const uint32_t winner = wave_reduce(candidate, [](uint32_t a, uint32_t b) { return min(a, b); });
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (candidate == winner && i == at) v[i] = -INFINITY;
    if (lane == 0) {
      selected[base + rank] = winner;
      ordered[rank] = top;
    }
  }
  // One wave selects (a second one, if any, returned above): lane 0's LDS writes reach its other lanes.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (uint32_t rank = lane; rank < p.top_k; rank += 64) {
    float denominator = 0.0f;
    if (router == SQ_MOE_ROUTER_SOFTMAX) {
      for (uint32_t o = 0; o < p.top_k; ++o) denominator += exp2f((ordered[o] - ordered[0]) * 1.44269504089f);
      weights[base + rank] = exp2f((ordered[rank] - ordered[0]) * 1.44269504089f) / denominator;
    } else {
      for (uint32_t o = 0; o < p.top_k; ++o) denominator += sigmoid(ordered[o]);
      weights[base + rank] = sigmoid(ordered[rank]) / (denominator + 1e-20f);
    }
  }
}

// One workgroup groups every route (moe.metal:184-278): count per expert, exclusive prefix of the experts' tiles in
// expert order, tile descriptors, then each routed route's grouped row. Routes of an expert take its rows in route
// order (a bitmap of the rows that route to each expert, 512 rows at a time, gives a route's rank), so the
// grouping, and every expert pass after it, is deterministic. The `shared` slices' tiles follow the routed tiles,
// slice after slice, each slice's holding every row in order (route row * (top_k + shared) + top_k + slice).
// With verify_rows (a verify step: a live-row count per lane of lane_rows rows) the routed routes of a row past its
// lane's count are grouped into no tile and their route_rows are ~0u (moe_group_routes_verified,
// moe.metal:164-173); the shared slices still hold every row.
__global__ __launch_bounds__(512) void group_kernel(const uint32_t *selected, SqMoeTileDescriptor *tiles,
                                                    SqMoeTileCount *tile_count, uint32_t *grouped_routes,
                                                    uint32_t *route_rows, const uint32_t *verify_rows,
                                                    SqMoeGroupParams p, uint32_t shared) {
  // The row bitmaps and their prefixes: an expert's kWords words at a stride of kStride, so that the threads that
  // walk their experts' words together (thread e, word w) take different LDS banks.
  constexpr uint32_t kChunk = 512, kWords = kChunk / 32, kStride = kWords + 1;
  __shared__ uint32_t counts[SQ_MOE_WIDE_EXPERT_SLOTS], offsets[SQ_MOE_WIDE_EXPERT_SLOTS],
      running[SQ_MOE_WIDE_EXPERT_SLOTS];
  __shared__ uint32_t bits[SQ_MOE_WIDE_EXPERT_SLOTS * kStride], prefix[SQ_MOE_WIDE_EXPERT_SLOTS * kStride];
  __shared__ uint32_t total;
  const uint32_t tid = threadIdx.x, per_row = p.top_k + shared, tr = p.tile_rows;
  // Routed route k of row r: selected[r * per_row + k].
  const auto route_of = [&](uint32_t i) { return i / p.top_k * per_row + i % p.top_k; };
  // The route select writes expert ids below `experts` only; the clamp keeps a corrupted selection inside the
  // tables below.
  const auto expert_of = [&](uint32_t i) { return min(selected[route_of(i)], p.experts - 1u); };
  const auto dead = [&](uint32_t i) {
    const uint32_t row = i / p.top_k;
    return verify_rows != nullptr && row % p.lane_rows >= verify_rows[row / p.lane_rows];
  };
  // When one chunk takes every row and a row has at most kHeld routes, each thread loads its routes' expert ids once
  // (route tid + 512 k, k < top_k), counts them and sets their row bits in one pass, and ranks them from registers:
  // one read of the selection instead of three. Up to kStaged routes otherwise go through LDS once (each route's
  // expert id, ~0u for a dead one), which the passes below read instead of the selection.
  constexpr uint32_t kHeld = 8, kStaged = 4 * kChunk * kHeld;
  const uint32_t routes = p.rows * p.top_k;
  const bool one = p.rows <= kChunk && p.top_k <= kHeld, staged = !one && routes <= kStaged;
  __shared__ uint32_t stage[kStaged];
  // Route i's expert, or ~0u for a dead route.
  const auto live_expert = [&](uint32_t i) __attribute__((always_inline)) {
    return staged ? stage[i] : dead(i) ? ~0u : expert_of(i);
  };
  uint32_t held[kHeld];
#pragma unroll
  for (uint32_t k = 0; k < kHeld; ++k) {
    const uint32_t i = tid + 512 * k;
    held[k] = one && i < routes && !dead(i) ? expert_of(i) : ~0u;   // ~0u: no live route
  }
  __shared__ uint32_t duplicated;
  counts[tid] = 0;
  running[tid] = 0;
  if (one) {
    for (uint32_t i = tid; i < p.experts * kStride; i += 512) bits[i] = 0;
    if (tid == 0) duplicated = 0;
  }
  __syncthreads();
  if (one) {
#pragma unroll
    for (uint32_t k = 0; k < kHeld; ++k) {
      const uint32_t i = tid + 512 * k;
      if (i >= routes) continue;
      if (held[k] == ~0u) {
        route_rows[route_of(i)] = ~0u;
        continue;
      }
      const uint32_t local = i / p.top_k, bit = 1u << (local % 32);
      atomicAdd(&counts[held[k]], 1u);
      // A bit already set names another route of the same row to the same expert (see below).
      if (atomicOr(&bits[held[k] * kStride + local / 32], bit) & bit) duplicated = 1;
    }
  } else {
    for (uint32_t i = tid; i < routes; i += 512) {
      const uint32_t e = dead(i) ? ~0u : expert_of(i);
      if (staged) stage[i] = e;
      if (e != ~0u) atomicAdd(&counts[e], 1u);
    }
  }
  __syncthreads();
  {
    // Exclusive prefix of the experts' tile counts: a scan within each wave, then over the eight wave totals.
    __shared__ uint32_t wave_sum[8];
    const uint32_t mine = tid < p.experts ? (counts[tid] + tr - 1) / tr : 0u, lane = tid & 63, wave = tid >> 6;
    uint32_t inclusive = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t up = (uint32_t)__shfl_up((int)inclusive, d);
      if (lane >= (uint32_t)d) inclusive += up;
    }
    if (lane == 63) wave_sum[wave] = inclusive;
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t w = 0; w < wave; ++w) before += wave_sum[w];
    offsets[tid] = before + inclusive - mine;
    if (tid == 511) total = before + inclusive;
  }
  __syncthreads();
  if (tid < p.experts) {
    const uint32_t c = counts[tid], n = (c + tr - 1) / tr, first = offsets[tid];
    for (uint32_t t = 0; t < n; ++t) tiles[first + t] = SqMoeTileDescriptor{tid, min(tr, c - t * tr)};
    for (uint32_t row = first * tr + c; row < (first + n) * tr; ++row) grouped_routes[row] = ~0u;
  }
  for (uint32_t chunk = 0; chunk < p.rows; chunk += kChunk) {
    const uint32_t i0 = chunk * p.top_k, i1 = min(p.rows, chunk + kChunk) * p.top_k;
    if (!one) {
      for (uint32_t i = tid; i < p.experts * kStride; i += 512) bits[i] = 0;
      if (tid == 0) duplicated = 0;
      __syncthreads();
    }
    for (uint32_t i = i0 + tid; !one && i < i1; i += 512) {
      const uint32_t e = live_expert(i);
      if (e == ~0u) {
        route_rows[route_of(i)] = ~0u;
        continue;
      }
      const uint32_t local = i / p.top_k - chunk, bit = 1u << (local % 32);
      // A bit already set names another route of the same row to the same expert: a row with fewer scores above
      // -inf than top_k routes (an all-NaN row selects expert 0 at every rank). Such a chunk is ranked serially.
      if (atomicOr(&bits[e * kStride + local / 32], bit) & bit) duplicated = 1;
    }
    __syncthreads();
    if (!duplicated) {
      // Rows of the chunk before word w that route to expert e: one pass per expert, then each route's rank is a
      // table read and one population count.
      if (tid < p.experts) {
        uint32_t before = 0;
        for (uint32_t w = 0; w < kWords; ++w) {
          prefix[tid * kStride + w] = before;
          before += __popc(bits[tid * kStride + w]);
        }
      }
      __syncthreads();
      const auto place = [&](uint32_t i, uint32_t e) __attribute__((always_inline)) {
        const uint32_t r = route_of(i), local = i / p.top_k - chunk;
        uint32_t rank = running[e] + prefix[e * kStride + local / 32];
        rank += __popc(bits[e * kStride + local / 32] & ((1u << (local % 32)) - 1u));
        const uint32_t row = offsets[e] * tr + rank;
        grouped_routes[row] = r;
        route_rows[r] = row;
      };
      if (one) {
#pragma unroll
        for (uint32_t k = 0; k < kHeld; ++k)
          if (tid + 512 * k < routes && held[k] != ~0u) place(tid + 512 * k, held[k]);
      } else {
        for (uint32_t i = i0 + tid; i < i1; i += 512) {
          const uint32_t e = live_expert(i);
          if (e != ~0u) place(i, e);
        }
      }
      __syncthreads();
      if (tid < p.experts) {
        uint32_t ranked = running[tid];
        for (uint32_t w = 0; w < kWords; ++w) ranked += __popc(bits[tid * kStride + w]);
        running[tid] = ranked;
      }
    } else if (tid < p.experts) {
      // Thread e takes its expert's routes of the chunk in route order.
      for (uint32_t i = i0; i < i1; ++i) {
        if (live_expert(i) != tid) continue;
        const uint32_t r = route_of(i), row = offsets[tid] * tr + running[tid]++;
        grouped_routes[row] = r;
        route_rows[r] = row;
      }
    }
    __syncthreads();
  }
  // Shared slices (moe.metal:245-270): slice s's tiles after slice s - 1's, each of every row in order.
  const uint32_t shared_tiles = (p.rows + tr - 1) / tr, shared_base = total * tr;
  for (uint32_t i = tid; i < shared * shared_tiles; i += 512) {
    const uint32_t slice = i / shared_tiles, t = i % shared_tiles;
    tiles[total + i] = SqMoeTileDescriptor{p.experts + slice, min(tr, p.rows - t * tr)};
  }
  for (uint32_t i = tid; i < shared * shared_tiles * tr; i += 512) {
    const uint32_t slice = i / (shared_tiles * tr), row = i % (shared_tiles * tr);
    if (row < p.rows) {
      const uint32_t r = row * per_row + p.top_k + slice;
      grouped_routes[shared_base + i] = r;
      route_rows[r] = shared_base + i;
    } else {
      grouped_routes[shared_base + i] = ~0u;
    }
  }
  if (tid == 0) {
    const uint32_t live = total + shared * shared_tiles;
    *tile_count = SqMoeTileCount{live, {p.gate_up_columns, live, 1}, {p.down_columns, live, 1}, {0, 0, 0}};
  }
}

// Workgroup (four 64-column tiles, expert tile): wave w streams column tile 4 blockIdx.x + w of the tile's expert
// over all of K against the tile's rows (at most 32: the expert's grouped rows from tile * tile_rows), so each
// wave owns its outputs and no wave waits on another. The gate/up pass reads its rows through the grouped routes
// (row r of the tile is input row routes[r] / top_k: the reference's gather copy folds into these loads) and
// writes bf16(bf16(up) silu(bf16(gate))); a gate and up of different formats run as two such gathering passes, the
// gate's output feeding the up pass's epilogue; the down pass reads the grouped intermediate rows
// (moe_gguf.metal:121-206, moe_expert_slab.h:13-99).
// The passes that stream chunks of two groups with operands built just before their MFMAs: those of 4-bit affine
// codes in groups of 32 or 64 (a gate/up pair then fits two waves a SIMD, a single tensor three), every
// single-tensor pass whose scale groups fit a two-group chunk (the K-quants and 8-bit codes then fit two waves a SIMD
// instead of one), and the Q4_K and Q5_K gate/up pairs, whose coefficients each lane derives for its own column only
// (rowtile.hpp: 239 and 250 registers, two waves a SIMD). The other gate/up pairs (Q6_K's halves, 8-bit codes, groups
// of 128) would spill there and keep four-group chunks with operands a group ahead, one wave a SIMD. Chunks hold
// whole scale groups either way, so the sums are the same bits.
template <uint32_t FMT>
constexpr bool affine4_short() { return FMT == SQ_FMT_AF4G32 || FMT == SQ_FMT_AF4G64; }
template <uint32_t FMT, int NT>
constexpr bool short_chunks() {
  return affine4_short<FMT>() || (NT == 1 && Fmt<FMT>::SG <= 2) || FMT == SQ_FMT_Q4K || FMT == SQ_FMT_Q5K;
}
template <uint32_t FMT, int NT>
constexpr int expert_waves() { return affine4_short<FMT>() ? (NT == 2 ? 2 : 3) : short_chunks<FMT, NT>() ? 2 : 1; }

// Rows row0..row0 + rows - 1 of tile `tile` (all of them, or a 16-row half of it).
template <uint32_t FMT, int MB, int NT>
__device__ __forceinline__ void expert_tile(const MoeExpertArgs &a, SqMoeTileDescriptor d, uint32_t tile,
                                            uint32_t ct, uint32_t row0, uint32_t rows) {
  using F = Fmt<FMT>;
  const uint32_t column_tiles = a.output_size / 64;
  const uint32_t first_row = tile * a.tile_rows + row0;
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const uint32_t G = a.K >> 5;
  // The plane tile: routed expert e's from tile slots[e] of its projection on, shared slice s's from tile s of the
  // shared segment on.
  const bool shared = d.expert >= a.experts;
  // A down pass of two tensor slots (pair) streams column tiles ct and ct + 1 of its one tensor, both against the
  // same input loads.
  const bool pair = NT == 2 && !a.gate_up;
  const uint32_t ptile = (shared ? d.expert - a.experts : a.slots[d.expert]) * column_tiles + ct;
  const uint8_t *plane[NT], *high[NT], *meta[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const int slot = pair ? 0 : n;
    const size_t pt = ptile + (pair ? n : 0);
    plane[n] = (shared ? a.shared_plane0[slot] : a.plane0[slot]) + (pt * G * 64 + lane) * F::P0;
    high[n] = F::P1 ? (shared ? a.shared_plane1[slot] : a.plane1[slot]) + (pt * G * 64 + lane) * F::P1 : nullptr;
    meta[n] = (shared ? a.shared_meta[slot] : a.meta[slot]) + (pt * (G / F::UNIT) * 64 + lane) * F::META;
  }
  // Lane (j, q) of row block b reads row 16 b + j (row 0 past the tile's rows: nothing stores those results), its
  // 16-byte chunk q of each group in the read order.
  const uint16_t *xrow[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    const uint32_t r = 16u * b + j < rows ? 16u * b + j : 0u;
    const uint32_t source = a.gather ? a.routes[first_row + r] / a.routes_per_row : first_row + r;
    xrow[b] = a.input + (size_t)source * a.K + 8 * q;
  }
  float acc[NT][4][MB][4];
  clear(acc);
  // Two register sets (one chunk of loads ahead): the passes are bound by instruction issue, and a third set for a
  // gate/up pair only moves more of its MFMA results through the accumulation registers. Short chunks fit more
  // waves a SIMD (expert_kernel), and each resident wave covers more of the others' dependency stalls.
  constexpr bool kShort = short_chunks<FMT, NT>();
  row_stream<FMT, MB, NT, 2, kShort ? 2 : 4, !kShort>(plane, high, meta, xrow, G, acc);
  // Column 16 t + j of the tile: the gathering passes store it at its place in the read order (chunk 4 g + j / 4 of
  // group g = 2 ct + t / 2, then position 4 (t % 2) + j % 4), for the down pass; the down pass in column order.
  const uint32_t column = a.gather ? 8 * (j >> 2) + (j & 3) : j;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t r = 16u * b + 4u * q + i;
        if (r >= rows) continue;
        const uint32_t c = a.gather ? 32 * (t >> 1) + 4 * (t & 1) + column : 16 * t + column;
        const size_t at = (size_t)(first_row + r) * a.output_size + ct * 64 + c;
        if (pair) {
          a.output[at] = f32_to_bf16(acc[0][t][b][i]);
          a.output[at + 64] = f32_to_bf16(acc[NT - 1][t][b][i]);
        } else if constexpr (NT == 2) {
          const float g = bf16_to_f32(f32_to_bf16(acc[0][t][b][i])), u = bf16_to_f32(f32_to_bf16(acc[1][t][b][i]));
          a.output[at] = f32_to_bf16(u * silu(g));
        } else if (a.gate) {
          const float u = bf16_to_f32(f32_to_bf16(acc[0][t][b][i]));
          a.output[at] = f32_to_bf16(u * silu(bf16_to_f32(a.gate[at])));
        } else {
          a.output[at] = f32_to_bf16(acc[0][t][b][i]);
        }
      }
}

// The tile workgroup row y runs, longest first: the tiles of more than 16 rows (two row blocks, about twice the work)
// in tile order, then the others in tile order, so that the cheap tiles fill the compute units' last round instead of
// a few expensive ones trailing it. The workgroup ranks the live tiles itself (each thread counts a run of them, then
// a scan of the counts); past kOrderedTiles live tiles it keeps the tile order.
constexpr uint32_t kOrderedTiles = 2048;
__device__ uint32_t longest_first_tile(const SqMoeTileDescriptor *tiles, uint32_t n, uint32_t y) {
  constexpr uint32_t kThreads = 256, kWaves = kThreads / 64;
  __shared__ uint32_t wave_total[kWaves], picked;
  if (n > kOrderedTiles) return y;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t run = (n + kThreads - 1) / kThreads, begin = min(n, tid * run), end = min(n, begin + run);
  uint32_t big = 0;
  for (uint32_t t = begin; t < end; ++t) big += tiles[t].rows > 16;
  // Inclusive scan of the threads' counts of big tiles.
  uint32_t inclusive = big;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t up = (uint32_t)__shfl_up((int)inclusive, d);
    if (lane >= (uint32_t)d) inclusive += up;
  }
  if (lane == 63) wave_total[wave] = inclusive;
  __syncthreads();
  uint32_t before = 0, all = 0;
#pragma unroll
  for (uint32_t w = 0; w < kWaves; ++w) {
    before += w < wave ? wave_total[w] : 0u;
    all += wave_total[w];
  }
  const uint32_t big_before = before + inclusive - big;   // big tiles before this thread's run
  // Row y takes big tile y (y < all), else small tile y - all; the thread whose run holds it writes its index.
  const bool want_big = y < all;
  const uint32_t rank = want_big ? y : y - all;
  const uint32_t mine_before = want_big ? big_before : begin - big_before, mine = want_big ? big : end - begin - big;
  if (rank >= mine_before && rank < mine_before + mine) {
    uint32_t seen = mine_before;
    for (uint32_t t = begin; t < end; ++t)
      if ((tiles[t].rows > 16) == want_big && seen++ == rank) {
        picked = t;
        break;
      }
  }
  __syncthreads();
  return picked;
}

// Tiles of at most 16 rows (most of an expert's last tiles) take the one-block path. With row_halves the grid's x
// holds two copies of the column groups, and copy h takes rows 16 h..16 h + 15 of each tile on the one-block path
// (a launch of few tiles then fills twice the SIMDs; each row computes what it does in the whole tile).
template <uint32_t FMT, int MB, int NT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(expert_waves<FMT, NT>())))
void expert_kernel(MoeExpertArgs a) {
  const uint32_t n = a.tile_count->tiles;
  if (blockIdx.y >= n) return;
  const uint32_t tile = longest_first_tile(a.tiles, n, blockIdx.y);
  const uint32_t groups = a.row_halves ? gridDim.x / 2 : gridDim.x, half = blockIdx.x / groups;
  const uint32_t ct = (blockIdx.x % groups * 4 + (threadIdx.x >> 6)) * (NT == 2 && !a.gate_up ? 2 : 1);
  if (ct >= a.output_size / 64) return;
  const SqMoeTileDescriptor d = a.tiles[tile];
  if (a.mode != 2 && (d.expert >= a.experts) != (a.mode == 1)) return;
  if (a.row_halves) {
    if (16 * half < d.rows) expert_tile<FMT, 1, NT>(a, d, tile, ct, 16 * half, min(16u, d.rows - 16 * half));
    return;
  }
  if (MB == 1 || d.rows <= 16) expert_tile<FMT, 1, NT>(a, d, tile, ct, 0, d.rows);
  else expert_tile<FMT, MB, NT>(a, d, tile, ct, 0, d.rows);
}

// Thread: one 16-byte chunk of the table, chunk c of a group of 32 inputs: its 4-input units c and c + 4 (inputs
// 4c..4c+3 and 16+4c..19+4c, the group's dwords 2c, 2c + 1 and 8 + 2c, 9 + 2c), the prefill's half rows order
// (half_rows.hpp). The reference's routed pass opens with its gather of the input rows into the grouped input
// (MoE.cpp:480-517); here the rows keep their order and the gate/up pass gathers through the routes as it reads.
// Four threads a group, so each wave reads and writes 1 KiB contiguous.
__global__ __launch_bounds__(256) void input_rows_kernel(const uint16_t *input, uint64_t chunks, uint16_t *table) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;   // chunk i % 4 of group i / 4, rows back to back
  if (i >= chunks) return;
  const uint32_t *in = (const uint32_t *)(input + 32 * (i / 4)) + 2 * (i % 4);
  const u32x2 lo = *(const u32x2 *)in, hi = *(const u32x2 *)(in + 8);
  *(u32x4 *)(table + 8 * i) = u32x4{lo[0], lo[1], hi[0], hi[1]};
}

// out[r][d] = bf16(residual + sum_slot w_slot * expert_out[route_rows[slot]][d]) in slot order (moe.metal:480-505).
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t *expert_output, const uint32_t *route_rows,
                                                      const float *weights, const uint16_t *residual,
                                                      uint16_t *output, SqMoeCombineParams p) {
  // Thread: eight consecutive outputs of row blockIdx.x (the hidden size is a multiple of 64).
  const uint32_t r = blockIdx.x, d = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (d >= p.hidden_size) return;
  const size_t at = (size_t)r * p.hidden_size + d;
  float v[8];
  const u32x4 res = residual ? *(const u32x4 *)(residual + at) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 4; ++e) v[2 * e] = bf16_to_f32(res[e] & 0xFFFFu), v[2 * e + 1] = bf16_to_f32(res[e] >> 16);
  const size_t route = (size_t)r * p.routes_per_row;
  // Eight slots at a time: their route rows (one scalar load each: the row is the workgroup's), then every live
  // slot's 16 bytes in flight together, then the sums in slot order; the slots past the last eight one at a time. A
  // route row of ~0u (a dead verify row) adds nothing, not even a zero.
  constexpr uint32_t kBatch = 8;
  uint32_t s0 = 0;
  for (; s0 + kBatch <= p.routes_per_row; s0 += kBatch) {
    uint32_t grouped[kBatch];
    u32x4 x[kBatch];
    float w[kBatch];
#pragma unroll
    for (uint32_t k = 0; k < kBatch; ++k) {
      grouped[k] = route_rows[route + s0 + k];
      w[k] = 0.0f;
      x[k] = u32x4{0u, 0u, 0u, 0u};
      if (grouped[k] != ~0u) {
        w[k] = weights[route + s0 + k];
        x[k] = *(const u32x4 *)(expert_output + (size_t)grouped[k] * p.hidden_size + d);
      }
    }
#pragma unroll
    for (uint32_t k = 0; k < kBatch; ++k) {
      if (grouped[k] == ~0u) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = fmaf(w[k], bf16_to_f32(x[k][e] & 0xFFFFu), v[2 * e]);
        v[2 * e + 1] = fmaf(w[k], bf16_to_f32(x[k][e] >> 16), v[2 * e + 1]);
      }
    }
  }
  for (; s0 < p.routes_per_row; ++s0) {
    const uint32_t grouped = route_rows[route + s0];
    if (grouped == ~0u) continue;
    const float w = weights[route + s0];
    const u32x4 x = *(const u32x4 *)(expert_output + (size_t)grouped * p.hidden_size + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = fmaf(w, bf16_to_f32(x[e] & 0xFFFFu), v[2 * e]);
      v[2 * e + 1] = fmaf(w, bf16_to_f32(x[e] >> 16), v[2 * e + 1]);
    }
  }
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = (uint32_t)f32_to_bf16(v[2 * e]) | ((uint32_t)f32_to_bf16(v[2 * e + 1]) << 16);
  *(u32x4 *)(output + at) = out;
}

template <uint32_t FMT, int MB, int NT>
hipError_t launch_expert_rows(const MoeExpertArgs &a, hipStream_t stream) {
  const uint32_t per = NT == 2 && !a.gate_up ? 8 : 4;   // column tiles a workgroup
  const dim3 grid((a.output_size / 64 + per - 1) / per * (a.row_halves ? 2 : 1), a.max_tiles), block(256);
  hipLaunchKernelGGL((expert_kernel<FMT, MB, NT>), grid, block, 0, stream, a);
  return hipGetLastError();
}

// The down pass over 4-bit affine codes in groups of 32 or 64 streams column tiles in pairs (an even count of them):
// each input load then serves two tiles, for the same registers as a gate/up pair (two waves a SIMD instead of three;
// the pass is bound by its vector memory instructions more than by its waves: c4 174 -> 168 us).
template <uint32_t FMT>
hipError_t launch_expert_format(const MoeExpertArgs &a, hipStream_t stream) {
  const bool pairs = affine4_short<FMT>() && !a.gate_up && !a.gather && (a.output_size / 64) % 2 == 0;
  if (a.tile_rows <= 16 || a.row_halves)
    return a.gate_up || pairs ? launch_expert_rows<FMT, 1, 2>(a, stream) : launch_expert_rows<FMT, 1, 1>(a, stream);
  return a.gate_up || pairs ? launch_expert_rows<FMT, 2, 2>(a, stream) : launch_expert_rows<FMT, 2, 1>(a, stream);
}

}  // namespace

hipError_t launch_moe_route_select(const float *scores, uint32_t stride, uint32_t *selected, float *weights,
                                   const SqMoeRouteParams &p, const uint16_t *input, const float *shared_gate,
                                   uint32_t router, uint32_t shared, uint16_t *rows_table, hipStream_t stream) {
  if (rows_table && p.input_size % 32) return hipErrorInvalidValue;
  hipLaunchKernelGGL(route_select_kernel, dim3(p.rows), dim3(rows_table ? 128 : 64), 0, stream, scores, stride,
                     selected, weights, p, input, shared_gate, router, shared, rows_table);
  return hipGetLastError();
}

hipError_t launch_moe_group(const uint32_t *selected, SqMoeTileDescriptor *tiles, SqMoeTileCount *tile_count,
                            uint32_t *grouped_routes, uint32_t *route_rows, const uint32_t *verify_rows,
                            const SqMoeGroupParams &p, uint32_t shared, hipStream_t stream) {
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(512), 0, stream, selected, tiles, tile_count, grouped_routes,
                     route_rows, verify_rows, p, shared);
  return hipGetLastError();
}

hipError_t launch_moe_input_rows(const uint16_t *input, uint32_t rows, uint32_t K, uint16_t *table,
                                 hipStream_t stream) {
  if (K % 32) return hipErrorInvalidValue;
  const uint64_t chunks = (uint64_t)rows * (K / 32) * 4;
  hipLaunchKernelGGL(input_rows_kernel, dim3((uint32_t)((chunks + 255) / 256)), dim3(256), 0, stream, input, chunks,
                     table);
  return hipGetLastError();
}

hipError_t launch_moe_expert(const MoeExpertArgs &a, hipStream_t stream) {
  switch (a.fmt) {
    case SQ_FMT_AF4G32: return launch_expert_format<SQ_FMT_AF4G32>(a, stream);
    case SQ_FMT_AF4G64: return launch_expert_format<SQ_FMT_AF4G64>(a, stream);
    case SQ_FMT_AF4G128: return launch_expert_format<SQ_FMT_AF4G128>(a, stream);
    case SQ_FMT_Q4K: return launch_expert_format<SQ_FMT_Q4K>(a, stream);
    case SQ_FMT_Q5K: return launch_expert_format<SQ_FMT_Q5K>(a, stream);
    case SQ_FMT_Q6K: return launch_expert_format<SQ_FMT_Q6K>(a, stream);
    case SQ_FMT_Q80: return launch_expert_format<SQ_FMT_Q80>(a, stream);
    case SQ_FMT_AF8G64: return launch_expert_format<SQ_FMT_AF8G64>(a, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_moe_combine(const uint16_t *expert_output, const uint32_t *route_rows, const float *weights,
                              const uint16_t *residual, uint16_t *output, const SqMoeCombineParams &p,
                              hipStream_t stream) {
  hipLaunchKernelGGL(combine_kernel, dim3(p.rows, (p.hidden_size / 8 + 255) / 256), dim3(256), 0, stream, expert_output,
                     route_rows, weights, residual, output, p);
  return hipGetLastError();
}

}  // namespace sq::kern
