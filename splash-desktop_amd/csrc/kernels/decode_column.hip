// The column tile of the decode GEMV: y[r][c] = sum_k x[r][k] w[c][k] for one to four rows of bf16 activations
// against plane weights of any format this build takes, fp32 accumulation (reference: gguf_decode / gguf_decode_tile,
// kernels/shared/gguf_linear.metal:71-192, with its K-split reduction, kernels/shared/split_reduce.h:14-45).
//
// CDNA4 mapping. The GEMV is HBM-bound at 0.5625 bytes per weight, so every lane owns one output column of a
// 64-column plane tile and the wave reads the tile's codes as they lie in the plane: per group of 32 inputs, one
// 16-byte load per lane (the column's 32 codes) and 1 KiB per wave, fully coalesced.
//  - The 32 codes become 32 exact bf16 operands 128 + q (one v_and_or_b32 per operand pair, code_pairs) and
//    meet the activations in eight 4x4x4 bf16 MFMAs whose B is the lane's own column (two accumulation chains); the
//    activations (A) of the MFMA's sixteen blocks are broadcast from one block (cbsz 4, abid): lane (b, i) holds row
//    i's inputs 4b..4b+3 of a pair of groups, so one 8-byte load per lane covers 64 inputs of up to four rows, and D
//    gives each lane its own column for the four rows.
//  - Each scale group closes in fp32: acc += s * sum x (128 + q) + (z - 128 s) * sum x, every product exact. The
//    rows' input sums of every group of the slice (of each half, for Q6_K) are summed once, before the slice's
//    stream, by eight lanes a group in a fixed DPP tree, and parked in the wave's own LDS; a close reads them with one
//    broadcast LDS read, so the stream's instructions are the operands, the MFMAs and the closes alone (the VALU
//    issue of the operands is what bounds this tile: a wave64 VALU instruction holds its SIMD four cycles).
//  - A workgroup of W waves takes one tile and W K slices of GW groups each (the split's last slice may be
//    shorter; slices start on meta units). Each wave streams its slice with P groups in flight: codes, meta and
//    activations are issued in the order they are consumed, every load unconditional (addresses past the slice
//    repeat its last group and are not computed on), so the wait counts stay exact and every wave draws bandwidth
//    for the whole dispatch instead of in one burst. The slices meet in LDS in slice order, each row's outputs
//    summed and stored by a wave of their own.
//  - One workgroup covers a tile's whole K unless the launcher's layout splits it: a split across workgroups adds
//    device-scope round trips at the end of the dispatch (split_reduce: the partials' stores, the counter, the last
//    arriver's loads, two splits a trip), which only pays when the tiles alone
//    leave most compute units idle.
//  - A dispatch of few tiles (column_slices 4) runs four 16-column workgroups a tile instead, each wave four of the
//    layout's K slices in its 16-lane quarters (the MFMA's A broadcast to a quarter's four blocks, cbsz 2): each
//    lane computes what the 64-column lane of its column computes for its slice, so the results are the same bits.
// A row's result depends only on its own activations and the layout (split, GW), never on the other rows.
#include "device.hpp"
#include "kernels.hpp"
#include "split.hpp"

namespace sq::kern {
namespace {

constexpr int kPipe = 4;   // groups in flight per wave

// Row i's inputs 4b..4b+3 of the pair, as fp32, summed in a fixed order.
__device__ __forceinline__ float quad_sum(u32x2 v) {
  const float x0 = __uint_as_float(v[0] << 16), x1 = __uint_as_float(v[0] & 0xFFFF0000u);
  const float x2 = __uint_as_float(v[1] << 16), x3 = __uint_as_float(v[1] & 0xFFFF0000u);
  return (x0 + x1) + (x2 + x3);
}
// v combined with the lane that DPP control CTRL names (quad_perm [1,0,3,2]: lane ^ 1; [2,3,0,1]: lane ^ 2;
// row_half_mirror: lane 7 - i within eight lanes).
template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Wave `slice`'s K slice of plane tile `tile` of segment `seg` (K partition `split`), in format FMT, into acc; the
// slice's input sums go through its own xsum[slice] (NHS slots a group, at least the format's halves; narrow: each
// quarter's xsum[4 slice + q]).
// NARROW: the wave takes columns 16 cs..16 cs + 15 of the tile and four K slices, 4 slice + q for its quarter q (lanes
// 16q..16q + 15, lane 16q + c column 16 cs + c), every slice whole; each lane computes exactly what the wide walk's
// lane of that column computes for that slice (the same activations, operands, MFMA blocks, input-sum tree and
// closes, in the same order), so the two layouts give the same bits.
template <uint32_t FMT, int MR, int GW, int NT, int NHS, bool NARROW>
__device__ __forceinline__ void column_walk(const DecodeArgs &a, const Segment &seg, uint32_t tile, uint32_t split,
                                            uint32_t slice, uint32_t cs, float (&xsum)[kColumnMaxWaves][GW][NHS][4],
                                            float (&acc)[NT][MR]) {
  using F = Fmt<FMT>;
  // Groups in flight: 8-bit codes of a gate/up pair (four 16-byte loads a group) keep two, to fit the registers of
  // a full workgroup.
  constexpr int kDepth = F::P0 == 32 && NT == 2 ? 2 : kPipe;
  constexpr int SG = F::SG, UNIT = F::UNIT, P = GW < kDepth ? GW : kDepth;
  static_assert(GW % UNIT == 0 && GW % 2 == 0 && GW % SG == 0, "a slice holds whole meta units and group pairs");
  const int lane = threadIdx.x & 63, b = lane >> 2, i = lane & 3, c16 = lane & 15, xa = c16 >> 2;
  const uint32_t G = a.K >> 5, units = G / UNIT, gs = G / a.splits, slices = gs / GW;
  // The lane's column and slice; a narrow quarter past the split's slices streams its first slice again (nothing
  // reads its sums).
  const uint32_t col = NARROW ? 16 * cs + c16 : lane, mine = NARROW ? 4 * slice + (lane >> 4) : slice;
  const uint32_t gb = split * gs + (NARROW && mine >= slices ? 0 : mine) * GW;
  const uint32_t live = NARROW ? GW : min((uint32_t)GW, gs - min(gs, slice * GW));
  // The slice's last group: wave-uniform (the scalar offsets below clamp to it).
  const uint32_t last = __builtin_amdgcn_readfirstlane(live ? live - 1 : 0);

  // Buffer resources over the tile's planes (scalar registers) and a 32-bit offset a lane: the slice's start and
  // the lane's column. Group g's loads add g's offset as the scalar offset, so the walk's addresses cost no vector
  // instructions; a load past the tile's planes reads zero.
  __amdgpu_buffer_rsrc_t planes[NT], metas[NT], highs_at[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    const Segment &src = NT == 2 && n == 0 ? a.gate : seg;
    planes[n] = buffer_rsrc(src.plane0 + (size_t)tile * G * 64 * F::P0, G * 64 * F::P0);
    metas[n] = buffer_rsrc(src.meta + (size_t)tile * units * 64 * F::META, units * 64 * F::META);
    if constexpr (F::P1) highs_at[n] = buffer_rsrc(src.plane1 + (size_t)tile * G * 64 * F::P1, G * 64 * F::P1);
  }
  const uint32_t pv = (gb * 64 + col) * F::P0, hv = (gb * 64 + col) * F::P1;
  const uint32_t mv = (gb / UNIT * 64 + col) * F::META;
  // Wide: lane (b, i) reads row i's inputs 4 (b % 8)..+3 of the pair's group b / 8. Narrow: lane (q, a, i) =
  // 16q + 4a + i reads row i's inputs 8a..8a + 7 of each group of its quarter's slice, so block 4q + a holds the
  // group's input quads 2a (low half) and 2a + 1 (high half). Rows past the live ones read row 0, whose MFMA rows
  // nothing reads.
  const __amdgpu_buffer_rsrc_t inputs = buffer_rsrc(a.input, a.rows * a.K * 2);
  const uint32_t xv = (((i < MR && (uint32_t)i < a.rows ? i : 0) * a.K + (NARROW ? 8 * xa : 4 * (b & 7)) + gb * 32) +
                       (NARROW ? 0 : 32 * (b >> 3))) * 2;
  const CodeConstants cc = make_code_constants();

#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[n][r] = 0.0f;

  constexpr bool kWide = F::P0 == 32;   // 8-bit codes: two 16-byte loads and two operand sets a group
  u32x2 xp[NARROW ? 1 : GW / 2];
  u32x4 xn[NARROW ? GW : 1];
  u32x4 codes[NT][GW];
  u32x4 codes_hi[NT][kWide ? GW : 1];
  u32x2 highs[NT][F::P1 ? GW : 1];
  MetaWords mw[NT][GW / UNIT];
  // Groups past the slice repeat its last one (the clamp is wave-uniform, so scalar); a wide pair's high lanes read
  // the group after it, which nothing computes on past the slice.
  const auto issue = [&](int u) __attribute__((always_inline)) {
    const uint32_t g = min((uint32_t)u, last);
    if constexpr (NARROW) xn[u] = buffer_b128<0>(inputs, xv, (uint32_t)u * 64);
    else if (u % 2 == 0) xp[u / 2] = buffer_b64<0>(inputs, xv, g * 64);
    if (u % UNIT == 0) {
      const uint32_t v = min((uint32_t)(u / UNIT), last / UNIT);
#pragma unroll
      for (int n = 0; n < NT; ++n) mw[n][u / UNIT] = buffer_meta<FMT>(metas[n], mv, v * 64 * F::META);
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      codes[n][u] = buffer_b128(planes[n], pv, g * 64 * F::P0);
      if constexpr (kWide) codes_hi[n][u] = buffer_b128(planes[n], pv, g * 64 * F::P0 + 16);
      if constexpr (F::P1 == 4) highs[n][u][0] = buffer_b32(highs_at[n], hv, g * 64 * F::P1);
      if constexpr (F::P1 == 8) highs[n][u] = buffer_b64(highs_at[n], hv, g * 64 * F::P1);
    }
  };
  // The rows' input sums of the slice's groups (of each half for Q6_K): lanes 8j..8j+7 take one (row, group), each
  // lane four inputs, then a fixed tree over the eight lanes (quads first: the halves). Rows past the live ones and
  // groups past the slice's sum to zero, which no close reads. Their inputs are loaded before the stream's first
  // groups, so waiting for them waits for nothing else. A narrow wave sums its four slices' (item quarter q: slice
  // 4 slice + q; a slice past the split's sums nothing).
  constexpr int NH = F::HALVES ? 2 : 1, kItems = (NARROW ? 4 : 1) * MR * GW * 8, kIt = (kItems + 63) / 64;
  static_assert(NH <= NHS, "the kernel's input-sum slots hold the format's halves");
  static_assert(kIt <= 16, "the input sums' loads fit the registers of a full workgroup");
  const auto item_of = [&](int it, int &e, int &g, int &r, uint32_t &sl) __attribute__((always_inline)) {
    const int item = it * 64 + lane, rest = item >> 3;
    e = item & 7;
    g = rest % GW;
    r = (rest / GW) % MR;
    sl = NARROW ? 4 * slice + (uint32_t)(rest / (GW * MR)) : slice;
    return item < kItems;
  };
  u32x2 xq[kIt];
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    int e, g, r;
    uint32_t sl;
    const bool in = item_of(it, e, g, r, sl);
    const bool use = in && (uint32_t)r < a.rows && (uint32_t)g < live && (!NARROW || sl < slices);
    const size_t at = (size_t)r * a.K + (size_t)(split * gs + sl * GW + g) * 32 + 4 * e;
    xq[it] = use ? *(const u32x2 *)(a.input + at) : u32x2{0u, 0u};
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = 0; u < P; ++u) issue(u);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    int e, g, r;
    uint32_t sl;
    const bool in = item_of(it, e, g, r, sl);
    float v = quad_sum(xq[it]);
    v = dpp_add<0xB1>(v);
    v = dpp_add<0x4E>(v);
    if (F::HALVES && in && e % 4 == 0) xsum[sl][g][e / 4][r] = v;
    v = dpp_add<0x141>(v);
    if (!F::HALVES && in && e == 0) xsum[sl][g][0][r] = v;
  }
  // The wave reads back what its own lanes wrote.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 C0[NT], C1[NT], H0[NT], H1[NT];   // H: the high nibbles' chains of 8-bit codes
  // Input quad Q (inputs 4Q..4Q + 3) of group u against the lane's four operands: wide, block 8 (u % 2) + Q of the
  // pair's register broadcast to the wave; narrow, block Q / 2 of the quarter (half Q % 2 of its register) broadcast
  // to the quarter.
  const auto quad_mfma = [&](int u, int Q, u32x2 operands, f32x4 c) __attribute__((always_inline)) {
    if constexpr (NARROW)
      return mfma_bcast_quarter(Q >> 1, Q & 1 ? u32x2{xn[u][2], xn[u][3]} : u32x2{xn[u][0], xn[u][1]}, operands, c);
    else
      return mfma_bcast(8 * (u & 1) + Q, xp[u >> 1], operands, c);
  };
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    if (u + P < GW) issue(u + P);
    __builtin_amdgcn_sched_barrier(0);
    if ((uint32_t)u < live) {
      const bool first = u % SG == 0;
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          // Chunk d: plane word d (8-bit codes: words 2d and 2d + 1 of the 32-byte unit) and its plane1 bits.
          uint32_t w0 = codes[n][u][d], w1 = 0u, hb = 0u;
          if constexpr (kWide) {
            w0 = d < 2 ? codes[n][u][2 * d] : codes_hi[n][u][2 * d - 4];
            w1 = d < 2 ? codes[n][u][2 * d + 1] : codes_hi[n][u][2 * d - 3];
          }
          if constexpr (F::P1 == 4) hb = (highs[n][u][0] >> (8 * d)) & 0xFFu;
          if constexpr (F::P1 == 8) hb = (highs[n][u][d >> 1] >> (16 * (d & 1))) & 0xFFFFu;
          u32x4 lo, hi;
          chunk_operands<FMT>(w0, w1, hb, cc, lo, hi);
          C0[n] = quad_mfma(u, d, u32x2{lo[0], lo[1]}, first && d == 0 ? zero : C0[n]);
          C1[n] = quad_mfma(u, 4 + d, u32x2{lo[2], lo[3]}, first && d == 0 ? zero : C1[n]);
          if constexpr (kWide) {
            H0[n] = quad_mfma(u, d, u32x2{hi[0], hi[1]}, first && d == 0 ? zero : H0[n]);
            H1[n] = quad_mfma(u, 4 + d, u32x2{hi[2], hi[3]}, first && d == 0 ? zero : H1[n]);
          }
        }
      if ((u + 1) % SG == 0) {
        // The rows' input sums of the scale group (of the group's halves for Q6_K), in group order.
        float sx[MR], sh[2][MR];
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          if constexpr (F::HALVES) {
            sh[0][r] = xsum[mine][u][0][r];
            sh[1][r] = xsum[mine][u][NH - 1][r];
          } else {
            sx[r] = xsum[mine][u + 1 - SG][0][r];
#pragma unroll
            for (int k = 1; k < SG; ++k) sx[r] += xsum[mine][u + 1 - SG + k][0][r];
          }
        }
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          if constexpr (F::HALVES) {
            // Q6_K: value = s_h (q - 32) = s_h (128 + q) - 160 s_h, a scale per half.
            const float s0 = q6k_scale(mw[n][u / UNIT], u, 0), s1 = q6k_scale(mw[n][u / UNIT], u, 1);
#pragma unroll
            for (int r = 0; r < MR; ++r) {
              acc[n][r] = fmaf(s0, C0[n][r], acc[n][r]);
              acc[n][r] = fmaf(s1, C1[n][r], acc[n][r]);
              acc[n][r] = fmaf(-160.0f * s0, sh[0][r], acc[n][r]);
              acc[n][r] = fmaf(-160.0f * s1, sh[1][r], acc[n][r]);
            }
          } else {
            const Coef k = coef<FMT>(mw[n][u / UNIT], u);
            // 8-bit codes: sum x u = C_lo + 16 C_hi - 2176 sum x (Q8_0's value d (u - 128): z = -128 d).
            const float zc = kWide ? fmaf(-2176.0f, k.s, FMT == SQ_FMT_Q80 ? -128.0f * k.s : k.z)
                                   : fmaf(-128.0f, k.s, k.z);
#pragma unroll
            for (int r = 0; r < MR; ++r) {
              float c = C0[n][r] + C1[n][r];
              if constexpr (kWide) c = fmaf(16.0f, H0[n][r] + H1[n][r], c);
              acc[n][r] = fmaf(k.s, c, acc[n][r]);
              acc[n][r] = fmaf(zc, sx[r], acc[n][r]);
            }
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <uint32_t FMT>
constexpr int xsum_halves() {
  if constexpr (FMT == kSegmentFormats) return 2;
  else return Fmt<FMT>::HALVES ? 2 : 1;
}

// FMT kSegmentFormats: each workgroup runs its segment's format.
// NARROW: workgroup x takes columns 16 (x % 4)..+15 of tile x / 4 over the whole K (one split, whole slices), its
// waves four slices each; the slices then meet in LDS as the wide workgroup's do.
template <uint32_t FMT, int MR, int GW, int NT, uint32_t EP, bool F32OUT, bool NARROW>
__global__ __launch_bounds__(64 * kColumnMaxWaves) void column_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t slice = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), waves = blockDim.x >> 6;
  const uint32_t split = blockIdx.y, cs = NARROW ? blockIdx.x & 3 : 0;
  uint32_t tile = NARROW ? blockIdx.x >> 2 : blockIdx.x, s = 0;
  while (s + 1 < a.segments && tile >= a.seg[s].tiles) tile -= a.seg[s++].tiles;
  const Segment seg = a.seg[s];
  constexpr int NHS = xsum_halves<FMT>();
  __shared__ float xsum[kColumnMaxWaves][GW][NHS][4];
  float acc[NT][MR];
  if constexpr (FMT == kSegmentFormats)
    with_format(seg.fmt, [&](auto f) {
      column_walk<decltype(f)::value, MR, GW, NT, NHS, NARROW>(a, seg, tile, split, slice, cs, xsum, acc);
    });
  else
    column_walk<FMT, MR, GW, NT, NHS, NARROW>(a, seg, tile, split, slice, cs, xsum, acc);

  // Slices meet in LDS; row r's outputs (of both tensors) belong to wave r % waves, which adds them in slice order
  // and stores them (or stages them for the split reduce). Narrow: lane 16q + c holds slice 4 wave + q of column
  // 16 cs + c, and lanes 0..15 of the row's wave add the slices.
  __shared__ float red[kColumnMaxWaves][NT][MR][64];
  const uint32_t slices = NARROW ? (a.K >> 5) / a.splits / GW : waves, c = NARROW ? lane & 15 : lane;
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int r = 0; r < MR; ++r) red[NARROW ? 4 * slice + (lane >> 4) : slice][n][r][c] = acc[n][r];
  __syncthreads();
  const uint32_t col = seg.out_offset + tile * 64 + 16 * cs + c;
  const uint32_t cstride = NT == 2 ? 2 * a.out_stride : a.out_stride;
  float total[NT][MR];
  bool rlive[NT][MR];
  size_t index[NT][MR];
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      const bool mine = (uint32_t)r % waves == slice && (!NARROW || lane < 16);
      float v = 0.0f;
      if (mine) {
        // Every slot's read goes out at once (slots past the slices hold nothing the sum takes), then the adds run
        // in slice order.
        float part[kColumnMaxWaves];
#pragma unroll
        for (uint32_t w = 0; w < kColumnMaxWaves; ++w) part[w] = red[w][n][r][c];
#pragma unroll
        for (uint32_t w = 0; w < kColumnMaxWaves; ++w)
          if (w < slices) v += part[w];
      }
      total[n][r] = v;
      rlive[n][r] = mine && (uint32_t)r < a.rows;
      index[n][r] = (size_t)r * cstride + n * a.out_stride + col;
    }
  // Counters: one per workgroup column, a 16-column workgroup's among them (the plan holds one per 16 columns).
  if (a.splits > 1 && !split_reduce<NT, MR>(total, rlive, index, a.partials, (size_t)a.rows * cstride, split,
                                            a.splits, a.counters + blockIdx.x, true))
    return;
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    if (!rlive[0][r]) continue;
    const size_t o = (size_t)r * a.out_stride + col;
    if constexpr (NT == 2) {
      const float g = bf16_to_f32(f32_to_bf16(total[0][r])), up = bf16_to_f32(f32_to_bf16(total[1][r]));
      ((uint16_t *)a.output)[o] = f32_to_bf16(up * silu(g));
    } else {
      const float v = epilogue<EP>(total[0][r], a.aux, o);
      if constexpr (F32OUT) ((float *)a.output)[o] = v;
      else ((uint16_t *)a.output)[o] = f32_to_bf16(v);
    }
  }
}

// The narrow layout (16-column workgroups, each wave four K slices) runs when the caller asks for it
// (column_slices 4), the split's slices are whole, and the input sums of a wave's four slices fit its registers
// (rows x groups a slice at most 32); otherwise the wide one. Both give the same bits. Q6_K gate/up pairs keep the
// wide layout (their narrow walk of 16-group slices spills).
template <uint32_t FMT, int MR, int GW, int NT>
constexpr bool narrow_fits() {
  if constexpr (FMT != kSegmentFormats && NT == 2) {
    if (Fmt<FMT>::HALVES) return false;
  }
  return MR * GW <= 32;
}

template <uint32_t FMT, int MR, int GW, int NT, uint32_t EP, bool F32OUT>
void launch_gw(const DecodeArgs &a, uint32_t tiles, DecodeLayout layout, hipStream_t stream) {
  if constexpr (narrow_fits<FMT, MR, GW, NT>()) {
    if (a.column_slices == 4 && layout.nb * layout.ks == (a.K >> 5) / a.splits) {
      const dim3 grid(tiles * 4, a.splits), block(64 * ((layout.nb + 3) / 4));
      hipLaunchKernelGGL((column_kernel<FMT, MR, GW, NT, EP, F32OUT, true>), grid, block, 0, stream, a);
      return;
    }
  }
  hipLaunchKernelGGL((column_kernel<FMT, MR, GW, NT, EP, F32OUT, false>), dim3(tiles, a.splits),
                     dim3(64 * layout.nb), 0, stream, a);
}

template <uint32_t FMT, int MR, int NT, uint32_t EP, bool F32OUT>
hipError_t launch_mr(const DecodeArgs &a, uint32_t tiles, DecodeLayout layout, hipStream_t stream) {
  switch (layout.ks) {
    case 8: launch_gw<FMT, MR, 8, NT, EP, F32OUT>(a, tiles, layout, stream); break;
    case 16: launch_gw<FMT, MR, 16, NT, EP, F32OUT>(a, tiles, layout, stream); break;
    default:
      if constexpr (NT == 1) launch_gw<FMT, MR, 32, NT, EP, F32OUT>(a, tiles, layout, stream);
      break;
  }
  return hipGetLastError();
}

template <uint32_t FMT, int NT, uint32_t EP, bool F32OUT>
hipError_t launch_rows(const DecodeArgs &a, uint32_t tiles, DecodeLayout layout, hipStream_t stream) {
  // One, two or four rows' closes and input sums (a row computes the same in each instance).
  return a.rows <= 1   ? launch_mr<FMT, 1, NT, EP, F32OUT>(a, tiles, layout, stream)
         : a.rows == 2 ? launch_mr<FMT, 2, NT, EP, F32OUT>(a, tiles, layout, stream)
                       : launch_mr<FMT, 4, NT, EP, F32OUT>(a, tiles, layout, stream);
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

hipError_t launch_decode_column(uint32_t fmt, uint32_t epilogue, bool f32_output, const DecodeArgs &a,
                                hipStream_t stream) {
  uint32_t tiles = 0;
  for (uint32_t s = 0; s < a.segments; ++s) tiles += a.seg[s].tiles;
  const bool pair = a.gate.plane0 != nullptr;
  // nb: the workgroup's waves (K slices), ks: a slice's groups of 32 inputs.
  const DecodeLayout layout = decode_layout(layout_format(fmt, a), tiles * 4, a.K, a.splits, pair, a.rows);
  if (!a.rows || a.rows > kColumnTileRows || !layout.nb) return hipErrorInvalidValue;
  switch (fmt) {
    case SQ_FMT_AF4G32: return launch_format<SQ_FMT_AF4G32>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case SQ_FMT_AF4G64: return launch_format<SQ_FMT_AF4G64>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case SQ_FMT_AF4G128: return launch_format<SQ_FMT_AF4G128>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case SQ_FMT_Q4K: return launch_format<SQ_FMT_Q4K>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case SQ_FMT_Q5K: return launch_format<SQ_FMT_Q5K>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case SQ_FMT_Q6K: return launch_format<SQ_FMT_Q6K>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case SQ_FMT_Q80: return launch_format<SQ_FMT_Q80>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case SQ_FMT_AF8G64: return launch_format<SQ_FMT_AF8G64>(epilogue, f32_output, pair, a, tiles, layout, stream);
    case kSegmentFormats:
      if (epilogue != EpNone || f32_output || pair) return hipErrorInvalidValue;
      return launch_rows<kSegmentFormats, 1, EpNone, false>(a, tiles, layout, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sq::kern
