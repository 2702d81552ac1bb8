// The row tile's inner loop, shared by the decode row tile (decode.hip) and the MoE expert passes (moe.hip): one
// wave streams one K slice of a 64-column plane tile against 16 or 32 rows of bf16 activations with exact operands
// (reference: the exact-operand register tile, kernels/decode/linear_gguf_sgmatrix.metal:37-328), and the waves of
// a workgroup meet in LDS.
//
// CDNA4 mapping. Per group of 32 inputs one 16-byte load per lane (lane l: column l's 32 codes), 1 KiB per wave,
// kRowPipe groups in flight, every load unconditional. The rows go on the 16-row side of the 16x16x32 bf16 MFMA:
//  - a 4x4 transpose of the four code dwords across the wave's four 16-lane rows (v_permlane32_swap, then
//    v_permlane16_swap) gives lane (j, q) word q of column 16t + j in register t, the MFMA's B layout for column
//    block t; each word becomes eight exact bf16 operands 128 + q (code_pairs);
//  - per group and 16-row block, four MFMAs (one per 16-column block) plus one against bf16 ones, which leaves
//    each lane its own rows' input sums: no cross-lane reduction;
//  - each scale group closes in fp32: acc += s * sum x (128 + q) + (z - 128 s) * sum x, every product exact.
// A row's result depends only on its own activations and the layout, never on the other rows.
#pragma once
#include "device.hpp"

namespace sq::kern {

constexpr int kRowPipe = 4;   // groups in flight per wave

// Lane (j, q) register t <- lane (j + 16 t) register q: the 4x4 transpose of words across the 16-lane rows.
__device__ __forceinline__ void transpose4(uint32_t (&r)[4]) {
  const auto a = __builtin_amdgcn_permlane32_swap(r[0], r[2], false, false);
  const auto b = __builtin_amdgcn_permlane32_swap(r[1], r[3], false, false);
  const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
  r[0] = c[0];
  r[1] = c[1];
  r[2] = d[0];
  r[3] = d[1];
}

// Adds GW groups (the first `live` of them) of NT tensors' plane tiles to acc[n][t][b][i] (tensor n, column
// block t, row block b, row 4q + i of the block). plane[n] and meta[n] point at the slice's first group for
// the lane (plane: + 16 lane; meta: + META j); xrow[b] at the lane's row 16 b + j, inputs 4q of the slice's first
// group.
template <uint32_t FMT, int MB, int GW, int NT>
__device__ __forceinline__ void row_slice(const uint8_t *const (&plane)[NT], const uint8_t *const (&meta)[NT],
                                          const uint16_t *const (&xrow)[MB], uint32_t live,
                                          float (&acc)[NT][4][MB][4]) {
  using F = Fmt<FMT>;
  constexpr int SG = F::SG, UNIT = F::UNIT, P = GW < kRowPipe ? GW : kRowPipe;
  static_assert(GW % UNIT == 0 && GW % SG == 0, "a slice holds whole meta units");
  const uint32_t last = live ? live - 1 : 0;
  const CodeConstants cc = make_code_constants();

  u32x4 xv[MB][GW];
  u32x4 codes[NT][GW];
  MetaWords mw[NT][4][GW / UNIT];
  const auto issue = [&](int u) __attribute__((always_inline)) {
    const uint32_t g = min((uint32_t)u, last);
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const u32x2 lo = *(const u32x2 *)(xrow[b] + (size_t)g * 32), hi = *(const u32x2 *)(xrow[b] + (size_t)g * 32 + 16);
      xv[b][u] = u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
    if (u % UNIT == 0) {
      const uint32_t v = min((uint32_t)(u / UNIT), last / UNIT);
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          mw[n][t][u / UNIT] = load_meta<FMT>(meta[n] + ((size_t)v * 64 + 16 * t) * F::META);
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) codes[n][u] = __builtin_nontemporal_load((const u32x4 *)(plane[n] + (size_t)g * 1024));
  };
#pragma unroll
  for (int u = 0; u < P; ++u) issue(u);

  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 C[NT][4][MB], S[MB];
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    if (u + P < GW) issue(u + P);
    __builtin_amdgcn_sched_barrier(0);
    if ((uint32_t)u < live) {
      const bool first = u % SG == 0;
#pragma unroll
      for (int b = 0; b < MB; ++b) S[b] = mfma_bf16(xv[b][u], ones_operand(), first ? zero : S[b]);
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        uint32_t r[4] = {codes[n][u][0], codes[n][u][1], codes[n][u][2], codes[n][u][3]};
        transpose4(r);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4 w = code_pairs(r[t], cc);
#pragma unroll
          for (int b = 0; b < MB; ++b) C[n][t][b] = mfma_bf16(xv[b][u], w, first ? zero : C[n][t][b]);
        }
      }
      if ((u + 1) % SG == 0) {
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const Coef k = coef<FMT>(mw[n][t][u / UNIT], u);
            const float zc = fmaf(-128.0f, k.s, k.z);
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                acc[n][t][b][i] = fmaf(k.s, C[n][t][b][i], acc[n][t][b][i]);
                acc[n][t][b][i] = fmaf(zc, S[b][i], acc[n][t][b][i]);
              }
          }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Adds all G groups of NT tensors' plane tiles to acc, as row_slice does, in one continuous stream: chunks of four
// groups, each chunk's loads (clamped to the last group, so every chunk issues as many) issued SETS - 1 chunks
// ahead into a ring of SETS register sets. plane[n], meta[n] and xrow[b] point at group 0 for the lane.
template <uint32_t FMT, int MB, int NT, int SETS = 2>
__device__ __forceinline__ void row_stream(const uint8_t *const (&plane)[NT], const uint8_t *const (&meta)[NT],
                                           const uint16_t *const (&xrow)[MB], uint32_t G,
                                           float (&acc)[NT][4][MB][4]) {
  using F = Fmt<FMT>;
  constexpr int SG = F::SG, UNIT = F::UNIT, CH = 4, MU = UNIT < CH ? CH / UNIT : 1;
  static_assert(CH % SG == 0, "a chunk holds whole scale groups");
  const uint32_t last = G - 1, chunks = (G + CH - 1) / CH;
  const CodeConstants cc = make_code_constants();
  u32x4 xv[SETS][MB][CH], codes[SETS][NT][CH];
  MetaWords mw[SETS][NT][4][MU];
  const auto issue = [&](uint32_t c, int set) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const uint32_t g = min(c * CH + u, last);
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const u32x2 lo = *(const u32x2 *)(xrow[b] + (size_t)g * 32);
        const u32x2 hi = *(const u32x2 *)(xrow[b] + (size_t)g * 32 + 16);
        xv[set][b][u] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
#pragma unroll
      for (int n = 0; n < NT; ++n)
        codes[set][n][u] = __builtin_nontemporal_load((const u32x4 *)(plane[n] + (size_t)g * 1024));
    }
#pragma unroll
    for (int m = 0; m < MU; ++m) {
      const uint32_t unit = min((c * CH) / UNIT + m, last / UNIT);
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int t = 0; t < 4; ++t) mw[set][n][t][m] = load_meta<FMT>(meta[n] + ((size_t)unit * 64 + 16 * t) * F::META);
    }
  };
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 C[NT][4][MB], S[MB];
  // Each group's exact operands (transposed words as bf16 128 + q) are built one group ahead, into the other of
  // two operand sets, so that building them interleaves with the previous group's MFMAs.
  u32x4 wop[2][NT][4];
  const auto prepare = [&](int set, int u, int os) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      uint32_t r[4] = {codes[set][n][u][0], codes[set][n][u][1], codes[set][n][u][2], codes[set][n][u][3]};
      transpose4(r);
#pragma unroll
      for (int t = 0; t < 4; ++t) wop[os][n][t] = code_pairs(r[t], cc);
    }
  };
  const auto compute = [&](uint32_t c, int set, int next_set) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const uint32_t g = c * CH + u;
      const int os = u & 1;   // CH is even: group g's operands sit in set g % 2
      if (g < G) {
        const bool first = u % SG == 0;
#pragma unroll
        for (int b = 0; b < MB; ++b) S[b] = mfma_bf16(xv[set][b][u], ones_operand(), first ? zero : S[b]);
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int b = 0; b < MB; ++b) C[n][t][b] = mfma_bf16(xv[set][b][u], wop[os][n][t], first ? zero : C[n][t][b]);
        // The next group's operands (the last group of a chunk takes the next chunk's first).
        if (u + 1 < CH) prepare(set, u + 1, os ^ 1);
        else prepare(next_set, 0, os ^ 1);
        if ((u + 1) % SG == 0) {
#pragma unroll
          for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const Coef k = coef<FMT>(mw[set][n][t][UNIT < CH ? u / UNIT : 0], g);
              const float zc = fmaf(-128.0f, k.s, k.z);
#pragma unroll
              for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                  acc[n][t][b][i] = fmaf(k.s, C[n][t][b][i], acc[n][t][b][i]);
                  acc[n][t][b][i] = fmaf(zc, S[b][i], acc[n][t][b][i]);
                }
            }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
#pragma unroll
  for (int c = 0; c < SETS - 1; ++c) issue(c, c);
  prepare(0, 0, 0);
  for (uint32_t c = 0; c < chunks; c += SETS) {
#pragma unroll
    for (int k = 0; k < SETS; ++k) {
      issue(c + k + SETS - 1, (k + SETS - 1) % SETS);
      __builtin_amdgcn_sched_barrier(0);
      compute(c + k, k, (k + 1) % SETS);
    }
  }
}

template <int MB, int NT>
__device__ __forceinline__ void clear(float (&acc)[NT][4][MB][4]) {
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[n][t][b][i] = 0.0f;
}

// The workgroup's slices meet in LDS (red: waves x A x 64 floats, A = NT * 4 * MB * 4): accumulator e of every
// tensor is added, in slice order, by wave owner(e) = (e % (4 MB 4)) % waves, which gets total[e]; owned[e] says
// whether this wave holds it.
template <int MB, int NT>
__device__ __forceinline__ void row_reduce(const float (&acc)[NT][4][MB][4], float *red, uint32_t slice,
                                           uint32_t waves, int lane, float (&total)[NT * 4 * MB * 4],
                                           bool (&owned)[NT * 4 * MB * 4]) {
  constexpr int A = NT * 4 * MB * 4;
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((slice * A) + ((n * 4 + t) * MB + b) * 4 + i) * 64 + lane] = acc[n][t][b][i];
  __syncthreads();
#pragma unroll
  for (int e = 0; e < A; ++e) {
    const uint32_t own = (uint32_t)(e % (4 * MB * 4)) % waves;
    float v = 0.0f;
    if (own == slice)
      for (uint32_t w = 0; w < waves; ++w) v += red[(w * A + e) * 64 + lane];
    total[e] = v;
    owned[e] = own == slice;
  }
}

}  // namespace sq::kern
