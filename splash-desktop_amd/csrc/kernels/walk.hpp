// The per-wave K walk shared by the decode tile and the MoE expert passes: one wave accumulates a 64-column plane
// tile (four 16-column MFMA blocks) of NT weight tensors against up to MB 16-row blocks of bf16 activations, over
// scale groups [sg_begin, sg_end) of K.
//
// Per group of 32 inputs a wave reads the tile's 1 KiB of codes as four 256-byte rows of lanes (lane (j, q) takes
// word q of column 16t + j), turns each word into eight exact bf16 operands 128 + q (code_operands), and runs one
// 16x16x32 bf16 MFMA per 16 columns with the activation rows as A; one more MFMA against bf16 ones gives the rows'
// input sums. Each scale group then closes in fp32,
//   acc += s * sum x (128 + q) + (z - 128 s) * sum x,
// which is sum x (s q + z) with every product exact (the reference's exact-operand register tile does the same with
// its 8x8 matrices: kernels/decode/linear_gguf_sgmatrix.metal). The next scale group's loads are in flight while
// the current one computes.
#pragma once
#include "device.hpp"

namespace sq::kern {

// A lane's activation row for row block b: nullptr for rows past the live ones (zeros).
struct RowPtrs {
  const uint16_t *row[2];
};

template <uint32_t FMT, int MB, int NT> struct WalkStage {
  uint32_t codes[NT][Fmt<FMT>::SG][4];
  u32x4 x[Fmt<FMT>::SG][MB];
  MetaWords meta[NT][4];
};

// plane[n]: the tile's plane0 base advanced to the lane's (j, q) word (tile base + 16 j + 4 q); meta[n]: the tile's
// meta base advanced to column j (tile base + META j). R: accumulator rows kept per lane group (4, or the live rows
// when fewer than 4 exist in all).
template <uint32_t FMT, int MB, int R, int NT>
__device__ __forceinline__ void walk(const uint8_t *const (&plane)[NT], const uint8_t *const (&meta)[NT],
                                     const RowPtrs &x, uint32_t sg_begin, uint32_t sg_end, int q,
                                     f32x4 (&acc)[NT][4][MB]) {
  using F = Fmt<FMT>;
  const auto load = [&](WalkStage<FMT, MB, NT> &st, uint32_t sg) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < F::SG; ++u) {
      const uint32_t g = sg * F::SG + u;
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int t = 0; t < 4; ++t)
          st.codes[n][u][t] = __builtin_nontemporal_load((const uint32_t *)(plane[n] + (size_t)g * 1024 + t * 256));
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        if (x.row[b]) {
          const uint16_t *xr = x.row[b] + g * 32 + 4 * q;
          const u32x2 lo = *(const u32x2 *)xr, hi = *(const u32x2 *)(xr + 16);
          st.x[u][b] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        } else {
          st.x[u][b] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
    const uint32_t unit = sg * F::SG / F::UNIT;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int t = 0; t < 4; ++t) st.meta[n][t] = load_meta<FMT>(meta[n] + ((size_t)unit * 64 + 16 * t) * F::META);
  };

  const auto compute = [&](const WalkStage<FMT, MB, NT> &st, uint32_t sg) __attribute__((always_inline)) {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 sx[MB];
#pragma unroll
    for (int u = 0; u < F::SG; ++u)
#pragma unroll
      for (int b = 0; b < MB; ++b) sx[b] = mfma_bf16(st.x[u][b], ones_operand(), u ? sx[b] : zero);
#pragma unroll
    for (int n = 0; n < NT; ++n) {
      f32x4 c[4][MB];
#pragma unroll
      for (int u = 0; u < F::SG; ++u)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4 w = code_operands(st.codes[n][u][t]);
#pragma unroll
          for (int b = 0; b < MB; ++b) c[t][b] = mfma_bf16(st.x[u][b], w, u ? c[t][b] : zero);
        }
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const Coef k = coef<FMT>(st.meta[n][t], sg);
        const float zc = fmaf(-128.0f, k.s, k.z);
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
          for (int i = 0; i < R; ++i) {
            acc[n][t][b][i] = fmaf(k.s, c[t][b][i], acc[n][t][b][i]);
            acc[n][t][b][i] = fmaf(zc, sx[b][i], acc[n][t][b][i]);
          }
      }
    }
  };

  WalkStage<FMT, MB, NT> st0, st1;
  uint32_t sg = sg_begin;
  if (sg < sg_end) load(st0, sg);
  for (; sg + 1 < sg_end; sg += 2) {
    load(st1, sg + 1);
    compute(st0, sg);
    if (sg + 2 < sg_end) load(st0, sg + 2);
    compute(st1, sg + 1);
  }
  if (sg < sg_end) compute(st0, sg);
}

// The four waves' accumulators added in wave order; wave w returns the 16 columns of block t = w.
template <int MB, int R, int NT>
__device__ __forceinline__ void reduce_waves(const f32x4 (&acc)[NT][4][MB], float *lds, int wave, int lane,
                                             float (&total)[NT][MB][R]) {
  // lds: [4 waves][NT][4 t][MB][R][64] floats
  const auto at = [&](int w, int n, int t, int b, int i) { return ((((w * NT + n) * 4 + t) * MB + b) * R + i) * 64 + lane; };
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < R; ++i) lds[at(wave, n, t, b, i)] = acc[n][t][b][i];
  __syncthreads();
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) v += lds[at(w, n, wave, b, i)];
        total[n][b][i] = v;
      }
}

}  // namespace sq::kern
