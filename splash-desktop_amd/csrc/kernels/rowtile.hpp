// The row tile's inner loop, shared by the decode row tile (decode.hip) and the MoE expert passes (moe.hip): one
// wave streams one K slice of a 64-column plane tile against 16 or 32 rows of bf16 activations with exact operands
// (reference: the exact-operand register tile, kernels/decode/linear_gguf_sgmatrix.metal:37-328).
//
// CDNA4 mapping. Per group of 32 inputs one 16-byte load per lane (lane l: column l's 32 codes; 8-bit codes two,
// and Q5_K and Q6_K a plane1 word beside), 1 KiB per wave, kRowPipe groups in flight, every load unconditional. The
// rows go on the 16-row side of the 16x16x32 bf16 MFMA (the other formats' operands: row_operands):
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

// One group of 32 inputs of the lane's column: plane0 (16 bytes; 8-bit codes 32, `lo` then `hi`) and plane1 (Q5_K 4
// bytes, Q6_K 8). Members a format does not have are never read.
template <uint32_t FMT>
struct RowGroup {
  u32x4 lo, hi;
  u32x2 high;
};
// plane and high point at group 0 of the lane's column (plane + P0 lane, high + P1 lane).
template <uint32_t FMT>
__device__ __forceinline__ RowGroup<FMT> load_row_group(const uint8_t *plane, const uint8_t *high, uint32_t g) {
  using F = Fmt<FMT>;
  RowGroup<FMT> r;
  const uint8_t *p = plane + (size_t)g * 64 * F::P0;
  r.lo = __builtin_nontemporal_load((const u32x4 *)p);
  if constexpr (F::P0 == 32) r.hi = __builtin_nontemporal_load((const u32x4 *)(p + 16));
  if constexpr (F::P1 == 4) r.high[0] = __builtin_nontemporal_load((const uint32_t *)(high + (size_t)g * 64 * 4));
  if constexpr (F::P1 == 8) r.high = __builtin_nontemporal_load((const u32x2 *)(high + (size_t)g * 64 * 8));
  return r;
}

// One column block (16-column workgroups): lane (j, q) loads chunk q of its own column's group directly, the words
// the transpose would bring it: plane word q (8-bit codes: words 2q, 2q + 1, into lo[0..1]), and the plane1 word
// that holds chunk q's bits (Q5_K the column's word, Q6_K its word q / 2) into high[0]. plane points at chunk q of
// group 0 of the column (plane + P0 column + (P0 / 4) q), high at the word (high + P1 column (+ 4 (q / 2) for Q6_K)).
template <uint32_t FMT>
__device__ __forceinline__ RowGroup<FMT> load_row_chunk(const uint8_t *plane, const uint8_t *high, uint32_t g) {
  using F = Fmt<FMT>;
  RowGroup<FMT> r;
  const uint8_t *p = plane + (size_t)g * 64 * F::P0;
  if constexpr (F::P0 == 32) {
    const u32x2 w = __builtin_nontemporal_load((const u32x2 *)p);
    r.lo[0] = w[0];
    r.lo[1] = w[1];
  } else {
    r.lo[0] = __builtin_nontemporal_load((const uint32_t *)p);
  }
  if constexpr (F::P1) r.high[0] = __builtin_nontemporal_load((const uint32_t *)(high + (size_t)g * 64 * F::P1));
  return r;
}

// The decode walk's sources as buffer resources (scalar registers) over the tile's planes and the input rows, with
// a 32-bit offset a lane; group g's and unit v's offsets are scalar, so the walk's addresses cost no vector
// instructions (a load past a resource's range reads zero). pv, hv and mv: the lane's offsets at the slice's first
// group and unit, as load_row_group (TB 4) or load_row_chunk (TB 1) and load_meta expect their pointers; xv[b]: row
// block b's lane offset at inputs 8 q of the slice's first group.
template <uint32_t FMT, int NT, int MB, int TB>
struct RowBuffers {
  __amdgpu_buffer_rsrc_t plane[NT], high[NT], meta[NT], input;
  uint32_t pv, hv, mv, xv[MB];
  __device__ __forceinline__ u32x4 x(int b, uint32_t g) const { return buffer_b128<0>(input, xv[b], g * 64); }
  __device__ __forceinline__ MetaWords unit(int n, uint32_t v) const {
    return buffer_meta<FMT>(meta[n], mv, v * 64 * Fmt<FMT>::META);
  }
  __device__ __forceinline__ RowGroup<FMT> codes(int n, uint32_t g) const {
    using F = Fmt<FMT>;
    RowGroup<FMT> r;
    const uint32_t at = g * 64 * F::P0;
    if constexpr (TB == 1) {
      if constexpr (F::P0 == 32) {
        const u32x2 w = buffer_b64(plane[n], pv, at);
        r.lo[0] = w[0];
        r.lo[1] = w[1];
      } else {
        r.lo[0] = buffer_b32(plane[n], pv, at);
      }
      if constexpr (F::P1) r.high[0] = buffer_b32(high[n], hv, g * 64 * F::P1);
    } else {
      r.lo = buffer_b128(plane[n], pv, at);
      if constexpr (F::P0 == 32) r.hi = buffer_b128(plane[n], pv, at + 16);
      if constexpr (F::P1 == 4) r.high[0] = buffer_b32(high[n], hv, g * 64 * 4);
      if constexpr (F::P1 == 8) r.high = buffer_b64(high[n], hv, g * 64 * 8);
    }
    return r;
  }
};

// The lane's shift of its chunk's plane1 bits after the transpose (lane (j, q) holds chunk q): Q5_K byte q, Q6_K
// halfword q % 2 of the word the transpose brings.
template <uint32_t FMT>
__device__ __forceinline__ uint32_t row_high_shift(int lane) {
  const uint32_t q = (uint32_t)lane >> 4;
  return Fmt<FMT>::P1 == 4 ? 8 * q : Fmt<FMT>::P1 == 8 ? 16 * (q & 1) : 0;
}

// The exact bf16 B operands of a group: lane (j, q) gets chunk q of column 16 t + j in lo[t] (chunk_operands); 8-bit
// codes also get hi[t], the high nibbles as 16 (128 + q_hi), so that both add into one accumulator.
//  - 4-bit codes: one 4x4 transpose of the four plane words;
//  - 8-bit codes: chunk q is words 2q and 2q + 1 of the 32 bytes, one transpose of the even words and one of the odd;
//  - plane1 bits follow the plane words: Q5_K's word transposed (lane (j, q) gets column 16 t + j's word in every
//    register t, then byte q), Q6_K's two words as (w0, w0, w1, w1) (the word that holds halfword q).
template <uint32_t FMT>
__device__ __forceinline__ void row_operands(const RowGroup<FMT> &grp, uint32_t hshift, CodeConstants cc,
                                             u32x4 (&lo)[4], u32x4 (&hi)[4]) {
  using F = Fmt<FMT>;
  if constexpr (F::P0 == 32) {
    uint32_t e[4] = {grp.lo[0], grp.lo[2], grp.hi[0], grp.hi[2]}, o[4] = {grp.lo[1], grp.lo[3], grp.hi[1], grp.hi[3]};
    transpose4(e);
    transpose4(o);
#pragma unroll
    for (int t = 0; t < 4; ++t) chunk_operands<FMT, true>(e[t], o[t], 0u, cc, lo[t], hi[t]);
  } else {
    uint32_t r[4] = {grp.lo[0], grp.lo[1], grp.lo[2], grp.lo[3]};
    transpose4(r);
    uint32_t h[4] = {0u, 0u, 0u, 0u};
    if constexpr (F::P1 == 4) {
      h[0] = h[1] = h[2] = h[3] = grp.high[0];
      transpose4(h);
    } else if constexpr (F::P1 == 8) {
      h[0] = h[1] = grp.high[0];
      h[2] = h[3] = grp.high[1];
      transpose4(h);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) chunk_operands<FMT>(r[t], 0u, h[t] >> hshift, cc, lo[t], hi[t]);
  }
}

// The exact operands of one column block from load_row_chunk's words: what row_operands leaves in lo[t], hi[t] for
// the block's column.
template <uint32_t FMT>
__device__ __forceinline__ void row_operands_one(const RowGroup<FMT> &grp, uint32_t hshift, CodeConstants cc,
                                                 u32x4 (&lo)[1], u32x4 (&hi)[1]) {
  using F = Fmt<FMT>;
  if constexpr (F::P0 == 32) chunk_operands<FMT, true>(grp.lo[0], grp.lo[1], 0u, cc, lo[0], hi[0]);
  else chunk_operands<FMT>(grp.lo[0], 0u, F::P1 ? grp.high[0] >> hshift : 0u, cc, lo[0], hi[0]);
}

// One group's MFMAs. C[n][t][b] takes sum x (operand) over the group (Q6_K: over its first half, C2 the second) and
// S[b] the rows' input sums the same way, from zero when `first`. Q6_K's halves (one scale per 16 elements) run on
// the 16x16x16 MFMA: operand words 0..1 of every lane are a chunk's first-half elements, words 2..3 its second.
// `ones` is ones_operand(): the decode slices keep it in registers, the MoE streams rebuild it (their registers are
// spent).
template <uint32_t FMT, int MB, int NT, int TB = 4>
__device__ __forceinline__ void row_group_mfma(const u32x4 (&x)[MB], const u32x4 (&lo)[NT][TB],
                                               const u32x4 (&hi)[NT][TB], bool first, f32x4 (&C)[NT][TB][MB],
                                               f32x4 (&C2)[NT][TB][MB], f32x4 (&S)[MB], f32x4 (&S2)[MB],
                                               const u32x4 ones = ones_operand()) {
  using F = Fmt<FMT>;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  if constexpr (F::HALVES) {
    const u32x2 one = {0x3F803F80u, 0x3F803F80u};
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      S[b] = mfma_bf16_k16(u32x2{x[b][0], x[b][1]}, one, first ? zero : S[b]);
      S2[b] = mfma_bf16_k16(u32x2{x[b][2], x[b][3]}, one, first ? zero : S2[b]);
    }
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          C[n][t][b] = mfma_bf16_k16(u32x2{x[b][0], x[b][1]}, u32x2{lo[n][t][0], lo[n][t][1]}, first ? zero : C[n][t][b]);
          C2[n][t][b] = mfma_bf16_k16(u32x2{x[b][2], x[b][3]}, u32x2{lo[n][t][2], lo[n][t][3]}, first ? zero : C2[n][t][b]);
        }
  } else {
#pragma unroll
    for (int b = 0; b < MB; ++b) S[b] = mfma_bf16(x[b], ones, first ? zero : S[b]);
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int t = 0; t < TB; ++t)
#pragma unroll
        for (int b = 0; b < MB; ++b) C[n][t][b] = mfma_bf16(x[b], lo[n][t], first ? zero : C[n][t][b]);
    if constexpr (F::P0 == 32) {
#pragma unroll
      for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int t = 0; t < TB; ++t)
#pragma unroll
          for (int b = 0; b < MB; ++b) C[n][t][b] = mfma_bf16(x[b], hi[n][t], C[n][t][b]);
    }
  }
}

// A scale group's close in fp32, every product exact: acc += s C + zc S with zc = z - 128 s (4-bit and 5-bit codes
// 128 + q), z - 2176 s (8-bit codes, C = sum x u + 2176 sum x; Q8_0's value d (u - 128): z = -128 d), and Q6_K's
// s_h (q - 32) = s_h (128 + q) - 160 s_h per half. A lane holds four columns (16 t + j), so each lane derives the
// coefficients once, for its own column l (a Q4_K or Q5_K group's from its 16-byte header costs ~9 VALU, Q6_K's half
// scales ~14), and hands them to the lanes whose MFMA blocks hold the column: two ds_bpermute a column block, through
// the LDS crossbar (no LDS memory, not the VALU). `g` is the group's index in its meta unit's numbering (its
// super-block position).
// A column's close coefficients for one group: (s, zc = z - 128 s), or Q6_K's half scales (s0, s1).
struct CloseCoef {
  float a, b;
};
// TB 1 (16-column workgroups): each lane's meta is its own block column's, so its coefficients are its own.
template <uint32_t FMT, int NT, int TB = 4>
__device__ __forceinline__ void spread_coefs(const MetaWords (&own)[NT], uint32_t g, int j, CloseCoef (&k)[NT][TB]) {
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    CloseCoef mine;
    if constexpr (Fmt<FMT>::HALVES) {
      mine = {q6k_scale(own[n], g, 0), q6k_scale(own[n], g, 1)};
    } else {
      const Coef c = coef<FMT>(own[n], g);
      // row_group_close's zc: 8-bit codes' z - 2176 s (Q8_0: -128 d - 2176 d), else z - 128 s.
      const float zc = Fmt<FMT>::P0 == 32 ? fmaf(-2176.0f, c.s, FMT == SQ_FMT_Q80 ? -128.0f * c.s : c.z)
                                          : fmaf(-128.0f, c.s, c.z);
      mine = {c.s, zc};
    }
    if constexpr (TB == 1) {
      k[n][0] = mine;
    } else {
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        const int from = (16 * t + j) * 4;
        k[n][t].a = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(mine.a)));
        k[n][t].b = __int_as_float(__builtin_amdgcn_ds_bpermute(from, __float_as_int(mine.b)));
      }
    }
  }
}
// The close from the handed coefficients: acc += s C + zc S, or Q6_K's s0 C + s1 C2 - 160 s0 S - 160 s1 S2.
template <uint32_t FMT, int MB, int NT, int TB = 4>
__device__ __forceinline__ void row_group_close(const CloseCoef (&k)[NT][TB], const f32x4 (&C)[NT][TB][MB],
                                                const f32x4 (&C2)[NT][TB][MB], const f32x4 (&S)[MB],
                                                const f32x4 (&S2)[MB], float (&acc)[NT][TB][MB][4]) {
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const float s0 = k[n][t].a, s1 = k[n][t].b;
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (Fmt<FMT>::HALVES) {
            acc[n][t][b][i] = fmaf(s0, C[n][t][b][i], acc[n][t][b][i]);
            acc[n][t][b][i] = fmaf(s1, C2[n][t][b][i], acc[n][t][b][i]);
            acc[n][t][b][i] = fmaf(-160.0f * s0, S[b][i], acc[n][t][b][i]);
            acc[n][t][b][i] = fmaf(-160.0f * s1, S2[b][i], acc[n][t][b][i]);
          } else {
            acc[n][t][b][i] = fmaf(s0, C[n][t][b][i], acc[n][t][b][i]);
            acc[n][t][b][i] = fmaf(s1, S[b][i], acc[n][t][b][i]);
          }
        }
    }
}

// Adds GW groups (the first `live` of them) of NT tensors' plane tiles to acc[n][t][b][i] (tensor n, column
// block t, row block b, row 4q + i of the block), loading through src (RowBuffers): the slice's groups for the lane's
// column (load_row_group's words), the meta units of the lane's own column l (one load per unit and tensor, whose
// coefficients spread_coefs hands to the lanes whose MFMA blocks hold the column), and for each row block the lane's
// row 16 b + j, inputs 8q of each group (one 16-byte load a row block and group: the wave's LDS slot xlds, MB KiB,
// turns the lanes' contiguous chunks into the MFMA's A layout, inputs 4q..4q+3 and 16+4q..19+4q of the row, with a
// write and two reads instead of a second global load). TB 1: one column block, the lane's column j of it, its chunk
// q and meta loaded directly (load_row_chunk's words); the same operands, MFMAs and closes as that block's in the
// four-block walk.
template <uint32_t FMT, int MB, int GW, int NT, int TB = 4>
__device__ __forceinline__ void row_slice(const RowBuffers<FMT, NT, MB, TB> &src, uint8_t *xlds, uint32_t live,
                                          float (&acc)[NT][TB][MB][4]) {
  using F = Fmt<FMT>;
  // 8-bit codes (twice the bytes a group) keep fewer groups in flight, and so do the K-quants with plane1 bits in the
  // longest slices of one tensor's 16 rows (whose workgroups hold the most waves, 128 registers each), Q6_K (two
  // scales a group) in every slice of 16 rows, and the 64-column workgroups of 32 rows (measured, graph-replayed, M =
  // 32, four groups against two: K 4096 x N 14336 / 4096 and K 14336 x N 4096 and K 5120 x N 27648 15.85 / 10.90 /
  // 18.22 / 39.70 -> 15.18 / 10.54 / 17.12 / 38.38 us; the 16-row and 16-column workgroups measured within noise).
  constexpr bool kTight = F::P1 && MB == 1 && ((NT == 1 && GW == 32) || F::HALVES);
  constexpr int kDepth = F::P0 == 32 || kTight || (TB == 4 && MB == 2) ? kRowPipe / 2 : kRowPipe;
  constexpr int SG = F::SG, UNIT = F::UNIT, P = GW < kDepth ? GW : kDepth;
  static_assert(GW % UNIT == 0 && GW % SG == 0, "a slice holds whole meta units");
  // The slice's last group, wave-uniform: groups past it repeat it, with scalar offsets.
  const uint32_t last = __builtin_amdgcn_readfirstlane(live ? live - 1 : 0);
  const CodeConstants cc = make_code_constants();
  const uint32_t hshift = row_high_shift<FMT>(threadIdx.x & 63);

  u32x4 xv[MB][GW];
  RowGroup<FMT> codes[NT][GW];
  MetaWords own[NT][GW / UNIT];
  const auto issue = [&](int u) __attribute__((always_inline)) {
    const uint32_t g = min((uint32_t)u, last);
#pragma unroll
    for (int b = 0; b < MB; ++b) xv[b][u] = src.x(b, g);
    if (u % UNIT == 0) {
      const uint32_t v = min((uint32_t)(u / UNIT), last / UNIT);
#pragma unroll
      for (int n = 0; n < NT; ++n) own[n][u / UNIT] = src.unit(n, v);
    }
#pragma unroll
    for (int n = 0; n < NT; ++n) codes[n][u] = src.codes(n, g);
  };
#pragma unroll
  for (int u = 0; u < P; ++u) issue(u);

  f32x4 C[NT][TB][MB], C2[NT][TB][MB], S[MB], S2[MB];
  const int j = threadIdx.x & 15, lane = threadIdx.x & 63, q = lane >> 4;
  // Lane (j, q) reads inputs 4q..4q+3 (chunk q / 2 of its row, half q % 2) and 16+4q..19+4q (chunk 2 + q / 2).
  const uint32_t from_lo = ((q >> 1) * 16 + j) * 16 + (q & 1) * 8, from_hi = ((2 + (q >> 1)) * 16 + j) * 16 + (q & 1) * 8;
  // The input sums' bf16 ones, built once and held (the compiler otherwise rebuilds them every group).
  u32x4 ones = ones_operand();
  asm volatile("" : "+v"(ones));
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    if (u + P < GW) issue(u + P);
    __builtin_amdgcn_sched_barrier(0);
    if ((uint32_t)u < live) {
      u32x4 x[MB], lo[NT][TB], hi[NT][TB];
#pragma unroll
      for (int b = 0; b < MB; ++b) *(u32x4 *)(xlds + b * 1024 + lane * 16) = xv[b][u];
      // The wave reads back what its own lanes wrote, and writes the next group's only after reading this one's.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        const u32x2 l = *(const u32x2 *)(xlds + b * 1024 + from_lo), h = *(const u32x2 *)(xlds + b * 1024 + from_hi);
        x[b] = u32x4{l[0], l[1], h[0], h[1]};
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        if constexpr (TB == 1) row_operands_one<FMT>(codes[n][u], hshift, cc, lo[n], hi[n]);
        else row_operands<FMT>(codes[n][u], hshift, cc, lo[n], hi[n]);
      }
      row_group_mfma<FMT, MB, NT, TB>(x, lo, hi, u % SG == 0, C, C2, S, S2, ones);
      if ((u + 1) % SG == 0) {
        MetaWords unit[NT];
#pragma unroll
        for (int n = 0; n < NT; ++n) unit[n] = own[n][u / UNIT];
        CloseCoef k[NT][TB];
        spread_coefs<FMT, NT, TB>(unit, u, j, k);
        row_group_close<FMT, MB, NT, TB>(k, C, C2, S, S2, acc);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Adds all G groups of NT tensors' plane tiles to acc, as row_slice does, in one continuous stream: chunks of CH
// groups, each chunk's loads (clamped to the last group, so every chunk issues as many) issued SETS - 1 chunks
// ahead into a ring of SETS register sets; AHEAD builds each group's operands a group ahead (else just before its
// MFMAs). plane[n] and high[n] point at group 0 for the lane, meta[n] at unit 0 of the lane's own column l (one
// load per unit and tensor, spread_coefs hands each lane the columns its MFMA blocks hold). The input rows come in the
// tile's read order
// (16-byte chunk 4 g + c of a row: inputs 32 g + 4 c .. +3 then 32 g + 16 + 4 c .. +3), so each group of a row block
// is one 16-byte load a lane, half the vector memory instructions of two 8-byte loads from a row in input order:
// xrow[b] points at chunk q of group 0 of the lane's row 16 b + j.
template <uint32_t FMT, int MB, int NT, int SETS = 2, int CH = 4, bool AHEAD = true>
__device__ __forceinline__ void row_stream(const uint8_t *const (&plane)[NT], const uint8_t *const (&high)[NT],
                                           const uint8_t *const (&meta)[NT], const uint16_t *const (&xrow)[MB],
                                           uint32_t G, float (&acc)[NT][4][MB][4]) {
  using F = Fmt<FMT>;
  constexpr int SG = F::SG, UNIT = F::UNIT, MU = UNIT < CH ? CH / UNIT : 1;
  static_assert(CH % SG == 0, "a chunk holds whole scale groups");
  const uint32_t last = G - 1, chunks = (G + CH - 1) / CH;
  const CodeConstants cc = make_code_constants();
  const uint32_t hshift = row_high_shift<FMT>(threadIdx.x & 63);
  u32x4 xv[SETS][MB][CH];
  RowGroup<FMT> codes[SETS][NT][CH];
  MetaWords own[SETS][NT][MU];
  const auto issue = [&](uint32_t c, int set) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const uint32_t g = min(c * CH + u, last);
#pragma unroll
      for (int b = 0; b < MB; ++b) xv[set][b][u] = *(const u32x4 *)(xrow[b] + (size_t)g * 32);
#pragma unroll
      for (int n = 0; n < NT; ++n) codes[set][n][u] = load_row_group<FMT>(plane[n], high[n], g);
    }
#pragma unroll
    for (int m = 0; m < MU; ++m) {
      const uint32_t unit = min((c * CH) / UNIT + m, last / UNIT);
#pragma unroll
      for (int n = 0; n < NT; ++n) own[set][n][m] = load_meta<FMT>(meta[n] + (size_t)unit * 64 * F::META);
    }
  };
  f32x4 C[NT][4][MB], C2[NT][4][MB], S[MB], S2[MB];
  // Each group's exact operands are built one group ahead, into the other of two operand sets, so that building
  // them interleaves with the previous group's MFMAs; 8-bit codes (two operand sets a group), and callers that ask
  // for it to fit the registers, build them just before their MFMAs.
  constexpr bool kAhead = F::P0 != 32 && AHEAD;
  u32x4 lo[2][NT][4], hi[2][NT][4];
  const auto prepare = [&](int set, int u, int os) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < NT; ++n) row_operands<FMT>(codes[set][n][u], hshift, cc, lo[os][n], hi[os][n]);
  };
  const int j = threadIdx.x & 15;
  const auto compute = [&](uint32_t c, int set, int next_set) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const uint32_t g = c * CH + u;
      const int os = kAhead ? u & 1 : 0;   // CH is even: group g's operands sit in set g % 2
      if (g < G) {
        u32x4 x[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) x[b] = xv[set][b][u];
        if constexpr (!kAhead) prepare(set, u, 0);
        row_group_mfma<FMT, MB, NT>(x, lo[os], hi[os], u % SG == 0, C, C2, S, S2);
        // The next group's operands (the last group of a chunk takes the next chunk's first).
        if constexpr (kAhead) {
          if (u + 1 < CH) prepare(set, u + 1, os ^ 1);
          else prepare(next_set, 0, os ^ 1);
        }
        if ((u + 1) % SG == 0) {
          MetaWords unit[NT];
#pragma unroll
          for (int n = 0; n < NT; ++n) unit[n] = own[set][n][UNIT < CH ? u / UNIT : 0];
          CloseCoef k[NT][4];
          spread_coefs<FMT, NT>(unit, g, j, k);
          row_group_close<FMT, MB, NT>(k, C, C2, S, S2, acc);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
#pragma unroll
  for (int c = 0; c < SETS - 1; ++c) issue(c, c);
  if constexpr (kAhead) prepare(0, 0, 0);
  for (uint32_t c = 0; c < chunks; c += SETS) {
#pragma unroll
    for (int k = 0; k < SETS; ++k) {
      issue(c + k + SETS - 1, (k + SETS - 1) % SETS);
      __builtin_amdgcn_sched_barrier(0);
      compute(c + k, k, (k + 1) % SETS);
    }
  }
}

template <int MB, int NT, int TB>
__device__ __forceinline__ void clear(float (&acc)[NT][TB][MB][4]) {
#pragma unroll
  for (int n = 0; n < NT; ++n)
#pragma unroll
    for (int t = 0; t < TB; ++t)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[n][t][b][i] = 0.0f;
}

}  // namespace sq::kern
