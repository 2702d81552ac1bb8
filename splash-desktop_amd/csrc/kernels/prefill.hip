// The prefill tile: y[r][c] = sum_k x[r][k] w[c][k] for chunks of more than 32 rows (reference: gguf_prefill_tile
// and the gguf_prefill_<fmt>_{a,r,g} kernels, kernels/shared/gguf_linear.metal:36-55,237-276).
//
// Numerics follow the reference's prefill tile: each weight is dequantised once to fp16(fma(q, s, z))
// (kernels/common/gguf_staged.h:11-16), every product with an input is exact, and sums are fp32. On CDNA4 the fp16
// weights feed the fp16 MFMA, so the inputs enter as fp16 too: a prepare dispatch scales each row by a power of two
// that brings its largest magnitude below 2^16 (so inputs past half's range, like the reference's +-1e5 sparse
// rows, stay finite) and converts the row to fp16, which is exact for every bf16 input in half's normal range; the
// epilogue multiplies the row's sums back by the same power of two.
//
// CDNA4 mapping. A workgroup of four waves (one per SIMD) computes BM rows x 256 columns; wave w owns one 64-column
// plane tile and all BM rows of it, as BM/16 x 4 16x16x32 f16 MFMAs per 32 inputs (BM fp32 accumulators per lane,
// held in the accumulation registers). The product runs weights x activations, so each lane ends holding eight
// consecutive outputs of a row twice over and stores them as 16-byte vectors. Per 64-input step:
//  - the activations (fp16, BM x 64) go global -> LDS with global_load_lds_dwordx4, no registers on the way, two
//    steps ahead into a ring of three stages; all four waves read them as MFMA B fragments, four blocks at a time;
//  - each wave's plane tile codes and meta go global -> LDS the same way, three steps ahead into a ring of four
//    slots only that wave reads, and the wave dequantises its own A fragments from them straight into registers:
//    lane (j, q) takes plane word q of one column, whose eight codes are inputs 4q..4q+3 and 16+4q..19+4q of the
//    group. The prepare dispatch stores each group of 32 fp16 inputs in that order (16-byte chunk q = inputs
//    4q..4q+3 then 16+4q..19+4q), so one 16-byte activation read pairs with one plane word: the dot product over
//    the group is the same sum in another order of its terms;
//  - group 1's weights are dequantised during the step's first half of MFMAs, the next step's group 0 during the
//    second half, in pieces of four weights between MFMAs.
// LDS rows are 128 bytes whose 16-byte chunk c sits in slot c ^ (row % 8), so fragment reads (16 rows x one chunk
// per 16 lanes) and the copies spread over all banks. One barrier a step.
#include <algorithm>
#include <type_traits>

#include "device.hpp"
#include "half_rows.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

constexpr int BK = 64, kStages = 3;
constexpr int kRowBytes = BK * 2;                  // one LDS activation row: 64 fp16
constexpr int kLdsLimit = 160 * 1024;              // LDS a workgroup may hold
// A workgroup of W waves computes BM rows x 256 columns (four plane tiles): W = 4, one wave a SIMD, each owning a
// 64-column plane tile; or W = 8, two waves a SIMD, each owning one half (32 columns) of a plane tile, so that one
// wave's dependency and LDS stalls are covered by the other's work.
// Formats whose codes are 16 bytes a column-group and who have no plane1 (4-bit affine and Q4_K) run W = 8.
template <uint32_t FMT>
constexpr int tile_waves() { return Fmt<FMT>::P0 == 16 && Fmt<FMT>::P1 <= 4 ? 8 : 4; }
// A wave's LDS slot for one step: the step's two groups of the wave's codes (its 256 / W columns x P0 bytes each),
// their plane1 bits (P1 each), then the meta the step reads for the whole plane tile (its meta unit, or both groups'
// units of a format with a unit a group). Each part lies in the planes as in the slot, so it arrives by whole 16-byte
// or dword copies. With four waves the 4-bit formats without plane1 keep 1 KiB for the meta.
template <uint32_t FMT, int W>
struct StepSlot {
  using F = Fmt<FMT>;
  static constexpr int cols = 256 / W;            // the wave's columns of its plane tile
  static constexpr int plane_step = 2 * 64 * F::P0, plane_high_step = 2 * 64 * F::P1;   // a tile's step in the planes
  static constexpr int code = 2 * cols * F::P0, high = 2 * cols * F::P1;
  static constexpr int meta = (F::UNIT == 1 ? 2 : 1) * 64 * F::META;
  static constexpr int high_at = code, meta_at = code + high;
  static constexpr int wave =
      meta_at + (W == 4 ? (F::P0 == 16 && F::P1 == 0 ? 1024 : (meta + 15) / 16 * 16) : (meta + 255) / 256 * 256);
  static constexpr int all = W * wave;            // the slot of every wave
};
template <int BM> constexpr int stage_bytes() { return BM * kRowBytes; }
template <int BM> constexpr int code_base() { return kStages * stage_bytes<BM>(); }
// Step slots per wave: four (a step's copies run three steps ahead, into the slot two behind the one being read),
// or three where four do not fit beside a 256-row tile's stages. Then step s's copies of step s + 3 go to step s's
// own slot, which the wave finished reading (into registers, its LDS reads waited for) and rewriting in place
// (step_coefficients) during step s - 1; nothing reads it during step s.
template <uint32_t FMT, int BM, int W>
constexpr int step_slots() { return code_base<BM>() + 4 * StepSlot<FMT, W>::all <= kLdsLimit ? 4 : 3; }
template <uint32_t FMT, int BM, int W>
constexpr int lds_bytes() { return code_base<BM>() + step_slots<FMT, BM, W>() * StepSlot<FMT, W>::all; }

// global -> LDS copy of SIZE bytes per lane (global_load_lds): lane l's bytes land at lds + SIZE l.
// (The size is spelled as a literal: the host pass of hipcc does not take a template argument there.)
template <int SIZE>
__device__ __forceinline__ void copy_to_lds(const void *src, uint8_t *lds) {
  static_assert(SIZE == 4 || SIZE == 16, "dword or dwordx4 copies");
  const auto dst = (__attribute__((address_space(3))) void *)lds;
  if constexpr (SIZE == 16) __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
  else __builtin_amdgcn_global_load_lds(src, dst, 4, 0, 0);
}
// The workgroup barrier between steps: the waits before it are explicit (a __syncthreads() fence would also wait for
// copies still in flight); LDS writes complete under vmcnt / lgkmcnt are visible to every wave of the workgroup.
// The empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// s_waitcnt immediate for vmcnt(n) alone (gfx9: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int wait_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0070 | 0x0F00; }
// Byte offset of 16-byte chunk c of LDS row r (the XOR swizzle).
__device__ __forceinline__ uint32_t chunk_at(uint32_t r, uint32_t c) { return r * kRowBytes + ((c ^ (r & 7)) << 4); }

// ---------------------------------------------------------------- prepare

// One workgroup per row: the largest magnitude of the row's bf16 inputs (a wave reduction and LDS), then the half
// rows table of the row (half_rows.hpp). Rows of at most 256 NV output chunks are read once, into registers
// (NV > 0); longer ones are read twice.
template <int NV>
__global__ __launch_bounds__(256) void prepare_kernel(const uint16_t *input, uint32_t K, uint16_t *half_input,
                                                      float *row_scale) {
  const uint32_t r = blockIdx.x, vectors = K / 8;
  const u32x2 *units = (const u32x2 *)(input + (size_t)r * K);   // 4-input units
  u32x4 *h = (u32x4 *)(half_input + (size_t)r * K);
  const auto chunk = [&](uint32_t v) __attribute__((always_inline)) {
    const uint32_t u = half_rows_unit(v);
    const u32x2 lo = units[u], hi = units[u + 4];
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };
  uint32_t largest = 0;
  u32x4 held[NV > 0 ? NV : 1];
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t v = threadIdx.x + 256u * i;
      held[i] = v < vectors ? chunk(v) : u32x4{0u, 0u, 0u, 0u};
      largest = max(largest, bf16_largest(held[i]));
    }
  } else {
    for (uint32_t v = threadIdx.x; v < vectors; v += 256) largest = max(largest, bf16_largest(chunk(v)));
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) largest = max(largest, (uint32_t)__shfl_xor((int)largest, d));
  __shared__ uint32_t part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = largest;
  __syncthreads();
  largest = max(max(part[0], part[1]), max(part[2], part[3]));
  const int shift = half_rows_shift(largest);
  const float down = ldexpf(1.0f, -shift);
  if (threadIdx.x == 0) row_scale[r] = ldexpf(1.0f, shift);
  if constexpr (NV > 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t v = threadIdx.x + 256u * i;
      if (v < vectors) h[v] = half_rows_chunk(held[i], down);
    }
  } else {
    for (uint32_t v = threadIdx.x; v < vectors; v += 256) h[v] = half_rows_chunk(chunk(v), down);
  }
}

// ---------------------------------------------------------------- GEMM

// One code of a masked plane word as a float: after masking every other nibble each byte holds one code
// (v_cvt_f32_ubyte0..3). The mask arrives in a register the compiler cannot see through, so each code costs one
// conversion instead of an extract and a conversion.
__device__ __forceinline__ float byte_float(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
// fp16(fma(q, s, z)) of two codes, rounded as the reference rounds: to fp32 by the fma, then to fp16 (the empty asm
// keeps the compiler from fusing the two roundings into one mixed-precision fma).
__device__ __forceinline__ uint32_t dequant_pair(float q0, float q1, Coef k) {
  float v0 = fmaf(q0, k.s, k.z), v1 = fmaf(q1, k.s, k.z);
  asm volatile("" : "+v"(v0), "+v"(v1));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{v0, v1}, half2));
}
// The slot position of column c's 16 bytes of 4-bit codes (and of a Q4_K or Q5_K column's 16-byte header) in a
// step's LDS slot, an involution on 0..63 and on 0..31: lane l of the copy fetches column code_slot(l). Bit 2 of the
// column is flipped with bit 4, so the sixteen columns column_of(j, t) that one read takes over j = 0..15 lie on
// sixteen different 16-byte slots modulo 256 bytes: with the four words q, 64 banks conflict-free (32 banks two-way,
// the least for 32 lanes of 4-byte reads) instead of four ways. Measured: LDS bank conflicts 23% -> 9% of the tile's
// LDS active cycles. (A half tile's 32 columns, 8 a + 4 t + b, keep the property: bits 3 and 2 ^ 4 of the slot take
// four values over a for each t.)
__device__ __forceinline__ uint32_t code_slot(uint32_t c) { return c ^ ((c >> 2) & 4u); }
// The plane tile column whose weights lane j of the MFMA's A operand carries in column block t. The product runs
// weights x activations (D = W X^T), so lane (j', q) of D holds column column_of(4q + i, t) for i = 0..3: with
// this order those are columns 8q + 4(t % 2) + i (blocks 0, 1) and 32 + 8q + 4(t % 2) + i (blocks 2, 3), eight
// consecutive outputs of one row twice over.
__device__ __forceinline__ uint32_t column_of(uint32_t j, int t) {
  return (t >> 1) * 32 + 8 * (j >> 2) + 4 * (t & 1) + (j & 3);
}

// The meta of column c for group h of one step out of the wave's LDS slot: af4g32 the words of its two groups,
// af4g64, af4g128 and af8g64 the one word covering the step, Q8_0 the group's half d, Q4_K and Q5_K the fp32 (s, z)
// and Q6_K the fp32 scales of its two halves that step_coefficients left in place of the column's meta.
template <uint32_t FMT>
__device__ __forceinline__ MetaWords slot_meta(const uint8_t *meta, uint32_t c, int h) {
  if constexpr (FMT == SQ_FMT_Q4K || FMT == SQ_FMT_Q5K) {
    const u32x2 v = *(const u32x2 *)(meta + code_slot(c) * 16 + h * 8);
    return MetaWords{{v[0], v[1], 0u, 0u, 0u}};
  } else if constexpr (FMT == SQ_FMT_Q6K) {
    const uint32_t *w = (const uint32_t *)(meta + c * 20 + h * 8);   // 4-byte aligned
    return MetaWords{{w[0], w[1], 0u, 0u, 0u}};
  } else if constexpr (FMT == SQ_FMT_Q80) {
    return MetaWords{{*(const uint16_t *)(meta + h * 128 + c * 2), 0u, 0u, 0u, 0u}};
  } else if constexpr (FMT == SQ_FMT_AF4G32) {
    return MetaWords{{*(const uint32_t *)(meta + c * 4), *(const uint32_t *)(meta + 256 + c * 4), 0u, 0u, 0u}};
  } else {
    return MetaWords{{*(const uint32_t *)(meta + c * 4), 0u, 0u, 0u, 0u}};
  }
}
// The coefficients of group h (0, 1) of the step, the step's group `group` of the tile, for the first and second
// half of its elements (the same unless the format scales halves, Q6_K). value = fma(q, s, z) with Q6_K's
// s (q - 32) as fma(q, s, -32 s) and Q8_0's d v as fma(v + 128, d, -128 d): both exact, the same values.
template <uint32_t FMT>
__device__ __forceinline__ void group_coef(const MetaWords &m, uint32_t group, int h, Coef &first, Coef &second) {
  if constexpr (FMT == SQ_FMT_Q4K || FMT == SQ_FMT_Q5K) {
    first = Coef{__uint_as_float(m.w[0]), __uint_as_float(m.w[1])};
  } else if constexpr (FMT == SQ_FMT_Q6K) {
    const float s0 = __uint_as_float(m.w[0]), s1 = __uint_as_float(m.w[1]);
    first = Coef{s0, -32.0f * s0};
    second = Coef{s1, -32.0f * s1};
  } else if constexpr (FMT == SQ_FMT_Q80) {
    const float d = f16_to_f32(m.w[0]);
    first = Coef{d, -128.0f * d};
  } else if constexpr (FMT == SQ_FMT_AF4G32) {
    first = coef<FMT>(MetaWords{{m.w[h], 0u, 0u, 0u, 0u}}, group);
  } else {
    first = coef<FMT>(m, group);
  }
  if constexpr (!Fmt<FMT>::HALVES) second = first;
}
// Q4_K and Q5_K: lane l turns column l's 16-byte header in the slot into the fp32 (s, z) of the step's two groups,
// Q6_K its 20 bytes into the fp32 scales of the two groups' halves, in place, so each lane derives one column's
// coefficients instead of four (the wave's reads precede its writes).
template <uint32_t FMT>
__device__ __forceinline__ void step_coefficients(uint8_t *meta, uint32_t step, int lane) {
  if constexpr (FMT == SQ_FMT_Q4K || FMT == SQ_FMT_Q5K) {
    const u32x4 v = *(const u32x4 *)(meta + lane * 16);
    const MetaWords m{{v[0], v[1], v[2], v[3], 0u}};
    const Coef c0 = coef<FMT>(m, 2 * step), c1 = coef<FMT>(m, 2 * step + 1);
    *(f32x4 *)(meta + lane * 16) = f32x4{c0.s, c0.z, c1.s, c1.z};
  } else if constexpr (FMT == SQ_FMT_Q6K) {
    uint32_t *w = (uint32_t *)(meta + lane * 20);   // 4-byte aligned
    const MetaWords m{{w[0], w[1], w[2], w[3], w[4]}};
    const float a = q6k_scale(m, 2 * step, 0), b = q6k_scale(m, 2 * step, 1);
    const float c = q6k_scale(m, 2 * step + 1, 0), d = q6k_scale(m, 2 * step + 1, 1);
    w[0] = __float_as_uint(a);
    w[1] = __float_as_uint(b);
    w[2] = __float_as_uint(c);
    w[3] = __float_as_uint(d);
  }
}

// The dequantisation of one group's NT plane words (one a column block of the wave) as a sequence of
// micro-operations: kind 0 prepares word arg (masks, coefficients), kinds 1, 2, 3 convert, multiply-add and pack
// weight pair arg (word arg / 4). Pairs are software pipelined: pair i's conversion comes after pair i - 1's
// multiply-add and pair i - 2's pack.
struct Micro {
  int kind, arg;
};
template <int NT>
constexpr int micro_ops() { return NT + 3 * 4 * NT; }
template <int NT>
struct MicroTable {
  Micro op[micro_ops<NT>()];
};
template <int NT>
constexpr MicroTable<NT> make_micro_table() {
  MicroTable<NT> t{};
  int n = 0;
  for (int i = 0; i < 4 * NT + 2; ++i) {
    if (i < 4 * NT && i % 4 == 0) t.op[n++] = {0, i / 4};
    if (i < 4 * NT) t.op[n++] = {1, i};
    if (i >= 1 && i <= 4 * NT) t.op[n++] = {2, i - 1};
    if (i >= 2) t.op[n++] = {3, i - 2};
  }
  return t;
}
template <int NT>
constexpr MicroTable<NT> kMicroTable = make_micro_table<NT>();
static_assert(kMicroTable<4>.op[micro_ops<4>() - 1].kind == 3 && kMicroTable<4>.op[micro_ops<4>() - 1].arg == 15,
              "52 micro-operations for four words");
static_assert(kMicroTable<2>.op[micro_ops<2>() - 1].kind == 3 && kMicroTable<2>.op[micro_ops<2>() - 1].arg == 7,
              "26 micro-operations for two words");

// Raw buffer access (the descriptor's last dword for untyped dword access on CDNA3/4): loads past `bytes` read
// zero and stores past it are dropped. kCoherent is the sc1 cache policy, the agent-scope coherence an agent-scope
// atomic load or store takes, so that a piece's sums are seen by a workgroup on another XCD.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_over(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
constexpr int kCoherent = 16;
// A stream dispatch's partials: two slots a workgroup (at most kPrefillUnits workgroups), each holding every wave's
// fp32 sums of one piece, [wave][mi NT + ni][lane] as 16-byte vectors (32 KiB a wave).
constexpr uint32_t kStreamSlotBytes = 256 * 256 * 4, kStreamPartialBytes = 2 * kPrefillUnits * kStreamSlotBytes;
constexpr uint32_t kAbsent = 0x80000000u;   // an offset past the partials: reads zero

// A piece of stream tile t cut in `pieces` pieces (prefill_stream: at most three) arrives at the tile's counter. It
// stores its fp32 sums to the partials at byte offset `slot` (the wave's, acc[mi][ni] at 16 ((mi NT + ni) 64 +
// lane)) and adds one to the counter; the last of the tile's pieces to arrive returns true, returns the counter to
// zero and runs the epilogue, which adds the pieces' sums in K order (so the sum does not depend on the order of
// arrival). The partials go through agent-scope coherent (sc1) accesses and the counter through agent-scope atomics,
// ordered as the decode split reduce orders them (split.hpp): each wave waits for its stores to complete before the
// barrier, thread 0 adds to the counter after it, and the last piece loads only after its add returns. Every wave of
// the workgroup calls it, after its last LDS reads; the counter's value passes through the tile's first LDS word
// (the copies have landed by then).
template <int MI, int NT>
__device__ __forceinline__ bool stream_arrive(const PrefillArgs &a, const f32x4 (&acc)[MI][NT], uint32_t t,
                                              uint32_t pieces, uint32_t slot, int lane, uint8_t *lds) {
  uint32_t &arrival = *(uint32_t *)lds;
  const __amdgpu_buffer_rsrc_t parts = buffer_over(a.partials, kStreamPartialBytes);
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NT; ++ni)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mi][ni]), parts,
                                             slot + ((mi * NT + ni) * 64 + lane) * 16, 0, kCoherent);
  __builtin_amdgcn_s_waitcnt(0);   // this wave's partial stores have completed
  __syncthreads();                 // ... and every wave's
  if (threadIdx.x == 0) {
    const uint32_t before = __hip_atomic_fetch_add(a.counters + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The last arrival is the counter's last use in the dispatch.
    if (before == pieces - 1) __hip_atomic_store(a.counters + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    arrival = before;
  }
  __syncthreads();
  return arrival == pieces - 1;
}

// The prefill dispatch: each workgroup runs one or more pieces of tiles, a piece being steps [first, first + n) of
// row block `row_block` of the dispatch's column group `column_group`.
//   whole tiles: workgroup (x, y) runs row block x of column group y, all of K;
//   SPLIT: workgroup (x, y, z) runs piece z of that tile, cut at split_at, whose fp32 sums a close dispatch adds
//     (prefill_schedule);
//   STREAM (prefill_stream): the first stream_dp workgroups run whole tiles; each of the others runs a range of
//     steps of its row block's stream tiles laid end to end (below), one piece a tile it meets; a piece of every
//     step runs the epilogue itself, and a tile's partial pieces meet through the partials (stream_arrive).
// The body stays in the kernel (the pieces are an outer loop) rather than in a function it calls: the same body
// optimised as a separate function before inlining takes more registers and spills.
template <uint32_t FMT, uint32_t EP, int BM, bool SPLIT, int W, bool STREAM>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(W / 4, W / 4)))
void prefill_kernel(PrefillArgs a) {
  static_assert(!(SPLIT && STREAM), "a stream piece runs its own epilogue");
  using F = Fmt<FMT>;
  using S = StepSlot<FMT, W>;
  static_assert(W == 4 || (W == 8 && F::P0 == 16 && F::P1 <= 4), "eight waves take 16-byte codes, plane1 of 4 bytes");
  constexpr int MI = BM / 16;                         // 16-row blocks of the wave
  constexpr int NT = 16 / W;                          // 16-column blocks of the wave: 4 (a plane tile) or 2 (a half)
  static_assert(MI == 8 || MI == 16, "128- or 256-row tiles");
  constexpr int kStage = stage_bytes<BM>(), kCodeBase = code_base<BM>(), kSlotBytes = S::all;
  constexpr int kSlots = step_slots<FMT, BM, W>();
  // The step's plane copies: the codes, plane1 and meta parts by 16-byte copies of 1 KiB and dword copies of 256 B.
  constexpr int kCode16 = S::code / 1024, kHigh16 = S::high / 1024, kHigh4 = S::high % 1024 / 256;
  constexpr int kHighGroups = F::P1 ? 256 / (32 * (F::P1 ? F::P1 : 1)) : 1;   // eight waves: groups a dword copy
  constexpr int kMeta16 = S::meta / 1024, kMeta4 = S::meta % 1024 / 256;
  static_assert(S::code % 1024 == 0 && S::high % 256 == 0 && S::meta % 256 == 0, "whole copies");
  constexpr int kBCopies = kCode16 + kHigh16 + kHigh4 + kMeta16 + kMeta4;
  constexpr int kACopies = BM / (8 * W);              // activation copies (eight rows each) a wave issues per step
  constexpr int kCopies = kACopies + kBCopies;        // copy instructions a wave issues per step
  static_assert(kCopies < 64, "vmcnt counts to 63");
  static_assert(lds_bytes<FMT, BM, W>() <= kLdsLimit, "the tile's LDS fits a workgroup");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[lds_bytes<FMT, BM, W>()];
  const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t G = a.K >> 5, units = G / F::UNIT, steps = a.K / BK;
  // STREAM: workgroups below stream_dp run one whole tile each (row block b % row blocks, column group b / row
  // blocks); the others run the steps [i range, (i + 1) range) of their row block's stream tiles laid end to end
  // (workgroup stream_dp + i row_blocks + row block), a piece a tile it meets. A row block's workgroups then share
  // their XCD (workgroup b runs on XCD b % 8) and its L2's copy of the row block's activations.
  const uint32_t stream_blocks = STREAM ? a.stream_row_blocks : 1u;
  const bool stream_whole = STREAM && blockIdx.x < a.stream_dp;
  const uint32_t stream_b = blockIdx.x - (STREAM && !stream_whole ? a.stream_dp : 0u);
  const uint32_t stream_rb = stream_b % stream_blocks, stream_i = stream_b / stream_blocks;
  uint32_t stream_at = 0, stream_end = 0;
  if constexpr (STREAM) {
    stream_at = stream_whole ? 0u : stream_i * a.stream_range;
    stream_end = stream_whole ? steps : min(stream_at + a.stream_range, a.stream_tiles / stream_blocks * steps);
  }
  // Byte offset of this wave's part of slot `slot` of the workgroup that runs range ii of this row block.
  const auto slot_at = [&](uint32_t ii, uint32_t slot) __attribute__((always_inline)) {
    return ((2 * (ii * stream_blocks + stream_rb) + slot) * W + wave) * (kStreamSlotBytes / W);
  };
  for (bool again = false;; again = true) {
    uint32_t row_block = blockIdx.x, column_group = blockIdx.y;
    // A stream piece: its tile, the tile's pieces (one a range it meets) and the piece's place among them.
    uint32_t stream_tile = 0, stream_pieces = 1, stream_piece = 0, range0 = 0;
    // The piece's steps of the tile (cut at a multiple of four steps, whole meta units of every format) run with their
    // own numbers from 0, from plane and input pointers moved on by `first`.
    uint32_t first = SPLIT && blockIdx.z ? a.split_at : 0;
    uint32_t n = SPLIT ? (blockIdx.z ? steps - a.split_at : a.split_at) : steps;
    if constexpr (STREAM) {
      if (stream_at >= stream_end) return;
      if (stream_whole) {
        row_block = blockIdx.x % stream_blocks;
        column_group = blockIdx.x / stream_blocks;
        stream_at = stream_end;
      } else {
        const uint32_t c = stream_at / steps;   // the stream column group
        first = stream_at % steps;
        const uint32_t last = min(steps, stream_end - c * steps);
        n = last - first;
        stream_at = c * steps + last;
        row_block = stream_rb;
        column_group = a.stream_dp / stream_blocks + c;
        stream_tile = c * stream_blocks + stream_rb;
        range0 = c * steps / a.stream_range;
        stream_pieces = (c * steps + steps - 1) / a.stream_range - range0 + 1;
        stream_piece = stream_i - range0;
      }
      if (again) {
        // The last piece's copies have landed and every wave has done with the LDS before this piece's copies.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    }
    const uint32_t row0 = row_block * BM;

    // The wave's plane tile (the dispatch's column groups start at column_group0) and its half of it (eight waves).
    // A grid whose tile count is not a multiple of 4 ends short: a spare wave runs tile 0 of its segment and stores
    // nothing.
    const uint32_t half = W == 8 ? (wave & 1u) : 0u;
    uint32_t ptile = (a.column_group0 + column_group) * 4 + wave / (W / 4), s = 0;
    while (s + 1 < a.segments && ptile >= a.seg[s].tiles) ptile -= a.seg[s++].tiles;
    const bool live = ptile < a.seg[s].tiles;
    const Segment seg = a.seg[s];
    // The lane's copy sources in the plane tile: 16-byte copies read 16 lane bytes on, dword copies 4 lane. Four waves:
    // code copy k is group k of the step, lane l column code_slot(l). Eight waves: one code copy a step, lane l group
    // l / 32, column code_slot(l % 32) of the wave's half.
    const size_t tile = live ? ptile : 0;
    const size_t unit0 = F::UNIT == 1 ? 2 * first : 2 * first / F::UNIT;
    const uint32_t code_lane = W == 8 ? (lane >> 5) * 1024 + (32 * half + code_slot(lane & 31)) * 16
                                      : 16 * (F::P0 == 16 ? code_slot(lane) : lane);
    const uint8_t *bplane = seg.plane0 + (tile * G * 64 * F::P0 + (size_t)first * S::plane_step + code_lane);
    const uint8_t *bhigh16 =
        F::P1 ? seg.plane1 + (tile * G * 64 * F::P1 + (size_t)first * S::plane_high_step + 16 * lane) : nullptr;
    // Eight waves copy their half's plane1 bytes only (32 P1 a group), the step's groups packed one after the other
    // in the slot: a dword copy holds kHighGroups groups, lane l byte 4 (l % (64 / kHighGroups)) of group
    // l / (64 / kHighGroups)'s half.
    const uint32_t high_lane = W == 8 ? lane / (64 / kHighGroups) * 64 * F::P1 + 32 * half * F::P1 +
                                            lane % (64 / kHighGroups) * 4
                                      : 4 * lane;
    const uint8_t *bhigh4 =
        F::P1 ? seg.plane1 + (tile * G * 64 * F::P1 + (size_t)first * S::plane_high_step + high_lane) : nullptr;
    const uint8_t *bmeta16 =
        seg.meta + ((tile * units + unit0) * 64 * F::META + 16 * (F::META == 16 ? code_slot(lane) : lane));
    const uint8_t *bmeta4 = seg.meta + ((tile * units + unit0) * 64 * F::META + 4 * lane);
    const uint8_t *xin = (const uint8_t *)a.half_input + (size_t)first * BK * 2;
    uint8_t *const wave_slot = lds + kCodeBase + wave * S::wave;
    uint32_t mask = 0x0F0F0F0Fu;
    asm volatile("" : "+s"(mask));

    // Activations: wave w copies LDS rows BM/W w .. BM/W (w + 1) - 1, eight per instruction: lane l fills chunk slot
    // l % 8 of row 8 i + l / 8, i.e. input chunk (l % 8) ^ (row % 8) (row % 8 = l / 8, the same for every i).
    constexpr int kRowsPerWave = BM / W;
    // Byte offsets of the lane's copy sources, rows clamped to the last live one (a tile past the rows reads it again).
    uint32_t aoff[kACopies];
#pragma unroll
    for (int i = 0; i < kACopies; ++i) {
      const uint32_t r = min(row0 + kRowsPerWave * wave + 8 * i + (lane >> 3), a.rows - 1);
      aoff[i] = (r * a.K + 8 * ((lane & 7) ^ (lane >> 3))) * 2;
    }
    // Step `step`'s activations into stage `stage` (sources clamped to the last step: every step issues as many
    // copies, which the vmcnt waits count on).
    const auto copy_a = [&](uint32_t step, uint32_t stage) __attribute__((always_inline)) {
      const uint8_t *from = xin + (size_t)min(step, n - 1) * BK * 2;
#pragma unroll
      for (int i = 0; i < kACopies; ++i)
        copy_to_lds<16>(from + aoff[i], lds + stage * kStage + (kRowsPerWave * wave + 8 * i) * kRowBytes);
    };
    // Plane copy k of step `from` (clamped) into the wave's slot at dst: the codes' 1 KiB pieces, then plane1's and the
    // meta's 1 KiB and 256-byte pieces.
    const auto copy_b_one = [&](uint32_t from, int k, uint8_t *dst) __attribute__((always_inline)) {
      const size_t meta = (size_t)(F::UNIT == 1 ? 2 * from : 2 * from / F::UNIT) * 64 * F::META;
      if (k < kCode16) {
        copy_to_lds<16>(bplane + (size_t)from * S::plane_step + 1024 * k, dst + 1024 * k);
      } else if (k < kCode16 + kHigh16) {
        const int i = k - kCode16;
        copy_to_lds<16>(bhigh16 + (size_t)from * S::plane_high_step + 1024 * i, dst + S::high_at + 1024 * i);
      } else if (k < kCode16 + kHigh16 + kHigh4) {
        const int i = k - kCode16 - kHigh16;
        copy_to_lds<4>(bhigh4 + (size_t)from * S::plane_high_step + 1024 * kHigh16 +
                           (W == 8 ? kHighGroups * 64 * F::P1 : 256) * i,
                       dst + S::high_at + 1024 * kHigh16 + 256 * i);
      } else if (k < kCode16 + kHigh16 + kHigh4 + kMeta16) {
        const int i = k - kCode16 - kHigh16 - kHigh4;
        copy_to_lds<16>(bmeta16 + meta + 1024 * i, dst + S::meta_at + 1024 * i);
      } else {
        const int i = k - kCode16 - kHigh16 - kHigh4 - kMeta16;
        copy_to_lds<4>(bmeta4 + meta + 1024 * kMeta16 + 256 * i, dst + S::meta_at + 1024 * kMeta16 + 256 * i);
      }
    };
    // Step `step`'s codes, plane1 and meta into slot `slot` of this wave.
    const auto copy_b = [&](uint32_t step, uint32_t slot) __attribute__((always_inline)) {
#pragma unroll
      for (int k = 0; k < kBCopies; ++k) copy_b_one(min(step, n - 1), k, wave_slot + slot * kSlotBytes);
    };

    // Copy c of step `step`'s copies: c < kACopies the activation rows of step + 2, then step + 3's plane copies.
    const auto copy_one = [&](uint32_t step, int c) __attribute__((always_inline)) {
      if (c < kACopies) {
        const uint8_t *from = xin + (size_t)min(step + 2, n - 1) * BK * 2;
        uint8_t *stage = lds + ((step + 2) % kStages) * kStage;
        copy_to_lds<16>(from + aoff[c], stage + (kRowsPerWave * wave + 8 * c) * kRowBytes);
        return;
      }
      copy_b_one(min(step + 3, n - 1), c - kACopies, wave_slot + ((step + 3) % kSlots) * kSlotBytes);
    };

    f32x4 acc[MI][NT];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NT; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Weight fragments (the MFMA's A operand): wq[h][t] = group h of the step, column block t. Group 0 serves the first
    // half of a step's MFMAs while group 1 is dequantised into wq[1], then group 1 serves the second half while the
    // next step's group 0 is dequantised into wq[0]; each register set has one role, so the step loop needs no
    // unrolling.
    u32x4 wq[2][NT];
    // The plane words (8-bit codes: two words, cw and cw1), plane1 bits and meta of group h of a step for the lane's
    // NT columns, out of the step's slot: chunk q of the column (its codes of inputs 4q..4q+3 and 16+4q..19+4q). The
    // meta block holds the whole plane tile, the codes the wave's columns.
    uint32_t cw[2][NT], cw1[2][NT], hb[2][NT];
    MetaWords mw[2][NT];
    const auto read_b = [&](uint32_t slot, int h) __attribute__((always_inline)) {
      const uint8_t *src = wave_slot + slot * kSlotBytes;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t c = column_of(j, t);
        if constexpr (F::P0 == 32) {
          const u32x2 v = *(const u32x2 *)(src + h * 2048 + c * 32 + q * 8);
          cw[h][t] = v[0];
          cw1[h][t] = v[1];
        } else {
          cw[h][t] = *(const uint32_t *)(src + h * (S::code / 2) + code_slot(c) * 16 + q * 4);
        }
        if constexpr (F::P1 == 4) hb[h][t] = src[S::high_at + h * S::cols * 4 + c * 4 + q];
        if constexpr (F::P1 == 8) hb[h][t] = *(const uint16_t *)(src + S::high_at + h * S::cols * 8 + c * 8 + 2 * q);
        mw[h][t] = slot_meta<FMT>(src + S::meta_at, S::cols * half + c, h);
      }
    };
    // The dequantisation of one group's NT words runs as 13 NT micro-operations (see micro_op) spread one or two
    // after each MFMA: prep(t) masks word t and derives its coefficients, then every pair of weights p (word p / 4,
    // fragment register p % 4) is converted (C), multiplied and added (F) and packed to fp16 (P), software
    // pipelined so that no micro-operation waits on the one just before it.
    // 4-bit codes: lo holds the word's slots 0, 4, 1, 5 and hi its slots 2, 6, 3, 7, one a byte, so pair r (slots 2r,
    // 2r + 1) is bytes r / 2 and r / 2 + 2 of hi (r odd) or lo; plane1 bits go to bits 4 (and 5) of those bytes.
    // 8-bit codes: lo and hi are the two words, pair r bytes 2 (r % 2) and 2 (r % 2) + 1 of word r / 2.
    uint32_t lo[NT], hi[NT];
    Coef kw[NT], kw2[NT];
    float cf[4][2], vf[4][2];
    constexpr int kMicro = micro_ops<NT>();
    const auto micro = [&](int u, uint32_t step, int h) __attribute__((always_inline)) {
      const Micro m = kMicroTable<NT>.op[u];
      if (m.kind == 0) {
        const int t = m.arg;
        if constexpr (F::P0 == 32) {
          const uint32_t flip = FMT == SQ_FMT_Q80 ? 0x80808080u : 0u;   // the signed byte v as v + 128
          lo[t] = cw[h][t] ^ flip;
          hi[t] = cw1[h][t] ^ flip;
        } else {
          lo[t] = cw[h][t] & mask;
          hi[t] = (cw[h][t] >> 4) & mask;
          if constexpr (F::P1 == 4) {
            // Fifth bits (bit i of the byte: slot i): the product (24-bit operands, one v_mul_u32_u24) puts bits 0, 4,
            // 1, 5 at 4, 12, 20, 28, and carries between its partial products stay clear of those.
            lo[t] |= ((hb[h][t] & 0x33u) * 0x880110u) & 0x10101010u;
            hi[t] |= (((hb[h][t] >> 2) & 0x33u) * 0x880110u) & 0x10101010u;
          } else if constexpr (F::P1 == 8) {
            // High two bits (bits 2i, 2i + 1: slot i).
            lo[t] |= ((hb[h][t] & 0x0303u) << 4) | ((hb[h][t] & 0x0C0Cu) << 18);
            hi[t] |= (hb[h][t] & 0x3030u) | ((hb[h][t] & 0xC0C0u) << 14);
          }
        }
        group_coef<FMT>(mw[h][t], 2 * step + h, h, kw[t], kw2[t]);
      } else {
        const int p = m.arg, t = p >> 2, r = p & 3, slot = p & 3;
        if (m.kind == 1) {
          if constexpr (F::P0 == 32) {
            const uint32_t src = (r >> 1) ? hi[t] : lo[t];
            cf[slot][0] = byte_float(src, 2 * (r & 1));
            cf[slot][1] = byte_float(src, 2 * (r & 1) + 1);
          } else {
            const uint32_t src = (r & 1) ? hi[t] : lo[t];
            cf[slot][0] = byte_float(src, r >> 1);
            cf[slot][1] = byte_float(src, (r >> 1) + 2);
          }
        } else if (m.kind == 2) {
          // Pairs 0, 1 are the chunk's first-half elements, 2, 3 its second half.
          const Coef k = F::HALVES && r >= 2 ? kw2[t] : kw[t];
          vf[slot][0] = fmaf(cf[slot][0], k.s, k.z);
          vf[slot][1] = fmaf(cf[slot][1], k.s, k.z);
        } else {
          // fp32 by the fma, then fp16: the empty asm keeps the two roundings apart (no fused mixed-precision fma).
          asm volatile("" : "+v"(vf[slot][0]), "+v"(vf[slot][1]));
          wq[h][t][r] = __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{vf[slot][0], vf[slot][1]}, half2));
        }
      }
    };
    const auto dequant_group = [&](uint32_t step, int h) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kMicro; ++u) micro(u, step, h);
    };

    // Prologue: steps 0 and 1's activations, steps 0..2's codes; step 0's group-0 fragments.
    copy_b(0, 0);
    copy_b(1, 1);
    copy_b(2, 2);
    copy_a(0, 0);
    copy_a(1, 1);
    __builtin_amdgcn_s_waitcnt(wait_vm(0));
    lds_barrier();
    step_coefficients<FMT>(wave_slot + S::meta_at, 0, lane);
    read_b(0, 0);
    read_b(0, 1);
    dequant_group(0, 0);

    // Step s copies step s + 2's activations into stage (s + 2) % 3 and step s + 3's codes into slot (s + 3) % 4,
    // one copy instruction before each of its batches in turn (a burst of them at the top of the step stalls the wave
    // on the address unit). It dequantises its own group 1 during its first half and step s + 1's group 0 during its
    // second half, from words read half a step earlier (each half reads the words the next half dequantises: step
    // s + 1's slot has been in LDS since the last barrier). Before the barrier it waits for everything but its own
    // copies, so step s + 1's activations and step s + 2's codes are in.
    // The activation fragments go through registers in batches of four blocks (16 MFMAs), two batches in flight.
    // With copies to LDS outstanding the compiler can only wait for all LDS reads at once, so each batch waits for
    // its own reads (issued a batch earlier) before it issues the next batch's. A step's last batch runs after the
    // barrier, while the next step's first reads are in flight.
    constexpr int kGroups = 2 * MI, kBatch = 4, kBatches = kGroups / kBatch, kSlotsHalf = NT * MI;
    constexpr int kWaitLds = 0xC07F;   // s_waitcnt lgkmcnt(0), the other counters at their maximum
    u32x4 fa[2][kBatch];
    const auto read_batch = [&](uint32_t step, int b) __attribute__((always_inline)) {
      const uint8_t *sa = lds + (step % kStages) * kStage;
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int g = b * kBatch + i;
        fa[b & 1][i] = *(const u32x4 *)(sa + chunk_at((g % MI) * 16 + j, 4 * (g / MI) + q));
      }
    };
    const auto mfma_batch = [&](uint32_t step, int b) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int g = b * kBatch + i, kk = g / MI, mi = g % MI;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          acc[mi][t] = mfma_f16(wq[kk][t], fa[b & 1][i], acc[mi][t]);
          // This MFMA's share of the other group's micro-operations: slot s of the half runs micro-operations
          // [s kMicro / S, (s + 1) kMicro / S).
          const int slot = mi * NT + t, u0 = slot * kMicro / kSlotsHalf, u1 = (slot + 1) * kMicro / kSlotsHalf;
          static_assert(kMicro <= 2 * kSlotsHalf, "at most two micro-operations a slot");
          if (u0 < u1) micro(u0, kk == 0 ? step : step + 1, kk ^ 1);
          if (u0 + 1 < u1) micro(u0 + 1, kk == 0 ? step : step + 1, kk ^ 1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    };
    read_batch(0, 0);
    for (uint32_t step = 0; step < n; ++step) {
      if (step > 0) mfma_batch(step - 1, kBatches - 1);
#pragma unroll
      for (int b = 0; b < kBatches; ++b) {
#pragma unroll
        for (int c = 0; c < kCopies; ++c)
          if (c * kBatches / kCopies == b) copy_one(step, c);
        __builtin_amdgcn_s_waitcnt(kWaitLds);
        if (b + 1 < kBatches) read_batch(step, b + 1);
        if (b == 0) {
          step_coefficients<FMT>(wave_slot + ((step + 1) % kSlots) * kSlotBytes + S::meta_at, step + 1, lane);
          read_b((step + 1) % kSlots, 0);
        }
        if (b == kBatches / 2) read_b((step + 1) % kSlots, 1);
        if (b + 1 < kBatches) mfma_batch(step, b);
      }
      __builtin_amdgcn_s_waitcnt(wait_vm(kCopies));
      lds_barrier();
      if (step + 1 < n) read_batch(step + 1, 0);
    }
    mfma_batch(n - 1, kBatches - 1);

    if constexpr (SPLIT) {
      // Piece z of K: the fp32 sums, exactly, as two 16-bit planes of [rows][split_columns] (the high halves of the
      // bits, then the low; column 64 t + c of the dispatch's plane tile t), stored as the bf16 epilogue stores (eight
      // consecutive columns of a row twice over); split_close_kernel adds the pieces and applies the epilogue.
      if (!live) return;
      const size_t plane = (size_t)a.rows * a.split_columns;
      uint16_t *const high = (uint16_t *)a.partials + blockIdx.z * 2 * plane;
      uint16_t *const low = high + plane;
      const uint32_t col0 = (column_group * 4 + wave / (W / 4)) * 64 + S::cols * half + 8 * q;
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
        const uint32_t r = row0 + mi * 16 + j;
        if (r >= a.rows) continue;
#pragma unroll
        for (int hh = 0; hh < NT / 2; ++hh) {
          const size_t at = (size_t)r * a.split_columns + col0 + 32 * hh;
          u32x4 hi, lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f32x4 &v = acc[mi][2 * hh + (e >> 1)];
            const uint32_t b0 = __float_as_uint(v[2 * (e & 1)]), b1 = __float_as_uint(v[2 * (e & 1) + 1]);
            hi[e] = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
            lo[e] = __builtin_amdgcn_perm(b1, b0, 0x05040100u);
          }
          *(u32x4 *)(high + at) = hi;
          *(u32x4 *)(low + at) = lo;
        }
      }
      return;
    }
    // A tile cut in pieces: piece p's sums (stream_arrive) sit in slot 0 of its range when the range starts inside
    // the tile (every piece but the first, and the first when a range starts with the tile), else in slot 1 (the
    // range's last piece).
    bool complete = true;
    uint32_t slot0 = 0;
    if constexpr (STREAM) {
      if (stream_pieces > 1) {
        slot0 = (column_group - a.stream_dp / stream_blocks) * steps % a.stream_range ? 1u : 0u;
        complete = stream_arrive<MI, NT>(a, acc, stream_tile, stream_pieces,
                                         slot_at(stream_i, stream_piece ? 0u : slot0), lane, lds);
      }
    }
    // Epilogue: lane (j, q) holds row 16 mi + j of each row block at columns 8q..8q+7 of the wave's columns (blocks
    // 0, 1) and, with four column blocks, 32+8q..32+8q+7 (blocks 2, 3): one 16-byte store a row block and pair of
    // column blocks.
    if (live && complete) {
      const uint32_t col0 = seg.out_offset + ptile * 64 + S::cols * half + 8 * q;
      bool pieces_done = false;
      if constexpr (STREAM) {
        if (stream_pieces > 1) {
          // The last piece of a cut tile: the pieces' sums, the others' loaded ahead of their stores with the rows'
          // scales. No branches within, so that the loads overlap the stores: rows past the chunk fall past the
          // output's buffer range and are dropped.
          const __amdgpu_buffer_rsrc_t parts = buffer_over(a.partials, kStreamPartialBytes);
          const uint32_t out_bytes = a.rows * a.out_stride * 2;
          const __amdgpu_buffer_rsrc_t out = buffer_over(a.output, out_bytes);
          const __amdgpu_buffer_rsrc_t aux = buffer_over(a.aux, EP != EpNone ? out_bytes : 0u);
          const auto row_scale = [&](int mi) __attribute__((always_inline)) {
            return a.row_scale[min(row0 + mi * 16 + j, a.rows - 1)];
          };
          const auto piece = [&](uint32_t from, int mi, int ni) __attribute__((always_inline)) {
            return __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(parts, from + (mi * NT + ni) * 1024, 0, kCoherent));
          };
          const auto store_block = [&](int mi, const f32x4 (&sum)[NT], float scale) __attribute__((always_inline)) {
            const uint32_t r = row0 + mi * 16 + j;
#pragma unroll
            for (int hh = 0; hh < NT / 2; ++hh) {
              const uint32_t at = (r * a.out_stride + col0 + 32 * hh) * 2;
              u32x4 ax = {0u, 0u, 0u, 0u};
              if constexpr (EP != EpNone) ax = __builtin_amdgcn_raw_buffer_load_b128(aux, at, 0, 0);
              u32x4 o;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const f32x4 &v = sum[2 * hh + (e >> 1)];
                const float lo = epilogue_bits<EP>(v[2 * (e & 1)] * scale, ax[e] & 0xFFFFu);
                const float hi = epilogue_bits<EP>(v[2 * (e & 1) + 1] * scale, ax[e] >> 16);
                o[e] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
              }
              __builtin_amdgcn_raw_buffer_store_b128(o, out, at, 0, 0);
            }
          };
          if (stream_pieces == 2) {
            // Two pieces: a + b = b + a, so the wave's own sums take the other piece's in either order. Its loads run
            // D row blocks ahead.
            constexpr int D = 4;
            const uint32_t other = slot_at(range0 + (stream_piece ^ 1u), stream_piece ? slot0 : 0u) + lane * 16;
            f32x4 ahead[D][NT];
            float scale_ahead[D];
#pragma unroll
            for (int mi = 0; mi < D; ++mi) {
              scale_ahead[mi] = row_scale(mi);
#pragma unroll
              for (int ni = 0; ni < NT; ++ni) ahead[mi][ni] = piece(other, mi, ni);
            }
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
              f32x4 sum[NT];
#pragma unroll
              for (int ni = 0; ni < NT; ++ni) sum[ni] = acc[mi][ni] + ahead[mi % D][ni];
              const float scale = scale_ahead[mi % D];
              if (mi + D < MI) {
                scale_ahead[mi % D] = row_scale(mi + D);
#pragma unroll
                for (int ni = 0; ni < NT; ++ni) ahead[mi % D][ni] = piece(other, mi + D, ni);
              }
              store_block(mi, sum, scale);
            }
          } else {
            // Three pieces: (x0 + x1) + x2 in K order, a row block ahead. The wave's own piece comes from its
            // registers (its loads take kAbsent and read zero).
            uint32_t from[3];
#pragma unroll
            for (uint32_t p = 0; p < 3; ++p)
              from[p] = p == stream_piece ? kAbsent : slot_at(range0 + p, p ? 0u : slot0) + lane * 16;
            f32x4 next[3][NT];
            float next_scale = row_scale(0);
#pragma unroll
            for (int p = 0; p < 3; ++p)
#pragma unroll
              for (int ni = 0; ni < NT; ++ni) next[p][ni] = piece(from[p], 0, ni);
#pragma unroll
            for (int mi = 0; mi < MI; ++mi) {
              f32x4 sum[NT];
#pragma unroll
              for (int ni = 0; ni < NT; ++ni) {
                const f32x4 x0 = stream_piece == 0 ? acc[mi][ni] : next[0][ni];
                const f32x4 x1 = stream_piece == 1 ? acc[mi][ni] : next[1][ni];
                const f32x4 x2 = stream_piece == 2 ? acc[mi][ni] : next[2][ni];
                sum[ni] = (x0 + x1) + x2;
              }
              const float scale = next_scale;
              if (mi + 1 < MI) {
                next_scale = row_scale(mi + 1);
#pragma unroll
                for (int p = 0; p < 3; ++p)
#pragma unroll
                  for (int ni = 0; ni < NT; ++ni) next[p][ni] = piece(from[p], mi + 1, ni);
              }
              store_block(mi, sum, scale);
            }
          }
          pieces_done = true;
        }
      }
      if (!pieces_done) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const uint32_t r = row0 + mi * 16 + j;
          if (r >= a.rows) continue;
          const float scale = a.row_scale[r];
#pragma unroll
          for (int hh = 0; hh < NT / 2; ++hh) {
            const size_t at = (size_t)r * a.out_stride + col0 + 32 * hh;
            u32x4 aux = {0u, 0u, 0u, 0u};
            if constexpr (EP != EpNone) aux = *(const u32x4 *)(a.aux + at);
            u32x4 out;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const f32x4 &v = acc[mi][2 * hh + (e >> 1)];
              const float lo = epilogue_bits<EP>(v[2 * (e & 1)] * scale, aux[e] & 0xFFFFu);
              const float hi = epilogue_bits<EP>(v[2 * (e & 1) + 1] * scale, aux[e] >> 16);
              out[e] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
            }
            *(u32x4 *)(a.output + at) = out;
          }
        }
      }
    }
    if constexpr (!STREAM) return;
  }
}

// The close of a split dispatch: y = epilogue((piece 0 + piece 1) * 2^e) in bf16, eight columns of one of its plane
// tiles a thread, the pieces' fp32 sums rebuilt from their two 16-bit planes and added in K order.
template <uint32_t EP>
__global__ __launch_bounds__(256) void split_close_kernel(PrefillArgs a, uint32_t tiles) {
  const uint32_t r = blockIdx.y, g = blockIdx.x * 256 + threadIdx.x;
  if (g >= tiles * 8) return;
  uint32_t ptile = a.column_group0 * 4 + g / 8, s = 0;
  while (s + 1 < a.segments && ptile >= a.seg[s].tiles) ptile -= a.seg[s++].tiles;
  if (ptile >= a.seg[s].tiles) return;
  const size_t plane = (size_t)a.rows * a.split_columns, from = (size_t)r * a.split_columns + 8 * g;
  const uint16_t *partials = (const uint16_t *)a.partials;
  const u32x4 h0 = *(const u32x4 *)(partials + from), l0 = *(const u32x4 *)(partials + plane + from);
  const u32x4 h1 = *(const u32x4 *)(partials + 2 * plane + from), l1 = *(const u32x4 *)(partials + 3 * plane + from);
  const size_t at = (size_t)r * a.out_stride + a.seg[s].out_offset + ptile * 64 + 8 * (g % 8);
  const float scale = a.row_scale[r];
  u32x4 x = {0u, 0u, 0u, 0u};
  if constexpr (EP != EpNone) x = *(const u32x4 *)(a.aux + at);
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // Columns 2e, 2e + 1: bits (high << 16) | low of each piece.
    const float a0 = __uint_as_float(__builtin_amdgcn_perm(h0[e], l0[e], 0x05040100u));
    const float a1 = __uint_as_float(__builtin_amdgcn_perm(h0[e], l0[e], 0x07060302u));
    const float b0 = __uint_as_float(__builtin_amdgcn_perm(h1[e], l1[e], 0x05040100u));
    const float b1 = __uint_as_float(__builtin_amdgcn_perm(h1[e], l1[e], 0x07060302u));
    const float lo = epilogue_bits<EP>((a0 + b0) * scale, x[e] & 0xFFFFu);
    const float hi = epilogue_bits<EP>((a1 + b1) * scale, x[e] >> 16);
    out[e] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
  }
  *(u32x4 *)(a.output + at) = out;
}

template <uint32_t FMT, int BM, int MODE>
hipError_t launch_tile(uint32_t epilogue, const PrefillArgs &a, dim3 grid, hipStream_t stream) {
  constexpr int W = tile_waves<FMT>();
  constexpr bool STREAM = MODE == 2;
  constexpr bool SPLIT = MODE == 1;
  const dim3 block(64 * W);
  switch (epilogue) {
    case EpNone:
      hipLaunchKernelGGL((prefill_kernel<FMT, EpNone, BM, SPLIT, W, STREAM>), grid, block, 0, stream, a);
      break;
    case EpResidual:
      hipLaunchKernelGGL((prefill_kernel<FMT, EpResidual, BM, SPLIT, W, STREAM>), grid, block, 0, stream, a);
      break;
    default:
      hipLaunchKernelGGL((prefill_kernel<FMT, EpUpWithGate, BM, SPLIT, W, STREAM>), grid, block, 0, stream, a);
      break;
  }
  return hipGetLastError();
}

template <uint32_t FMT>
hipError_t launch_format(uint32_t epilogue, const PrefillArgs &args, hipStream_t stream) {
  static_assert(lds_bytes<FMT, 256, tile_waves<FMT>()>() <= kLdsLimit, "every format's 256-row tile fits the LDS");
  uint32_t tiles = 0;
  for (uint32_t s = 0; s < args.segments; ++s) tiles += args.seg[s].tiles;
  // The projection's whole width decides the halving, so every dispatch of it (one per format) halves alike.
  const bool split = prefill_split(args.rows, args.out_stride / 64, args.K);
  const PrefillSchedule sc = prefill_schedule(args.rows, tiles, args.K, split);
  PrefillArgs a = args;
  a.column_group0 = 0;
  if (!sc.split) {
    if (sc.bm == 128) return launch_tile<FMT, 128, 0>(epilogue, a, dim3(sc.row_blocks, sc.column_groups), stream);
    // Stream pieces run in the eight-wave tile of formats without plane1 only: the four-wave tile's 256 sums a lane
    // leave no registers for the piece loop (its stream instance spills), and so do Q5_K's plane1 bits in the
    // eight-wave one. Their epilogue addresses the output with 32-bit byte offsets, rows past the chunk included (up
    // to the last row block's end), which must not wrap.
    if constexpr (tile_waves<FMT>() == 8 && Fmt<FMT>::P1 == 0) {
      const PrefillStream st = prefill_stream(sc.row_blocks, sc.column_groups, args.K);
      if (st.stream_tiles && (uint64_t)sc.row_blocks * 256 * args.out_stride * 2 < (1ull << 31)) {
        if (!a.partials || !a.counters) return hipErrorInvalidValue;
        a.stream_dp = st.dp_tiles;
        a.stream_tiles = st.stream_tiles;
        a.stream_range = st.range;
        a.stream_row_blocks = sc.row_blocks;
        return launch_tile<FMT, 256, 2>(epilogue, a, dim3(st.workgroups), stream);
      }
    }
    return launch_tile<FMT, 256, 0>(epilogue, a, dim3(sc.row_blocks, sc.column_groups), stream);
  }
  if (!a.partials) return hipErrorInvalidValue;
  a.column_group0 = sc.whole_groups;
  a.split_at = sc.split_at;
  a.split_columns = (sc.column_groups - sc.whole_groups) * 256;
  hipError_t e = launch_tile<FMT, 256, 1>(epilogue, a, dim3(sc.row_blocks, sc.column_groups - sc.whole_groups, 2),
                                          stream);
  if (e != hipSuccess) return e;
  const uint32_t split_tiles = tiles - 4 * sc.whole_groups;
  const dim3 grid((split_tiles * 8 + 255) / 256, a.rows), block(256);
  switch (epilogue) {
    case EpNone: hipLaunchKernelGGL(split_close_kernel<EpNone>, grid, block, 0, stream, a, split_tiles); break;
    case EpResidual: hipLaunchKernelGGL(split_close_kernel<EpResidual>, grid, block, 0, stream, a, split_tiles); break;
    default: hipLaunchKernelGGL(split_close_kernel<EpUpWithGate>, grid, block, 0, stream, a, split_tiles); break;
  }
  return hipGetLastError();
}

}  // namespace

// Whether a projection of `rows` x `plane_tiles` plane tiles halves its tiles' K: when its 256-row tiles number
// kPrefillSplitTiles to kPrefillUnits / 2 (one round of halves over the compute units, where whole tiles would leave
// half of them idle or take 128-row tiles at 0.7 of the cost each, measured: the dequantisation and the step's fixed
// work are shared by half the rows), and each half starts on whole meta units (K a multiple of 512). Costs in 256-row
// steps a compute unit: a half costs its steps, about two for its prologue and stores, and about six for the close.
// (Whole rounds of tiles followed by cut ones were measured too: 4096 x 14336 at M 2048 ran 309 us against 266 whole,
// and 5120 x 27648 gained nothing.)
bool prefill_split(uint32_t rows, uint32_t plane_tiles, uint32_t K) {
  const uint32_t columns = (plane_tiles + 3) / 4, steps = K / BK, units = kPrefillUnits;
  const uint64_t tiles256 = (uint64_t)((rows + 255) / 256) * columns;
  const uint64_t tiles128 = (uint64_t)((rows + 127) / 128) * columns;
  if (tiles256 < kPrefillSplitTiles || 2 * tiles256 > units || steps % 8) return false;
  const double cost128 = 0.7 * steps * (double)((tiles128 + units - 1) / units);
  return steps / 2.0 + 8.0 < std::min(cost128, (double)steps);
}
// The tile height with fewer rounds of workgroups over the compute units (one workgroup a unit), a 128-row tile
// costing 0.7 of a 256-row one; 256 rows cut in halves for a halved projection.
PrefillSchedule prefill_schedule(uint32_t rows, uint32_t plane_tiles, uint32_t K, bool split) {
  const uint32_t columns = (plane_tiles + 3) / 4, units = kPrefillUnits;
  const uint32_t blocks128 = (rows + 127) / 128, blocks256 = (rows + 255) / 256;
  if (split) return {256, 1, blocks256, columns, 0, K / BK / 2};
  const uint64_t rounds128 = ((uint64_t)blocks128 * columns + units - 1) / units;
  const uint64_t rounds256 = ((uint64_t)blocks256 * columns + units - 1) / units;
  if (7 * rounds128 < 10 * rounds256) return {128, 0, blocks128, columns, 0, 0};
  return {256, 0, blocks256, columns, 0, 0};
}
// The stream schedule of a whole-K dispatch of 256-row tiles, row_blocks x column_groups of them, K / 64 steps each,
// in one dispatch. Whole rounds of kPrefillUnits tiles run as whole tiles (dp_tiles: whole column groups, so that the
// row blocks divide the units), one a workgroup; the rest (stream_tiles, between half a round and a round and a
// half) are cut into pieces: each row block's stream tiles have their steps laid end to end and cut into ranges of
// `range` steps (a multiple of four: whole meta units of every format), one a workgroup, kPrefillUnits / row_blocks
// ranges at most a row block, so that the last round's work spreads over every compute unit instead of leaving some
// idle. A tile meets at most ceil(steps / range) + 1 ranges: a range of at least half a tile cuts it in at most
// three pieces, which stream_arrive joins. None (stream_tiles 0) where the tiles fill whole rounds or fill less than
// one (a partial round alone runs each tile faster than a full one: measured on MI355X, a dispatch of 216 tiles
// ran 6% slower as stream pieces), or the steps or row blocks do not allow it. A partial last round's tiles also
// run faster than a full round's (fewer compute units share the memory system), which bounds the gain: measured, 4%
// on 448 tiles of K 4096, 1-2% on 864 of K 5120 and 6% on 544 of K 5120 (prefill_gemm_m2048_config2.txt).
PrefillStream prefill_stream(uint32_t row_blocks, uint32_t column_groups, uint32_t K) {
  const uint32_t units = kPrefillUnits, steps = K / BK, tiles = row_blocks * column_groups;
  if (K % (4 * BK) || steps < 8 || !row_blocks || units % row_blocks || tiles % units == 0 || tiles <= units)
    return {0, 0, 0, 0};
  const uint32_t rounds = tiles / units, rest = tiles % units;
  const uint32_t dp = 2 * rest >= units ? rounds * units : (rounds - 1) * units;
  const uint32_t stream = tiles - dp, ranges = units / row_blocks;   // ranges a row block
  const uint32_t work = stream / row_blocks * steps;                  // a row block's stream steps
  const uint32_t range = (work + 4 * ranges - 1) / (4 * ranges) * 4;
  if (steps > 2 * range) return {0, 0, 0, 0};
  return {dp, stream, range, dp + row_blocks * ((work + range - 1) / range)};
}
PrefillScratch prefill_scratch_bytes(uint32_t rows, uint32_t plane_tiles, uint32_t K) {
  if (prefill_split(rows, plane_tiles, K)) return {(uint64_t)2 * rows * ((plane_tiles + 3) / 4) * 256 * 4, 0};
  // A stream dispatch (any of the projection's, one a format, whose 256-row tiles are at most all of the
  // projection's, whether or not the whole projection's schedule takes 256-row tiles) stores the fp32 sums of at most
  // two pieces a stream workgroup, 256 x 256 x 4 bytes each, and keeps a counter a stream tile (at most a round and
  // a half of tiles). Reserved for every format: the plan does not know them.
  const uint32_t row_blocks = (rows + 255) / 256, columns = (plane_tiles + 3) / 4, tiles = row_blocks * columns;
  if (tiles <= kPrefillUnits || K % (4 * BK) || K / BK < 8 || kPrefillUnits % row_blocks) return {0, 0};
  const uint64_t stream = std::min<uint64_t>(tiles, 3 * kPrefillUnits / 2);
  return {(uint64_t)2 * kPrefillUnits * 256 * 256 * 4, stream * 4};
}

hipError_t launch_prefill_prepare(const uint16_t *input, uint32_t rows, uint32_t K, uint16_t *half_input,
                                  float *row_scale, hipStream_t stream) {
  const uint32_t chunks = K / 8;
  const dim3 grid(rows), block(256);
  if (chunks <= 256) hipLaunchKernelGGL(prepare_kernel<1>, grid, block, 0, stream, input, K, half_input, row_scale);
  else if (chunks <= 512) hipLaunchKernelGGL(prepare_kernel<2>, grid, block, 0, stream, input, K, half_input, row_scale);
  else if (chunks <= 1024) hipLaunchKernelGGL(prepare_kernel<4>, grid, block, 0, stream, input, K, half_input, row_scale);
  else if (chunks <= 2048) hipLaunchKernelGGL(prepare_kernel<8>, grid, block, 0, stream, input, K, half_input, row_scale);
  else hipLaunchKernelGGL(prepare_kernel<0>, grid, block, 0, stream, input, K, half_input, row_scale);
  return hipGetLastError();
}

hipError_t launch_prefill(uint32_t fmt, uint32_t epilogue, const PrefillArgs &a, hipStream_t stream) {
  switch (fmt) {
    case SQ_FMT_AF4G32: return launch_format<SQ_FMT_AF4G32>(epilogue, a, stream);
    case SQ_FMT_AF4G64: return launch_format<SQ_FMT_AF4G64>(epilogue, a, stream);
    case SQ_FMT_AF4G128: return launch_format<SQ_FMT_AF4G128>(epilogue, a, stream);
    case SQ_FMT_Q4K: return launch_format<SQ_FMT_Q4K>(epilogue, a, stream);
    case SQ_FMT_Q5K: return launch_format<SQ_FMT_Q5K>(epilogue, a, stream);
    case SQ_FMT_Q6K: return launch_format<SQ_FMT_Q6K>(epilogue, a, stream);
    case SQ_FMT_Q80: return launch_format<SQ_FMT_Q80>(epilogue, a, stream);
    case SQ_FMT_AF8G64: return launch_format<SQ_FMT_AF8G64>(epilogue, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sq::kern
