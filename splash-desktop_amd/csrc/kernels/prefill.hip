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
// CDNA4 mapping. A 512-thread workgroup computes a 256-row x 256-column tile, its eight waves 128 x 64 each as 8 x 4
// 16x16x32 f16 MFMAs per 32 inputs (128 fp32 accumulators per lane, two waves per SIMD, so one wave's VALU and LDS
// work runs under the other's MFMAs). Per 64-input step, double buffered in LDS (2 x 64 KiB):
//  - the activations (fp16, 256 x 64) go global -> LDS with global_load_lds_dwordx4, no registers on the way;
//  - the codes and meta of the tile's columns go global -> LDS the same way, one step ahead of their use, and lane
//    l of wave w dequantises group w / 4 of column l of plane tile w % 4 into fp16 in natural input order, written as
//    four 16-byte chunks;
//  - both tiles keep 128-byte rows whose 16-byte chunk c sits in slot c ^ (row % 8), so the MFMA fragment reads
//    (16 lanes, 16 rows, one chunk) and the chunk writes (8 lanes a pass, one row each) spread over all banks.
// Step s + 1's activation copies and step s + 2's code loads are issued before step s's MFMAs, and step s + 1's
// weights are dequantised into the other buffer between them, a 16-byte chunk after each 16-row block's MFMAs (one
// wave per SIMD has no other wave to hide the VALU and LDS work behind); one barrier a step.
#include <type_traits>

#include "device.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

constexpr int BM = 256, BN = 256, BK = 64, kThreads = 512;
constexpr int kRowBytes = BK * 2;                            // one LDS row: 64 fp16
constexpr int kStageBytes = (BM + BN) * kRowBytes;           // A rows then B rows
constexpr int kCodeBytes = BN * 32;                          // a step's raw codes: [4 tiles][2 groups][64 columns][16 B]
constexpr int kMetaBytes = BN * 16;                          // a step's meta: [4 tiles][up to 2 units][64 columns][META]
constexpr int kCodeBase = 2 * kStageBytes, kMetaBase = kCodeBase + 2 * kCodeBytes;
constexpr int kLdsBytes = kMetaBase + 2 * kMetaBytes;
// global -> LDS copy of SIZE bytes per lane (global_load_lds): lane l's bytes land at lds + SIZE l.
// (The size is spelled as a literal: the host pass of hipcc does not take a template argument there.)
template <int SIZE>
__device__ __forceinline__ void copy_to_lds(const void *src, uint8_t *lds) {
  static_assert(SIZE == 4 || SIZE == 16, "dword or dwordx4 copies");
  const auto dst = (__attribute__((address_space(3))) void *)lds;
  if constexpr (SIZE == 16) __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
  else __builtin_amdgcn_global_load_lds(src, dst, 4, 0, 0);
}
// s_waitcnt immediates (gfx9: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8): a vmcnt below 16 with
// lgkmcnt(0) (kWaitLgkm), or without an lgkm wait (kWaitVm).
constexpr int kWaitLgkm = 0x0070, kWaitVm = 0x0F70;
// The workgroup barrier between steps: the waits before it are explicit (a __syncthreads() fence would also wait for
// the code copies still in flight); LDS writes complete under lgkmcnt are visible to every wave of the workgroup.
// The empty asm statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// Byte offset of 16-byte chunk c of LDS row r (the XOR swizzle).
__device__ __forceinline__ uint32_t chunk_at(uint32_t r, uint32_t c) { return r * kRowBytes + ((c ^ (r & 7)) << 4); }

// ---------------------------------------------------------------- prepare

// One workgroup per row: the row's bf16 inputs in 16-byte vectors (K is a multiple of 64), the largest magnitude
// from a wave reduction and LDS, then the fp16 row scaled by 2^-e where 2^e brings the largest below 2^16.
__global__ __launch_bounds__(256) void prepare_kernel(const uint16_t *input, uint32_t K, uint16_t *half_input,
                                                      float *row_scale) {
  const uint32_t r = blockIdx.x, vectors = K / 8;
  const u32x4 *x = (const u32x4 *)(input + (size_t)r * K);
  u32x4 *h = (u32x4 *)(half_input + (size_t)r * K);
  uint32_t largest = 0;   // magnitude bits of the largest |x| (bf16 bit patterns order like the magnitudes)
  for (uint32_t v = threadIdx.x; v < vectors; v += 256) {
    const u32x4 w = x[v];
#pragma unroll
    for (int e = 0; e < 4; ++e) largest = max(largest, max(w[e] & 0x7FFFu, (w[e] >> 16) & 0x7FFFu));
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) largest = max(largest, (uint32_t)__shfl_xor((int)largest, d));
  __shared__ uint32_t part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = largest;
  __syncthreads();
  largest = max(max(part[0], part[1]), max(part[2], part[3]));
  // Exponent field of the largest magnitude: scale by 2^-(e - 15) when it is 2^16 or more, so it ends below 2^16.
  const int exponent = (int)(min(largest, 0x7F80u) >> 7) - 127;
  const int shift = exponent >= 16 ? exponent - 15 : 0;
  const float down = ldexpf(1.0f, -shift);
  if (threadIdx.x == 0) row_scale[r] = ldexpf(1.0f, shift);
  for (uint32_t v = threadIdx.x; v < vectors; v += 256) {
    const u32x4 w = x[v];
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = (uint32_t)f32_to_f16(bf16_to_f32(w[e] & 0xFFFFu) * down) |
             ((uint32_t)f32_to_f16(bf16_to_f32(w[e] >> 16) * down) << 16);
    h[v] = o;
  }
}

// ---------------------------------------------------------------- GEMM

// Eight codes of one plane word as floats in natural input order: word q holds inputs 4q..4q+3 at bits 0, 16, 4,
// 20 (part 0) and 16+4q..19+4q at bits 8, 24, 12, 28 (part 1).
// The codes of one plane word's part (inputs 4q..4q+3 at bits 0, 16, 4, 20, or 16+4q..19+4q at bits 8, 24, 12, 28)
// as floats: each byte of lo and hi holds one code (v_cvt_f32_ubyte0..3). The mask arrives in a register the
// compiler cannot see through, so each code costs one conversion instead of an extract and a conversion.
__device__ __forceinline__ float byte_float(uint32_t v, int b) { return (float)((v >> (8 * b)) & 0xFFu); }
__device__ __forceinline__ void word_codes(uint32_t w, uint32_t mask, int part, float (&v)[4]) {
  const uint32_t lo = w & mask, hi = (w >> 4) & mask;
  v[0] = byte_float(lo, part);
  v[1] = byte_float(lo, part + 2);
  v[2] = byte_float(hi, part);
  v[3] = byte_float(hi, part + 2);
}
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));
// fp16(fma(q, s, z)) of two codes, rounded as the reference rounds: to fp32 by the fma, then to fp16 (the empty asm
// keeps the compiler from fusing the two roundings into one mixed-precision fma).
__device__ __forceinline__ uint32_t dequant_pair(float q0, float q1, Coef k) {
  float v0 = fmaf(q0, k.s, k.z), v1 = fmaf(q1, k.s, k.z);
  asm volatile("" : "+v"(v0), "+v"(v1));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{v0, v1}, half2));
}

template <uint32_t FMT, uint32_t EP>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
  using F = Fmt<FMT>;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kLdsBytes];
  const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = wave >> 2, wn = wave & 3;   // the wave's 128-row and 64-column block
  const uint32_t row0 = blockIdx.x * BM;
  const uint32_t G = a.K >> 5, units = G / F::UNIT, steps = a.K / BK;

  // Weights: wave w brings group h = w / 4 of each step of plane tile 4 blockIdx.y + w % 4 and its meta unit into
  // LDS (both groups' waves copy a shared unit: the same bytes to the same place), and lane l dequantises the group
  // for column l of the tile. A grid of a
  // tile count not a multiple of 4 ends short: its spare waves dequantise tile 0 into columns nothing stores.
  const uint32_t bt = wave & 3, bh = wave >> 2;
  uint32_t ptile = blockIdx.y * 4 + bt, s = 0;
  while (s + 1 < a.segments && ptile >= a.seg[s].tiles) ptile -= a.seg[s++].tiles;
  const bool blive = ptile < a.seg[s].tiles;
  const Segment seg = a.seg[s];
  const uint8_t *bplane = seg.plane0 + ((size_t)(blive ? ptile : 0) * G * 64 + lane) * 16 + (size_t)bh * 1024;
  const uint8_t *bmeta = seg.meta + ((size_t)(blive ? ptile : 0) * units * 64 + lane) * F::META;
  const uint32_t bcol = 64 * bt + lane;
  // LDS offsets of this wave's codes and of the meta its group reads: [tile][group][64 columns][16 B] and
  // [tile][unit][64 columns][META], one unit per tile and step unless 32-input scale groups give each group its own
  // (at most 4 KiB either way: 16-byte meta comes in 256-input units).
  constexpr uint32_t MU = F::UNIT == 1 ? 2 : 1;
  static_assert(4 * MU * 64 * F::META <= kMetaBytes, "a step's meta fits its stage");
  const uint32_t code_at = (bt * 2 + bh) * 1024;
  const uint32_t meta_at = (bt * MU + (MU == 2 ? bh : 0)) * 64 * F::META;
  uint32_t mask = 0x0F0F0F0Fu;
  asm volatile("" : "+s"(mask));

  // Activations: wave w copies LDS rows 32 w .. 32 w + 31, eight per instruction: lane l fills chunk slot l % 8 of
  // row 8 i + l / 8, i.e. input chunk (l % 8) ^ (row % 8) (row % 8 = l / 8, the same for every i). The fp16 copy
  // holds whole 256-row tiles (rows past the live ones are never stored).
  const uint16_t *asrc = a.half_input + (size_t)(row0 + 32 * wave + (lane >> 3)) * a.K + 8 * ((lane & 7) ^ (lane >> 3));
  // Step `step`'s activations into stage `stage`; its codes and meta into code stage `cstage`.
  const auto copy_a = [&](uint32_t step, uint32_t stage) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      copy_to_lds<16>(asrc + (size_t)8 * i * a.K + (size_t)step * BK,
                      lds + stage * kStageBytes + (32 * wave + 8 * i) * kRowBytes);
  };
  const auto copy_b = [&](uint32_t step, uint32_t cstage) __attribute__((always_inline)) {
    copy_to_lds<16>(bplane + (size_t)(2 * step) * 1024, lds + kCodeBase + cstage * kCodeBytes + code_at);
    copy_to_lds<F::META>(bmeta + (size_t)((2 * step + bh) / F::UNIT) * 64 * F::META,
                         lds + kMetaBase + cstage * kMetaBytes + meta_at);
  };
  u32x4 code;
  MetaWords mw;
  const auto read_codes = [&](uint32_t cstage) __attribute__((always_inline)) {
    code = *(const u32x4 *)(lds + kCodeBase + cstage * kCodeBytes + code_at + lane * 16);
    const uint8_t *m = lds + kMetaBase + cstage * kMetaBytes + meta_at + lane * F::META;
    if constexpr (F::META == 4) {
      mw = MetaWords{{*(const uint32_t *)m, 0u, 0u, 0u}};
    } else {
      const u32x4 v = *(const u32x4 *)m;
      mw = MetaWords{{v[0], v[1], v[2], v[3]}};
    }
  };
  // Chunk mm = 0..3 (inputs 8 mm .. 8 mm + 7 of the wave's group of the step) into weight stage `stage`.
  const auto write_chunk = [&](uint32_t step, uint32_t stage, int mm) __attribute__((always_inline)) {
    const Coef k = coef<FMT>(mw, 2 * step + bh);
    float v0[4], v1[4];
    word_codes(code[(2 * mm) & 3], mask, mm >> 1, v0);
    word_codes(code[(2 * mm + 1) & 3], mask, mm >> 1, v1);
    const u32x4 out = {dequant_pair(v0[0], v0[1], k), dequant_pair(v0[2], v0[3], k), dequant_pair(v1[0], v1[1], k),
                       dequant_pair(v1[2], v1[3], k)};
    *(u32x4 *)(lds + stage * kStageBytes + BM * kRowBytes + chunk_at(bcol, 4 * bh + mm)) = out;
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int mi = 0; mi < 8; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Prologue: step 0's activations, codes and meta, then step 1's codes and meta; step 0's weights dequantised.
  copy_a(0, 0);
  copy_b(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  copy_b(min(1u, steps - 1), 1);
  read_codes(0);
#pragma unroll
  for (int mm = 0; mm < 4; ++mm) write_chunk(0, 0, mm);
  __builtin_amdgcn_s_waitcnt(0);
  lds_barrier();
  // Step s: stage s % 2 holds its activations and weights, code stage (s + 1) % 2 step s + 1's codes. The step
  // copies step s + 1's activations (stage (s + 1) % 2) and step s + 2's codes (code stage s % 2), and between its
  // MFMAs dequantises step s + 1's weights into stage (s + 1) % 2.
  constexpr int kCopies = 4 + 1 + 1;   // a step's copy instructions per wave: activations, codes, meta
  for (uint32_t step = 0; step < steps; ++step) {
    const uint32_t stage = step & 1, next = min(step + 1, steps - 1), ahead = min(step + 2, steps - 1);
    copy_a(next, stage ^ 1);
    copy_b(ahead, stage);
    // The codes and meta of step s + 1 (copied by this wave one step ago) are in: everything but this step's
    // copies has completed.
    __builtin_amdgcn_s_waitcnt(kWaitVm | kCopies);
    read_codes(stage ^ 1);
    const uint8_t *sa = lds + stage * kStageBytes, *sb = sa + BM * kRowBytes;
    // Sixteen groups g = (kk, mi): four MFMAs of A block mi against the four B blocks of input half kk. Each
    // group's A fragment is read two groups ahead (half 1's B fragments during half 0); after every fourth group,
    // one of the wave's four 16-byte chunks of the next step's weights.
    const auto read_a = [&](int g) __attribute__((always_inline)) {
      return *(const u32x4 *)(sa + chunk_at(wm * 128 + (g & 7) * 16 + j, 4 * (g >> 3) + q));
    };
    u32x4 fb[2][4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) fb[0][ni] = *(const u32x4 *)(sb + chunk_at(wn * 64 + ni * 16 + j, q));
    u32x4 fa[3];
    fa[0] = read_a(0);
    fa[1] = read_a(1);
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      const int kk = g >> 3, mi = g & 7;
      if (g + 2 < 16) fa[(g + 2) % 3] = read_a(g + 2);
      if (g < 4) fb[1][g] = *(const u32x4 *)(sb + chunk_at(wn * 64 + g * 16 + j, 4 + q));
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma_f16(fa[g % 3], fb[kk][ni], acc[mi][ni]);
      if (g % 4 == 3) write_chunk(next, stage ^ 1, g / 4);
    }
    // This step's activation copies (issued first) and chunk writes are done; its code and meta copies, read by
    // this wave only, may still be in flight.
    __builtin_amdgcn_s_waitcnt(kWaitLgkm | 2);
    lds_barrier();
  }

  // Epilogue: lane (j, q) holds rows 4q + i and column j of each 16 x 16 block.
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    const uint32_t lc = wn * 64 + ni * 16 + j;   // column within the workgroup's 256
    uint32_t ct = blockIdx.y * 4 + (lc >> 6), cs = 0;
    while (cs + 1 < a.segments && ct >= a.seg[cs].tiles) ct -= a.seg[cs++].tiles;
    if (ct >= a.seg[cs].tiles) continue;
    const uint32_t col = a.seg[cs].out_offset + ct * 64 + (lc & 63);
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t r = row0 + wm * 128 + mi * 16 + 4 * q + i;
        if (r >= a.rows) continue;
        const size_t at = (size_t)r * a.out_stride + col;
        a.output[at] = f32_to_bf16(epilogue<EP>(acc[mi][ni][i] * a.row_scale[r], a.aux, at));
      }
  }
}

template <uint32_t FMT>
hipError_t launch_format(uint32_t epilogue, const PrefillArgs &a, hipStream_t stream) {
  uint32_t tiles = 0;
  for (uint32_t s = 0; s < a.segments; ++s) tiles += a.seg[s].tiles;
  const dim3 grid((a.rows + BM - 1) / BM, (tiles + 3) / 4), block(kThreads);
  switch (epilogue) {
    case EpNone: hipLaunchKernelGGL((prefill_kernel<FMT, EpNone>), grid, block, 0, stream, a); break;
    case EpResidual: hipLaunchKernelGGL((prefill_kernel<FMT, EpResidual>), grid, block, 0, stream, a); break;
    default: hipLaunchKernelGGL((prefill_kernel<FMT, EpUpWithGate>), grid, block, 0, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_prepare(const uint16_t *input, uint32_t rows, uint32_t K, uint16_t *half_input,
                                  float *row_scale, hipStream_t stream) {
  hipLaunchKernelGGL(prepare_kernel, dim3(rows), dim3(256), 0, stream, input, K, half_input, row_scale);
  return hipGetLastError();
}

hipError_t launch_prefill(uint32_t fmt, uint32_t epilogue, const PrefillArgs &a, hipStream_t stream) {
  switch (fmt) {
    case SQ_FMT_AF4G32: return launch_format<SQ_FMT_AF4G32>(epilogue, a, stream);
    case SQ_FMT_AF4G64: return launch_format<SQ_FMT_AF4G64>(epilogue, a, stream);
    case SQ_FMT_AF4G128: return launch_format<SQ_FMT_AF4G128>(epilogue, a, stream);
    case SQ_FMT_Q4K: return launch_format<SQ_FMT_Q4K>(epilogue, a, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace sq::kern
