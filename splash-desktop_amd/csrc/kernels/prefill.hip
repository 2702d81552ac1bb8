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
// CDNA4 mapping: a 512-thread workgroup computes a 256-row x 128-column tile; per 64-input step it stages the
// activations (fp16, 256 x 64) and the dequantised weights (fp16, 128 x 64) in LDS, and its eight waves each run a
// 64 x 64 block as 4 x 4 16x16x32 f16 MFMAs per 32 inputs. The next step's global loads are in flight while the
// current step's MFMAs run.
#include "device.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

constexpr int BM = 256, BN = 128, BK = 64, kThreads = 512;
constexpr int kPad = 8;                      // halves of padding per LDS row
constexpr int kRow = BK + kPad;              // LDS row stride in halves

// ---------------------------------------------------------------- prepare

__global__ __launch_bounds__(256) void prepare_kernel(const uint16_t *input, uint32_t K, uint16_t *half_input,
                                                      float *row_scale) {
  const uint32_t r = blockIdx.x;
  const uint16_t *x = input + (size_t)r * K;
  uint32_t largest = 0;   // magnitude bits of the largest |x| (bf16 bits order like the values)
  for (uint32_t k = threadIdx.x; k < K; k += 256) largest = max(largest, (uint32_t)(x[k] & 0x7FFFu));
  __shared__ uint32_t part[256];
  part[threadIdx.x] = largest;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) part[threadIdx.x] = max(part[threadIdx.x], part[threadIdx.x + s]);
    __syncthreads();
  }
  largest = part[0];
  // Exponent field of the largest magnitude: scale by 2^-(e - 15) when it is 2^16 or more, so it ends below 2^16.
  const int exponent = (int)(min(largest, 0x7F80u) >> 7) - 127;
  const int shift = exponent >= 16 ? exponent - 15 : 0;
  const float down = ldexpf(1.0f, -shift);
  if (threadIdx.x == 0) row_scale[r] = ldexpf(1.0f, shift);
  uint16_t *h = half_input + (size_t)r * K;
  for (uint32_t k = threadIdx.x; k < K; k += 256) h[k] = f32_to_f16(bf16_to_f32(x[k]) * down);
}

// ---------------------------------------------------------------- GEMM

template <uint32_t FMT, uint32_t EP>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
  using F = Fmt<FMT>;
  __shared__ uint16_t lds_a[BM * kRow];
  __shared__ uint16_t lds_b[BN * kRow];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15, q = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;   // wave's 64-row and 64-column block

  // Column tile: BN columns = two 64-column plane tiles of one segment (segments hold whole 64-column tiles; a
  // workgroup's two tiles are consecutive tiles of the dispatch and may straddle two segments).
  const uint32_t row0 = blockIdx.x * BM;
  const uint32_t G = a.K >> 5, units = G / F::UNIT, steps = a.K / BK;

  // B staging: thread t dequantises 16 weights: column c = t % 128, group half h = t / 128 (0..3 -> G32 u = h >> 1,
  // 16-element half h & 1 of it).
  const int bc = tid & 127, bh = tid >> 7, bu = bh >> 1, bhalf = bh & 1;
  uint32_t ptile = blockIdx.y * 2 + (bc >> 6), s = 0;
  while (s + 1 < a.segments && ptile >= a.seg[s].tiles) ptile -= a.seg[s++].tiles;
  const Segment seg = a.seg[s];
  // A grid of an odd tile count ends in a workgroup whose second 64 columns lie past the last segment.
  const bool blive = ptile < seg.tiles;
  const uint8_t *bplane = seg.plane0 + ((size_t)(blive ? ptile : 0) * G * 64 + (bc & 63)) * 16;
  const uint8_t *bmeta = seg.meta + ((size_t)(blive ? ptile : 0) * units * 64 + (bc & 63)) * F::META;

  // A staging: thread t copies 64 bytes: row t / 2 ... 256 rows x 128 bytes = 32 KiB = 512 x 64 B.
  const int ar = tid >> 1, ah = tid & 1;
  const uint32_t arow = row0 + ar;
  const bool alive = arow < a.rows;
  const uint16_t *asrc = a.half_input + (size_t)(alive ? arow : 0) * a.K + ah * 32;

  u32x4 ra[4];
  uint32_t rb[2];
  MetaWords rm;
  const auto load = [&](uint32_t step) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[i] = alive ? *(const u32x4 *)(asrc + (size_t)step * BK + 8 * i) : u32x4{0u, 0u, 0u, 0u};
    const uint32_t g = step * 2 + bu;
    if (blive) {
      const u32x2 w = __builtin_nontemporal_load((const u32x2 *)(bplane + (size_t)g * 1024 + 8 * bhalf));
      rb[0] = w[0];
      rb[1] = w[1];
      rm = load_meta<FMT>(bmeta + (size_t)(g / F::UNIT) * 64 * F::META);
    } else {
      rb[0] = rb[1] = 0u;
      rm = MetaWords{{0u, 0u, 0u, 0u}};
    }
  };
  // Words c = 2 bhalf, 2 bhalf + 1 of the unit hold elements 4c..4c+3 and 16+4c..16+4c+3.
  const auto stage = [&](uint32_t step) __attribute__((always_inline)) {
    uint32_t *dst_a = (uint32_t *)(lds_a + ar * kRow + ah * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) *(u32x4 *)(dst_a + 4 * i) = ra[i];
    const uint32_t g = step * 2 + bu;
    const Coef k = coef<FMT>(rm, g / F::SG);
    uint16_t *dst_b = lds_b + bc * kRow + bu * 32;
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const uint32_t word = rb[cc], c = 2 * bhalf + cc;
      uint32_t lo[2], hi[2];   // elements 4c..4c+3 and 16+4c..16+4c+3 as fp16 pairs
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float v0 = fmaf((float)((word >> (4 * p)) & 15u), k.s, k.z);
        const float v1 = fmaf((float)((word >> (16 + 4 * p)) & 15u), k.s, k.z);
        const uint32_t pair = (uint32_t)f32_to_f16(v0) | ((uint32_t)f32_to_f16(v1) << 16);
        if (p < 2) lo[p] = pair;
        else hi[p - 2] = pair;
      }
      *(u32x2 *)(dst_b + 4 * c) = u32x2{lo[0], lo[1]};
      *(u32x2 *)(dst_b + 16 + 4 * c) = u32x2{hi[0], hi[1]};
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = f32x4{0.f, 0.f, 0.f, 0.f};

  load(0);
  for (uint32_t step = 0; step < steps; ++step) {
    stage(step);
    __syncthreads();
    if (step + 1 < steps) load(step + 1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 fa[4], fb[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
        fa[mi] = *(const u32x4 *)(lds_a + (wm * 64 + mi * 16 + j) * kRow + kk * 32 + 8 * q);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
        fb[ni] = *(const u32x4 *)(lds_b + (wn * 64 + ni * 16 + j) * kRow + kk * 32 + 8 * q);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma_f16(fa[mi], fb[ni], acc[mi][ni]);
    }
    __syncthreads();
  }

  // Epilogue: lane (j, q) holds rows 4q + i and column j of each 16 x 16 block.
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    const int lc = wn * 64 + ni * 16 + j;   // column within the workgroup's 128
    uint32_t ct = blockIdx.y * 2 + (lc >> 6), cs = 0;
    while (cs + 1 < a.segments && ct >= a.seg[cs].tiles) ct -= a.seg[cs++].tiles;
    if (ct >= a.seg[cs].tiles) continue;
    const uint32_t col = a.seg[cs].out_offset + ct * 64 + (lc & 63);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t r = row0 + wm * 64 + mi * 16 + 4 * q + i;
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
  const dim3 grid((a.rows + BM - 1) / BM, (tiles + 1) / 2), block(kThreads);
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
