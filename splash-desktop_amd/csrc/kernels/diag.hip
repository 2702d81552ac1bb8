// Measurement aids with no counterpart in the reference (bench.py reports them beside the tiles they bound):
//  - a read-only streaming kernel, the HBM floor of the GEMV on the same buffers and launch shapes: the grid strides
//    over the source in 16-byte nontemporal loads, two in flight a lane, folds them with xor and writes one word a
//    workgroup, so nothing it reads can be optimised away;
//  - an MFMA loop, the ceiling of the prefill GEMM: every wave runs eight independent chains of the 16x16x32 f16
//    MFMA the prefill tile runs, on operands the compiler cannot fold, and stores a value no run produces.
#include "device.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

__global__ __launch_bounds__(1024) void stream_read_kernel(const u32x4 *src, uint64_t vectors, uint32_t *sink) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t fold = 0;
  uint64_t v = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; v + stride < vectors; v += 2 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + v), b = __builtin_nontemporal_load(src + v + stride);
    fold ^= a[0] ^ a[1] ^ a[2] ^ a[3] ^ b[0] ^ b[1] ^ b[2] ^ b[3];
  }
  if (v < vectors) {
    const u32x4 a = __builtin_nontemporal_load(src + v);
    fold ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
  // A store only when the thread's vectors fold to the marker word 0x9E3779B9, which a measured source does not (a
  // test plants it): the reads stay, no atomic or store tail is timed, and the workgroup's sink word names the thread
  // (threadIdx.x + 1) whose fold matched.
  if (fold == 0x9E3779B9u) sink[blockIdx.x] = threadIdx.x + 1;
}

// Workgroups of four waves (one a SIMD). The launch holds residency to one or two waves a SIMD by the LDS each
// workgroup reserves, so both cases run the same code. (Compiled for two waves a SIMD: with more registers to spare
// the compiler rotates the accumulators through overlapping ranges, which chains the MFMAs.)
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mfma_peak_kernel(uint32_t iterations, float *sink) {
  const uint32_t seed = threadIdx.x * 2654435761u + blockIdx.x;
  // fp16 operands near 1 (exponent 0x3C, mantissa from the seed): sums grow but stay finite over any run.
  const uint32_t h = 0x3C003C00u | (seed & 0x00FF00FFu);
  const u32x4 a{h, h ^ 0x10001u, h ^ 0x20002u, h ^ 0x30003u}, b{h ^ 0x40004u, h ^ 0x50005u, h ^ 0x60006u, h};
  f32x4 acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (uint32_t i = 0; i < iterations; ++i)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = mfma_f16(a, b, acc[c]);
  float t = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) t += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  if (t == -1.0f) sink[blockIdx.x] = t;
}

}  // namespace

hipError_t launch_stream_read(const void *src, uint64_t bytes, uint32_t *sink, uint32_t workgroups, uint32_t threads,
                              hipStream_t stream) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(threads), 0, stream, (const u32x4 *)src, bytes / 16,
                     sink);
  return hipGetLastError();
}

hipError_t launch_mfma_peak(uint32_t workgroups, uint32_t waves_per_simd, uint32_t iterations, float *sink,
                            hipStream_t stream) {
  // 160 KiB of LDS a compute unit: 96 KiB a workgroup leaves room for one, 64 KiB for two.
  if (waves_per_simd != 1 && waves_per_simd != 2) return hipErrorInvalidValue;
  const uint32_t lds = waves_per_simd == 1 ? 96u << 10 : 64u << 10;
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(workgroups), dim3(256), lds, stream, iterations, sink);
  return hipGetLastError();
}

}  // namespace sq::kern
