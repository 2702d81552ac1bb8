// Measurement aid with no counterpart in the reference: a read-only streaming kernel, the floor that the HBM-bound
// tiles are judged against on the same buffers and launch shapes (bench.py reports it beside the GEMV).
//
// Workgroup w reads its contiguous share of the source in 16-byte nontemporal loads, four in flight a lane, folds
// them with xor and writes one word, so nothing it reads can be optimised away.
#include "device.hpp"
#include "kernels.hpp"

namespace sq::kern {
namespace {

__global__ __launch_bounds__(1024) void stream_read_kernel(const u32x4 *src, uint64_t vectors, uint32_t *sink) {
  const uint64_t share = (vectors + gridDim.x - 1) / gridDim.x, begin = share * blockIdx.x;
  const uint64_t end = begin + share < vectors ? begin + share : vectors;
  uint32_t fold = 0;
  uint64_t v = begin + threadIdx.x;
  for (; v + 3 * blockDim.x < end; v += 4 * blockDim.x) {
    u32x4 a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = __builtin_nontemporal_load(src + v + i * blockDim.x);
#pragma unroll
    for (int i = 0; i < 4; ++i) fold ^= a[i][0] ^ a[i][1] ^ a[i][2] ^ a[i][3];
  }
  for (; v < end; v += blockDim.x) {
    const u32x4 a = __builtin_nontemporal_load(src + v);
    fold ^= a[0] ^ a[1] ^ a[2] ^ a[3];
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) fold ^= (uint32_t)__shfl_xor((int)fold, d);
  if ((threadIdx.x & 63) == 0) atomicXor(sink + blockIdx.x, fold);
}

}  // namespace

hipError_t launch_stream_read(const void *src, uint64_t bytes, uint32_t *sink, uint32_t workgroups, uint32_t threads,
                              hipStream_t stream) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(threads), 0, stream, (const u32x4 *)src, bytes / 16,
                     sink);
  return hipGetLastError();
}

}  // namespace sq::kern
