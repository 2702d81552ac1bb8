// The K-split reduction shared by the decode tiles (reference: kernels/shared/split_reduce.h:14-45): each split's
// workgroup stores fp32 partials [split][rows][stride], and the last workgroup to arrive at the output block's
// counter adds them in split order and returns the counter to zero, so results do not depend on scheduling.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sq::kern {

// Adds this split's totals to the others' in split order when this workgroup arrives last; returns false when
// another workgroup still has to arrive. index[b][i]: the partial's offset within a split.
//
// Every access to the partials and the counter is an agent-scope atomic (sc1: coherent across the XCDs' L2s). Each
// wave waits for its partial stores to complete before thread 0 adds to the counter, and the last arriver loads the
// partials only after its add returns. This is the memory model's agent-scope release/acquire without the L2
// writeback and invalidate, which only ordinary (non-sc1) accesses need.
template <int NB, int R>
__device__ __forceinline__ bool split_reduce(float (&total)[NB][R], const bool (&live)[NB][R],
                                             const size_t (&index)[NB][R], float *partials, size_t split_elements,
                                             uint32_t split, uint32_t splits, uint32_t *counter, bool owner) {
  if (owner) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i)
        if (live[b][i])
          __hip_atomic_store(&partials[split * split_elements + index[b][i]], total[b][i], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  __shared__ uint32_t arrival;
  __builtin_amdgcn_s_waitcnt(0);   // this wave's partial stores have completed
  __syncthreads();                 // ... and every wave's
  if (threadIdx.x == 0) arrival = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (arrival != splits - 1) return false;
  if (owner) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i) {
        if (!live[b][i]) continue;
        float v = 0.0f;
        for (uint32_t p = 0; p < splits; ++p)
          v += p == split ? total[b][i]
                          : __hip_atomic_load(&partials[p * split_elements + index[b][i]], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        total[b][i] = v;
      }
  }
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

}  // namespace sq::kern
