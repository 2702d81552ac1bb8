// The K-split reduction shared by the decode tiles (reference: kernels/shared/split_reduce.h:14-45): each split's
// workgroup stores fp32 partials [split][rows][stride], and the last workgroup to arrive at the output block's
// counter adds them in split order and returns the counter to zero, so results do not depend on scheduling.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sq::kern {

// sum[i] = the live values' partials at at[i] + p * stride added in split order p = 0..splits-1 (from 0). Two splits'
// loads of every value go out before their adds, so the sum waits for one memory round trip per two splits; the
// loop stays a loop, so the tail's code stays short.
template <int N>
__device__ __forceinline__ void sum_splits(float (&sum)[N], const bool (&live)[N], float *const (&at)[N],
                                           size_t stride, uint32_t splits) {
#pragma unroll
  for (int i = 0; i < N; ++i) sum[i] = 0.0f;
  uint32_t p = 0;
#pragma unroll 1
  for (; p + 2 <= splits; p += 2) {
    float got[2][N];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int i = 0; i < N; ++i)
        got[d][i] = live[i] ? __hip_atomic_load(at[i] + (size_t)(p + d) * stride, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : 0.0f;
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int i = 0; i < N; ++i) sum[i] += got[d][i];
  }
  if (p < splits)
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (live[i]) sum[i] += __hip_atomic_load(at[i] + (size_t)p * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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
    // Every split's partials, this one's included (its stores above hold `total` bit for bit).
    float sum[NB * R], *at[NB * R];
    bool on[NB * R];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i) {
        at[b * R + i] = partials + index[b][i];
        on[b * R + i] = live[b][i];
      }
    sum_splits(sum, on, at, split_elements, splits);
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < R; ++i)
        if (live[b][i]) total[b][i] = sum[b * R + i];
  }
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

}  // namespace sq::kern
