// Work-group-wide lower-bound search over a monotone device array.
#pragma once

#include "common.h"

namespace spmm {

// First index i in [lo, hi] with value(i) >= pos (hi if none), for two
// positions at once: the first half of the work-group searches posA, the
// second half posB.  Each round probes `half` evenly spaced indices and keeps
// the bracket of the first hit, so a pointer array of 10^5..10^6 entries takes
// three or four rounds of one load per thread instead of a 17-20 step chain
// of dependent loads.  All threads of the work-group must call it.
template <typename F>
__device__ inline void wg_lower_bound2(F value, int64_t lo0, int64_t hi0, int64_t posA, int64_t posB,
                                       int64_t& outA, int64_t& outB) {
  __shared__ int s_min[2];
  __shared__ int64_t s_ans[2];
  const int half = blockDim.x >> 1;
  const int q = threadIdx.x >= half ? 1 : 0;
  const int k = threadIdx.x - q * half;
  const int64_t pos = q ? posB : posA;
  int64_t lo = lo0, hi = hi0;
  bool done = false;
  for (int round = 0; round < 12; ++round) {
    if (threadIdx.x < 2) s_min[threadIdx.x] = INT32_MAX;
    __syncthreads();
    const int64_t n = hi - lo;
    const bool final_round = n <= half;
    if (!done) {
      const int64_t r = final_round ? lo + k : lo + (n * (k + 1)) / (half + 1);
      if ((!final_round || k < n) && value(r) >= pos) atomicMin(&s_min[q], k);
    }
    __syncthreads();
    if (!done) {
      const int km = s_min[q];
      if (final_round) {
        if (km != INT32_MAX) hi = lo + km;
        done = true;
      } else if (km == INT32_MAX) {
        lo = lo + (n * half) / (half + 1) + 1;
      } else {
        const int64_t rk = lo + (n * (km + 1)) / (half + 1);
        lo = km == 0 ? lo : lo + (n * km) / (half + 1) + 1;
        hi = rk;
      }
    }
    if (__syncthreads_and(done)) break;
  }
  if (k == 0) s_ans[q] = hi;
  __syncthreads();
  outA = s_ans[0];
  outB = s_ans[1];
}

}  // namespace spmm
