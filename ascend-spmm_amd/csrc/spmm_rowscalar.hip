// Thread-per-row scalar CSR SpMM: the baseline that the block path's speed-up
// is also stated against.  It is not used by any operator.
//
// One thread owns one output row.  For each 16-byte piece of the row it walks
// the row's nonzeros in order and accumulates value * dense[col, piece] in
// fp32, then rounds once.  No work splitting, no shared memory, no
// cooperation between lanes: the classic scalar CSR kernel, widened to 16-byte
// loads so that the comparison is not against byte-sized accesses.
#include "common.h"
#include "lanevec.h"

namespace spmm {
namespace {

using lanes::LaneVec;
using lanes::clampi;

template <typename T, typename I>
__global__ __launch_bounds__(256) void csr_rowscalar(const I* __restrict__ rowptr, const I* __restrict__ col,
                                                     const T* __restrict__ value, const T* __restrict__ dense,
                                                     int64_t rows, int64_t nnz, int64_t K, int64_t N,
                                                     T* __restrict__ out) {
  constexpr int V = LaneVec<T>::V;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int64_t a = clampi(static_cast<int64_t>(rowptr[r]), 0, nnz);
  const int64_t b = clampi(static_cast<int64_t>(rowptr[r + 1]), a, nnz);
  for (int64_t c0 = 0; c0 < N; c0 += V) {
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
    lanes::accumulate<T, I>(acc, a, b, col, value, dense, K, N, c0);
    LaneVec<T>::store(out + r * N + c0, acc);
  }
}

}  // namespace

spmm_status launch_rowscalar(int32_t index_type, int32_t value_type, const void* rowptr, const void* col,
                             const void* value, int64_t rows, int64_t nnz, const void* dense, int64_t K,
                             int64_t N, void* out, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, 256)));
#define SPMM_ROWSCALAR(T, I)                                                                          \
  hipLaunchKernelGGL((csr_rowscalar<T, I>), grid, dim3(256), 0, stream, static_cast<const I*>(rowptr), \
                     static_cast<const I*>(col), static_cast<const T*>(value),                       \
                     static_cast<const T*>(dense), rows, nnz, K, N, static_cast<T*>(out))
  if (value_type == SPMM_VALUE_F16) {
    if (index_type == SPMM_INDEX_I32)
      SPMM_ROWSCALAR(_Float16, int32_t);
    else
      SPMM_ROWSCALAR(_Float16, int64_t);
  } else {
    if (index_type == SPMM_INDEX_I32)
      SPMM_ROWSCALAR(float, int32_t);
    else
      SPMM_ROWSCALAR(float, int64_t);
  }
#undef SPMM_ROWSCALAR
  return check_launch("csr_rowscalar");
}

}  // namespace spmm
