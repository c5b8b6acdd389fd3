// CSR gather path of the MI355X SpMM library (the vector/AIV part).
//
// Semantics follow the reference's vector engine
// (kernels/op_kernel/spmm_csr.cpp:383-423, 468-549 and the AIV branch of
// kernels/op_kernel/spmm_ascend_cube.cpp:586-673, 782-875):
//   out[i, :] = sum_{p in row i, nonzero order} value[p] * dense[col[p], :]
// accumulated in fp32 and rounded once to the output type.
//
// Work decomposition (MI355X-native, not the reference's 40-core split):
//  * The nonzero positions are cut into fixed ranges of kGatherRange
//    positions ([j*kGatherRange, (j+1)*kGatherRange)).  A "lane group" of
//    L lanes (L = width / 8 for fp16, width / 4 for fp32, capped at 64; each
//    lane owns 16 bytes of an output row) processes one range.
//  * A row that lies inside one range is accumulated sequentially by that
//    group and written directly.  A row that crosses range ends leaves one
//    fp32 partial per range in the workspace ("tail" in the range where it
//    starts, "head" in each later range); the fix-up kernel adds them in range
//    order.  Cut points depend only on the row pointer, so every output element
//    has the same operation sequence for every width N: results are
//    deterministic and bit-identical across widths.
//  * The dense row gather is a 16-byte load per lane; the L lanes of a group
//    read L*16 contiguous bytes of one dense row (coalesced).
#include "common.h"
#include "lanevec.h"

namespace spmm {
namespace {

using lanes::LaneVec;
using lanes::accumulate;
using lanes::clampi;

// Geometry shared by the main and fix-up kernels.  Ranges are absolute
// positions [j*kGatherRange, (j+1)*kGatherRange) of the nonzero arrays, so the
// host needs only the array extent (no read-back of the row pointer).
template <typename I>
struct Ranges {
  const I* rowptr;
  int64_t row_lo, row_hi;  // vector rows handled
  int64_t nnz;             // extent of col[] / value[]
  int64_t nranges;         // max(1, ceil(nnz / kGatherRange))

  // Row pointer clamped into [0, nnz] so no position leaves the arrays.
  __device__ inline int64_t rp(int64_t r) const {
    return clampi(static_cast<int64_t>(rowptr[r]), 0, nnz);
  }
  __device__ inline int64_t lo(int64_t j) const { return j * kGatherRange; }
  __device__ inline int64_t hi(int64_t j) const {
    const int64_t h = (j + 1) * kGatherRange;
    return h < nnz ? h : nnz;
  }
  // First row r in [row_lo, row_hi] with rp(r) >= pos.
  __device__ inline int64_t lower_row(int64_t pos) const {
    int64_t a = row_lo, b = row_hi;
    while (a < b) {
      int64_t m = a + ((b - a) >> 1);
      if (rp(m) < pos) a = m + 1; else b = m;
    }
    return a;
  }
  __device__ inline int64_t row_begin(int64_t j) const { return j == 0 ? row_lo : lower_row(lo(j)); }
  __device__ inline int64_t row_end(int64_t j) const { return j == nranges - 1 ? row_hi : lower_row(lo(j + 1)); }
};

// One lane group per (range j, column chunk cc).
template <typename T, typename I>
__global__ __launch_bounds__(256) void gather_main(Ranges<I> g, const I* __restrict__ col,
                                                   const T* __restrict__ value,
                                                   const T* __restrict__ dense, int64_t K,
                                                   int64_t N, T* __restrict__ out,
                                                   float* __restrict__ ws, int log2L,
                                                   int64_t chunks, int64_t slot) {
  constexpr int V = LaneVec<T>::V;
  const int L = 1 << log2L;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t item = tid >> log2L;
  const int lane = static_cast<int>(tid & (L - 1));
  if (item >= g.nranges * chunks) return;
  const int64_t j = item / chunks;
  const int64_t cc = item - j * chunks;
  const int64_t c0 = (cc * L + lane) * V;
  if (c0 >= N) return;

  const int64_t plo = g.lo(j), phi = g.hi(j);
  const int64_t rb = g.row_begin(j), re = g.row_end(j);

  // Head: positions [plo, ...) of a row that started in an earlier range.
  if (j > 0 && rb > g.row_lo) {
    const int64_t stop = g.rp(rb);
    if (stop > plo) {
      float acc[V];
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = 0.f;
      accumulate<T, I>(acc, plo, stop < phi ? stop : phi, col, value, dense, K, N, c0);
      float* dst = ws + (2 * j) * slot + c0;
#pragma unroll
      for (int i = 0; i < V; ++i) dst[i] = acc[i];
    }
  }
  for (int64_t r = rb; r < re; ++r) {
    const int64_t a = g.rp(r), b = g.rp(r + 1);
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
    if (b <= phi) {
      accumulate<T, I>(acc, a, b, col, value, dense, K, N, c0);
      LaneVec<T>::store(out + r * N + c0, acc);
    } else {
      // Tail: the row continues into the next range.
      accumulate<T, I>(acc, a, phi, col, value, dense, K, N, c0);
      float* dst = ws + (2 * j + 1) * slot + c0;
#pragma unroll
      for (int i = 0; i < V; ++i) dst[i] = acc[i];
    }
  }
}

// Adds the partials of every row that crosses range ends, in range order.
template <typename T, typename I>
__global__ __launch_bounds__(256) void gather_fixup(Ranges<I> g, int64_t N, T* __restrict__ out,
                                                    const float* __restrict__ ws, int log2L,
                                                    int64_t chunks, int64_t slot) {
  constexpr int V = LaneVec<T>::V;
  const int L = 1 << log2L;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t item = tid >> log2L;
  const int lane = static_cast<int>(tid & (L - 1));
  if (item >= (g.nranges - 1) * chunks) return;
  const int64_t j = item / chunks;
  const int64_t cc = item - j * chunks;
  const int64_t c0 = (cc * L + lane) * V;
  if (c0 >= N) return;

  const int64_t rb = g.row_begin(j), re = g.row_end(j);
  if (re <= rb) return;
  const int64_t r = re - 1;
  const int64_t stop = g.rp(r + 1);
  if (stop <= g.hi(j)) return;  // last row of range j ends inside it

  float acc[V];
  const float* src = ws + (2 * j + 1) * slot + c0;
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = src[i];
  for (int64_t k = j + 1; k < g.nranges && g.lo(k) < stop; ++k) {
    const float* h = ws + (2 * k) * slot + c0;
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = acc[i] + h[i];
  }
  LaneVec<T>::store(out + r * N + c0, acc);
}

template <typename T, typename I>
spmm_status gather_typed(const void* rowptr, const void* col, const void* value, int64_t nnz,
                         int64_t row_lo, int64_t row_hi, const void* dense, int64_t K,
                         int64_t N, void* out, void* ws, size_t ws_bytes, hipStream_t stream) {
  constexpr int V = LaneVec<T>::V;
  if (row_hi <= row_lo) return SPMM_OK;
  Ranges<I> g;
  g.rowptr = static_cast<const I*>(rowptr);
  g.row_lo = row_lo;
  g.row_hi = row_hi;
  g.nnz = nnz < 0 ? 0 : nnz;
  g.nranges = g.nnz > 0 ? ceil_div(g.nnz, kGatherRange) : 1;

  const int64_t lanes_needed = N / V;
  int log2L = 0;
  while ((1 << log2L) < lanes_needed && log2L < 6) ++log2L;
  const int L = 1 << log2L;
  const int64_t chunks = ceil_div(lanes_needed, L);
  const int64_t slot = gather_slot_floats(N);
  const size_t need = static_cast<size_t>(2 * g.nranges) * slot * sizeof(float);
  if (g.nranges > 1 && (ws == nullptr || ws_bytes < need))
    return fail(SPMM_ERR_CONTRACT, "gather workspace too small: need " + std::to_string(need) +
                                       " bytes, got " + std::to_string(ws_bytes));

  const int64_t threads = g.nranges * chunks * L;
  const int64_t blocks = ceil_div(threads, 256);
  hipLaunchKernelGGL((gather_main<T, I>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                     g, static_cast<const I*>(col), static_cast<const T*>(value),
                     static_cast<const T*>(dense), K, N, static_cast<T*>(out),
                     static_cast<float*>(ws), log2L, chunks, slot);
  spmm_status st = check_launch("gather_main");
  if (st != SPMM_OK || g.nranges < 2) return st;
  const int64_t fthreads = (g.nranges - 1) * chunks * L;
  hipLaunchKernelGGL((gather_fixup<T, I>), dim3(static_cast<unsigned>(ceil_div(fthreads, 256))),
                     dim3(256), 0, stream, g, N, static_cast<T*>(out),
                     static_cast<const float*>(ws), log2L, chunks, slot);
  return check_launch("gather_fixup");
}

}  // namespace

size_t gather_workspace_bytes(int64_t nnz, int64_t width) {
  const int64_t nr = (nnz > 0 ? ceil_div(nnz, kGatherRange) : 1);
  return static_cast<size_t>(2 * nr) * gather_slot_floats(width) * sizeof(float);
}

spmm_status launch_gather(int32_t index_type, int32_t value_type, const void* rowptr,
                          const void* col, const void* value, int64_t nnz, int64_t row_lo,
                          int64_t row_hi, const void* dense, int64_t dense_rows, int64_t width,
                          void* out, void* workspace, size_t workspace_bytes,
                          hipStream_t stream) {
  if (value_type == SPMM_VALUE_F16) {
    if (index_type == SPMM_INDEX_I32)
      return gather_typed<_Float16, int32_t>(rowptr, col, value, nnz, row_lo, row_hi, dense,
                                             dense_rows, width, out, workspace, workspace_bytes,
                                             stream);
    return gather_typed<_Float16, int64_t>(rowptr, col, value, nnz, row_lo, row_hi, dense,
                                           dense_rows, width, out, workspace, workspace_bytes,
                                           stream);
  }
  if (index_type == SPMM_INDEX_I32)
    return gather_typed<float, int32_t>(rowptr, col, value, nnz, row_lo, row_hi, dense,
                                        dense_rows, width, out, workspace, workspace_bytes,
                                        stream);
  return gather_typed<float, int64_t>(rowptr, col, value, nnz, row_lo, row_hi, dense, dense_rows,
                                      width, out, workspace, workspace_bytes, stream);
}

}  // namespace spmm
