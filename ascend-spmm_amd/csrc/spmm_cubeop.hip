// The legacy spmm_cube operator: 16-row windows whose nonzeros carry an
// encoded column id col = (c << 4) | r (c: dense row, r: row inside the
// window).  Semantics follow the reference kernel
// (kernels/op_kernel/spmm_cube.cpp:53-146): within window w, maximal runs of
// consecutive nonzeros with the same c form one 16x1 block whose row r holds
// the value of the run's last nonzero with row r, and
//   out[16*w + r, :] = sum over the window's runs of block[r] * dense[c, :].
//
// MI355X design: the encoded windows are decoded on the device into the
// BCSR 16x1 layout of the block path (one block per run), then the MFMA block
// kernel of spmm_ascend_cube runs on it.  Decoding is a handful of
// one-thread-per-item passes plus one rocPRIM scan:
//   1. mark window starts and ends, 2. flag run starts, 3. scan the flags,
//   4. record each run's first position and column, 5. window -> run
//   pointer, 6. each run writes its 16 block values (last write wins).
#include <rocprim/device/device_scan.hpp>

#include "common.h"

namespace spmm {
namespace {

constexpr int kThreads = 256;

template <typename I>
__device__ inline int64_t clamp_pos(const I* rowptr, int64_t w, int64_t nnz) {
  const int64_t v = static_cast<int64_t>(rowptr[w]);
  return v < 0 ? 0 : (v > nnz ? nnz : v);
}

template <typename I>
__device__ inline int64_t decode_col(I v) {
  return static_cast<int64_t>(v) >> 4;  // arithmetic shift: negative ids stay negative
}

__global__ void cube_clear(int32_t* __restrict__ flag, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) flag[i] = 0;
}

// Window boundaries start runs: positions rowptr[w] and rowptr[w+1] (clamped
// to [0, nnz]) of every non-empty window.
template <typename I>
__global__ void cube_window_marks(const I* __restrict__ rowptr, int64_t windows, int64_t nnz,
                                  int32_t* __restrict__ flag) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (w >= windows) return;
  const int64_t a = clamp_pos(rowptr, w, nnz), b = clamp_pos(rowptr, w + 1, nnz);
  if (a < b) {
    flag[a] = 1;
    if (b < nnz) flag[b] = 1;
  }
}

// flag[p] = 1 where a run starts: a window boundary, or a column change.
template <typename I>
__global__ void cube_run_flags(const I* __restrict__ col, int64_t nnz, int32_t* __restrict__ flag) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= nnz) return;
  const bool start = p == 0 || flag[p] != 0 || decode_col(col[p]) != decode_col(col[p - 1]);
  flag[p] = start ? 1 : 0;
}

// For every run start p (run k = excl[p]): its first position and column
// (-1 when outside [0, K)); the last thread stores the run count.
template <typename I>
__global__ void cube_runs(const I* __restrict__ col, int64_t nnz, int64_t K, const int32_t* __restrict__ flag,
                          const int32_t* __restrict__ excl, int32_t* __restrict__ run_pos,
                          int32_t* __restrict__ run_col, int32_t* __restrict__ total) {
  const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (p >= nnz) return;
  if (flag[p]) {
    const int64_t k = excl[p];
    const int64_t c = decode_col(col[p]);
    run_pos[k] = static_cast<int32_t>(p);
    run_col[k] = (c >= 0 && c < K) ? static_cast<int32_t>(c) : -1;
  }
  if (p == nnz - 1) *total = excl[p] + flag[p];
}

// Window w -> its first run: the number of runs that start before rowptr[w].
template <typename I>
__global__ void cube_window_ptr(const I* __restrict__ rowptr, int64_t windows, int64_t nnz,
                                const int32_t* __restrict__ excl, const int32_t* __restrict__ total,
                                int32_t* __restrict__ crow) {
  const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (w > windows) return;
  const int64_t a = clamp_pos(rowptr, w, nnz);
  crow[w] = a < nnz ? excl[a] : (nnz > 0 ? *total : 0);
}

// Run k writes its 16 block values: value of the run's last nonzero with row
// r, zero for rows without one.
template <typename T, typename I>
__global__ void cube_run_values(const I* __restrict__ col, const T* __restrict__ value, int64_t nnz,
                                const int32_t* __restrict__ run_pos, const int32_t* __restrict__ total,
                                T* __restrict__ block_value) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t runs = *total;
  if (k >= runs) return;
  const int64_t p0 = run_pos[k];
  const int64_t p1 = k + 1 < runs ? run_pos[k + 1] : nnz;
  T v[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) v[r] = static_cast<T>(0.f);
  for (int64_t p = p0; p < p1; ++p) {
    const int r = static_cast<int>(static_cast<int64_t>(col[p]) & 15);
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) v[rr] = rr == r ? value[p] : v[rr];
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) block_value[16 * k + r] = v[r];
}

// Workspace of one call ("decode" arrays, rocPRIM scan scratch, then the
// workspace of the mixed operator with an empty vector part).
struct CubeLayout {
  size_t flag = 0, excl = 0, run_pos = 0, run_col = 0, crow = 0, total = 0, value = 0, scan = 0, mixed = 0;
  size_t total_bytes = 0;
  spmm_mixed_desc md{};
  CubeLayout(const spmm_cube_op_desc* d) {
    const int64_t nnz = d->nnz > 0 ? d->nnz : 0;
    const int64_t w = d->windows > 0 ? d->windows : 0;
    const size_t vs = d->value_type == SPMM_VALUE_F16 ? 2 : 4;
    size_t off = 0;
    auto take = [&](size_t bytes) {
      const size_t at = off;
      off = align_up(off + (bytes > 0 ? bytes : 1), 256);
      return at;
    };
    flag = take(sizeof(int32_t) * nnz);
    excl = take(sizeof(int32_t) * nnz);
    run_pos = take(sizeof(int32_t) * nnz);
    run_col = take(sizeof(int32_t) * nnz);
    crow = take(sizeof(int32_t) * (w + 1));
    total = take(sizeof(int32_t));
    value = take(16 * vs * nnz);
    size_t scan_bytes = 0;
    (void)rocprim::exclusive_scan(nullptr, scan_bytes, static_cast<const int32_t*>(nullptr),
                                  static_cast<int32_t*>(nullptr), int32_t(0), static_cast<size_t>(nnz > 0 ? nnz : 1),
                                  rocprim::plus<int32_t>());
    scan = take(scan_bytes);
    md.block_windows = w;
    md.block_count = nnz;
    md.block_values = 16 * nnz;
    md.vector_rows = 0;
    md.vector_nnz = 0;
    md.dense_rows = d->dense_rows;
    md.width = d->width;
    md.index_type = SPMM_INDEX_I32;
    md.value_type = d->value_type;
    size_t mixed_bytes = 0;
    spmm_mixed_workspace(&md, &mixed_bytes);
    mixed = take(mixed_bytes);
    total_bytes = off;
  }
};

template <typename T, typename I>
spmm_status cube_typed(const spmm_cube_op_desc* d, const void* rowptr_v, const void* col_v, const void* value_v,
                       const void* dense, void* out, char* ws, const CubeLayout& lay, hipStream_t stream) {
  const I* rowptr = static_cast<const I*>(rowptr_v);
  const I* col = static_cast<const I*>(col_v);
  const T* value = static_cast<const T*>(value_v);
  const int64_t nnz = d->nnz, W = d->windows;
  int32_t* flag = reinterpret_cast<int32_t*>(ws + lay.flag);
  int32_t* excl = reinterpret_cast<int32_t*>(ws + lay.excl);
  int32_t* run_pos = reinterpret_cast<int32_t*>(ws + lay.run_pos);
  int32_t* run_col = reinterpret_cast<int32_t*>(ws + lay.run_col);
  int32_t* crow = reinterpret_cast<int32_t*>(ws + lay.crow);
  int32_t* total = reinterpret_cast<int32_t*>(ws + lay.total);
  T* block_value = reinterpret_cast<T*>(ws + lay.value);
  const unsigned pos_blocks = static_cast<unsigned>(ceil_div(nnz > 0 ? nnz : 1, kThreads));
  if (nnz > 0) {
    hipLaunchKernelGGL(cube_clear, dim3(pos_blocks), dim3(kThreads), 0, stream, flag, nnz);
    if (W > 0)
      hipLaunchKernelGGL((cube_window_marks<I>), dim3(static_cast<unsigned>(ceil_div(W, kThreads))),
                         dim3(kThreads), 0, stream, rowptr, W, nnz, flag);
    hipLaunchKernelGGL((cube_run_flags<I>), dim3(pos_blocks), dim3(kThreads), 0, stream, col, nnz, flag);
    if (spmm_status st = check_launch("spmm_cube decode")) return st;
    size_t scan_bytes = 0;
    (void)rocprim::exclusive_scan(nullptr, scan_bytes, flag, excl, int32_t(0), static_cast<size_t>(nnz),
                                  rocprim::plus<int32_t>());
    if (spmm_status st = check_hip(rocprim::exclusive_scan(ws + lay.scan, scan_bytes, flag, excl, int32_t(0),
                                                           static_cast<size_t>(nnz), rocprim::plus<int32_t>(),
                                                           stream),
                                   "spmm_cube scan"))
      return st;
    hipLaunchKernelGGL((cube_runs<I>), dim3(pos_blocks), dim3(kThreads), 0, stream, col, nnz, d->dense_rows,
                       flag, excl, run_pos, run_col, total);
  }
  hipLaunchKernelGGL((cube_window_ptr<I>), dim3(static_cast<unsigned>(ceil_div(W + 1, kThreads))), dim3(kThreads),
                     0, stream, rowptr, W, nnz, excl, total, crow);
  if (nnz > 0)
    hipLaunchKernelGGL((cube_run_values<T, I>), dim3(pos_blocks), dim3(kThreads), 0, stream, col, value, nnz,
                       run_pos, total, block_value);
  if (spmm_status st = check_launch("spmm_cube decode")) return st;
  // Block part on the decoded windows (no vector part: the block kernel
  // writes zeros to the rows of windows without blocks).
  return spmm_mixed_run(&lay.md, crow, run_col, block_value, crow, run_col, block_value, dense, out,
                        ws + lay.mixed, lay.total_bytes - lay.mixed, reinterpret_cast<spmm_stream>(stream));
}

}  // namespace
}  // namespace spmm

using namespace spmm;

extern "C" {

spmm_status spmm_cube_op_workspace(const spmm_cube_op_desc* d, size_t* bytes) {
  clear_error();
  if (d == nullptr || bytes == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "null argument");
  *bytes = CubeLayout(d).total_bytes;
  return SPMM_OK;
}

spmm_status spmm_cube_op_run(const spmm_cube_op_desc* d, const void* rowptr, const void* col, const void* value,
                             const void* dense, void* out, void* workspace, size_t workspace_bytes,
                             spmm_stream stream) {
  clear_error();
  if (d == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "null descriptor");
  if (d->index_type != SPMM_INDEX_I32 && d->index_type != SPMM_INDEX_I64)
    return fail(SPMM_ERR_CONTRACT, "spmm_cube: index arrays must be int32 or int64");
  if (d->value_type != SPMM_VALUE_F16 && d->value_type != SPMM_VALUE_F32)
    return fail(SPMM_ERR_CONTRACT, "spmm_cube supports only FP16 and FP32 dense tensors");
  // Feature-width contract of check_dense_contract(dense, 16, "spmm_cube")
  // (extension/custom_op.cpp:39-57, 102).
  const bool half = d->value_type == SPMM_VALUE_F16;
  const int64_t max_width = half ? 1024 : 512;
  if (d->width <= 0 || d->width > max_width)
    return fail(SPMM_ERR_CONTRACT, "spmm_cube requires 0 < feature width <= " + std::to_string(max_width) +
                                       " for " + (half ? "FP16" : "FP32") + ", but got " + std::to_string(d->width));
  if (d->width % 16 != 0)
    return fail(SPMM_ERR_CONTRACT, "spmm_cube requires feature width divisible by 16, but got " +
                                       std::to_string(d->width) +
                                       ". Pad and crop the dense tensor or use a safe PyTorch fallback.");
  if (d->windows < 0 || d->nnz < 0 || d->dense_rows < 0)
    return fail(SPMM_ERR_CONTRACT, "spmm_cube: negative extent");
  if ((reinterpret_cast<uintptr_t>(dense) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return fail(SPMM_ERR_CONTRACT, "spmm_cube: dense and out must be 16-byte aligned");
  if (d->nnz >= INT32_MAX) return fail(SPMM_ERR_CONTRACT, "spmm_cube: at most 2^31 - 2 nonzeros");
  if (d->windows == 0) return SPMM_OK;
  if (rowptr == nullptr || out == nullptr || (d->nnz > 0 && (col == nullptr || value == nullptr)) ||
      (d->dense_rows > 0 && dense == nullptr))
    return fail(SPMM_ERR_INVALID_ARGUMENT, "spmm_cube: null device pointer");
  const CubeLayout lay(d);
  if (workspace == nullptr || workspace_bytes < lay.total_bytes)
    return fail(SPMM_ERR_CONTRACT, "spmm_cube: workspace too small: need " + std::to_string(lay.total_bytes) +
                                       " bytes");
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = as_stream(stream);
  if (d->value_type == SPMM_VALUE_F16) {
    if (d->index_type == SPMM_INDEX_I32)
      return cube_typed<_Float16, int32_t>(d, rowptr, col, value, dense, out, ws, lay, s);
    return cube_typed<_Float16, int64_t>(d, rowptr, col, value, dense, out, ws, lay, s);
  }
  if (d->index_type == SPMM_INDEX_I32) return cube_typed<float, int32_t>(d, rowptr, col, value, dense, out, ws, lay, s);
  return cube_typed<float, int64_t>(d, rowptr, col, value, dense, out, ws, lay, s);
}

}  // extern "C"
