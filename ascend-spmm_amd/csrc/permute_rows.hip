// Row permutation of node tensors: the P / P^T applications of the graph
// layout (pack_node_tensor / restore_node_tensor, spmm_npu.py:23-62).
//
// Both directions run as one row gather dst[r, :] = src[map[r], :] with
// map[r] < 0 meaning "zero row".  Restore uses inv_permutation directly as the
// map.  Pack needs the opposite direction (packed row -> original row): it is
// built in the workspace by a fill and an atomicMax scatter (the largest
// original id wins if inv repeats a packed row, matching a sequential
// index_copy_ that lets the last write stand), so padding rows are written as
// zeros by the gather itself and the packed tensor needs no separate clear.
// One wavefront copies one row with 16-byte lane accesses where the row size
// and pointers allow it.
#include "common.h"

namespace spmm {
namespace {

typedef unsigned int uint4_t __attribute__((ext_vector_type(4)));

template <typename U>
__global__ __launch_bounds__(256) void gather_rows(const char* __restrict__ src,
                                                   int64_t src_rows, char* __restrict__ dst,
                                                   int64_t dst_rows, int64_t units,
                                                   const int64_t* __restrict__ map) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 6);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
       r < dst_rows; r += waves) {
    const int64_t s = map[r];
    U* d = reinterpret_cast<U*>(dst) + r * units;
    if (s >= 0 && s < src_rows) {
      const U* sp = reinterpret_cast<const U*>(src) + s * units;
      for (int64_t u = lane; u < units; u += 64) __builtin_nontemporal_store(sp[u], d + u);
    } else {
      U z;
      __builtin_memset(&z, 0, sizeof(U));
      for (int64_t u = lane; u < units; u += 64) __builtin_nontemporal_store(z, d + u);
    }
  }
}

__global__ void fill_minus_one(int64_t* __restrict__ p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = -1;
}

__global__ void scatter_inverse(const int64_t* __restrict__ inv, int64_t rows,
                                int64_t* __restrict__ perm, int64_t packed_rows) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t p = inv[i];
    if (p >= 0 && p < packed_rows)
      atomicMax(reinterpret_cast<long long*>(perm + p), static_cast<long long>(i));
  }
}

spmm_status launch_gather_rows(const void* src, int64_t src_rows, void* dst, int64_t dst_rows,
                               int64_t row_bytes, const int64_t* map, hipStream_t stream) {
  if (dst_rows <= 0 || row_bytes <= 0) return SPMM_OK;
  const uintptr_t align = reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst);
  const int64_t waves_per_block = 4;
  int64_t blocks = ceil_div(dst_rows, waves_per_block);
  if (blocks > 65536) blocks = 65536;
  if (row_bytes % 16 == 0 && align % 16 == 0) {
    hipLaunchKernelGGL(gather_rows<uint4_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, static_cast<const char*>(src), src_rows, static_cast<char*>(dst),
                       dst_rows, row_bytes / 16, map);
  } else if (row_bytes % 4 == 0 && align % 4 == 0) {
    hipLaunchKernelGGL(gather_rows<uint32_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, static_cast<const char*>(src), src_rows, static_cast<char*>(dst),
                       dst_rows, row_bytes / 4, map);
  } else {
    hipLaunchKernelGGL(gather_rows<uint8_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       stream, static_cast<const char*>(src), src_rows, static_cast<char*>(dst),
                       dst_rows, row_bytes, map);
  }
  return check_launch("gather_rows");
}

}  // namespace
}  // namespace spmm

using namespace spmm;

extern "C" {

size_t spmm_pack_workspace(int64_t packed_rows) {
  return static_cast<size_t>(packed_rows < 0 ? 0 : packed_rows) * sizeof(int64_t);
}

spmm_status spmm_pack_rows(const void* src, int64_t rows, int64_t row_bytes, const int64_t* inv,
                           void* packed, int64_t packed_rows, void* workspace,
                           size_t workspace_bytes, spmm_stream stream) {
  clear_error();
  if (rows < 0 || packed_rows < 0 || row_bytes < 0)
    return fail(SPMM_ERR_INVALID_ARGUMENT, "pack_node_tensor: negative extent");
  if (packed_rows == 0) return SPMM_OK;
  if (workspace == nullptr || workspace_bytes < spmm_pack_workspace(packed_rows))
    return fail(SPMM_ERR_CONTRACT, "pack_node_tensor: workspace too small");
  if (packed == nullptr || (rows > 0 && (src == nullptr || inv == nullptr)))
    return fail(SPMM_ERR_INVALID_ARGUMENT, "pack_node_tensor: null device pointer");
  hipStream_t s = as_stream(stream);
  int64_t* perm = static_cast<int64_t*>(workspace);
  const unsigned fb = static_cast<unsigned>(ceil_div(packed_rows, 256) > 4096 ? 4096 : ceil_div(packed_rows, 256));
  hipLaunchKernelGGL(fill_minus_one, dim3(fb), dim3(256), 0, s, perm, packed_rows);
  if (spmm_status st = check_launch("fill_minus_one")) return st;
  if (rows > 0) {
    const unsigned sb = static_cast<unsigned>(ceil_div(rows, 256) > 4096 ? 4096 : ceil_div(rows, 256));
    hipLaunchKernelGGL(scatter_inverse, dim3(sb), dim3(256), 0, s, inv, rows, perm, packed_rows);
    if (spmm_status st = check_launch("scatter_inverse")) return st;
  }
  return launch_gather_rows(src, rows, packed, packed_rows, row_bytes, perm, s);
}

spmm_status spmm_restore_rows(const void* packed, int64_t packed_rows, int64_t row_bytes,
                              const int64_t* inv, int64_t rows, void* dst, spmm_stream stream) {
  clear_error();
  if (rows < 0 || packed_rows < 0 || row_bytes < 0)
    return fail(SPMM_ERR_INVALID_ARGUMENT, "restore_node_tensor: negative extent");
  if (rows == 0) return SPMM_OK;
  if (dst == nullptr || inv == nullptr || (packed_rows > 0 && packed == nullptr))
    return fail(SPMM_ERR_INVALID_ARGUMENT, "restore_node_tensor: null device pointer");
  return launch_gather_rows(packed, packed_rows, dst, rows, row_bytes, inv, as_stream(stream));
}

}  // extern "C"
