// Block (BCSR 16x1) part of the mixed SpMM (the reference's AIC/cube branch).
//
// Semantics follow KernelMmad (kernels/op_kernel/spmm_ascend_cube.cpp:16-311):
//   out[16*s + r, :] = sum_{b in [Crowptr[s], Crowptr[s+1])} Cvalue[16*b + r] * dense[Ccol[b], :]
// The reference walks 96-block tiles per window on the cube unit and adds
// partial windows atomically.  Here one work-group owns one 16-row window
// (owner-computes, no atomics):
//
//  * MFMA: the window tile is A (16 x K, K = the window's blocks) and the
//    gathered dense rows are B (K x N).  fp16 uses v_mfma_f32_16x16x32_f16
//    (K-step 32 blocks), fp32 uses v_mfma_f32_16x16x4_f32 (K-step 4 blocks).
//  * Dense gather without an LDS transpose: lane (q = lane % 16, kg = lane / 16)
//    loads, for each of its K-step blocks, 4 consecutive columns
//    n0 + 4q .. n0 + 4q + 3 of the block's dense row (one 8-byte load for
//    fp16, 16 bytes for fp32; 16 lanes read 128/256 contiguous bytes).  MFMA j
//    (j = 0..3) takes element j of each load, so its B column q is the dense
//    column n0 + 4q + j.  Four MFMAs therefore cover a 64-column group and
//    the accumulator lane holds 4 consecutive output columns.
//  * The A fragment A[r][k] = Cvalue[16*(b0+k) + r] is read straight from the
//    [block][row] layout the reference's converters produce.
//  * Waves of the work-group take 64-column groups round-robin; each group
//    runs the whole K loop, so every output element sees the same MFMA
//    sequence for every width N.
//  * The fp32 window tile goes to LDS; the work-group then adds the vector
//    (CSR) nonzeros of the window's rows in order (shared-window residuals of
//    preprocess and the CSR part of block_level_split), rounds once and
//    stores coalesced rows.
//  * blockIdx -> window is XCD-aware: consecutive windows land on the same XCD
//    (work-groups are dealt round-robin over the 8 XCDs), so neighbouring
//    windows that gather the same dense rows share that XCD's L2.
#include "common.h"
#include "lanevec.h"

namespace spmm {
namespace {

using lanes::LaneVec;
using lanes::accumulate;
using lanes::clampi;

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kXcds = 8;

template <typename I>
__device__ inline void window_group_f16(float* __restrict__ tile, const I* __restrict__ Ccol,
                                        const _Float16* __restrict__ Cvalue, int64_t b0,
                                        int64_t b1, const _Float16* __restrict__ dense,
                                        int64_t K, int64_t N, int64_t n0, int lane) {
  const int q = lane & 15, kg = lane >> 4;
  const bool col_ok = (n0 + 4 * q) < N;
  float4_t acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = b0; k0 < b1; k0 += 32) {
    half8_t a;
    half4_t rows[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t blk = k0 + 8 * kg + e;
      const bool in = blk < b1;
      a[e] = in ? Cvalue[blk * 16 + q] : static_cast<_Float16>(0.f);
      const int64_t c = in ? static_cast<int64_t>(Ccol[blk]) : -1;
      if (col_ok && static_cast<uint64_t>(c) < static_cast<uint64_t>(K))
        rows[e] = *reinterpret_cast<const half4_t*>(dense + c * N + n0 + 4 * q);
      else
        rows[e] = half4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half8_t b;
#pragma unroll
      for (int e = 0; e < 8; ++e) b[e] = rows[e][j];
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[j], 0, 0, 0);
    }
  }
  if (col_ok) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float4_t v = float4_t{acc[0][e], acc[1][e], acc[2][e], acc[3][e]};
      *reinterpret_cast<float4_t*>(tile + (4 * kg + e) * N + n0 + 4 * q) = v;
    }
  }
}

template <typename I>
__device__ inline void window_group_f32(float* __restrict__ tile, const I* __restrict__ Ccol,
                                        const float* __restrict__ Cvalue, int64_t b0,
                                        int64_t b1, const float* __restrict__ dense, int64_t K,
                                        int64_t N, int64_t n0, int lane) {
  const int q = lane & 15, kg = lane >> 4;
  const bool col_ok = (n0 + 4 * q) < N;
  float4_t acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = b0; k0 < b1; k0 += 16) {
    float a[4];
    float4_t bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t blk = k0 + 4 * u + kg;
      const bool in = blk < b1;
      a[u] = in ? Cvalue[blk * 16 + q] : 0.f;
      const int64_t c = in ? static_cast<int64_t>(Ccol[blk]) : -1;
      if (col_ok && static_cast<uint64_t>(c) < static_cast<uint64_t>(K))
        bv[u] = *reinterpret_cast<const float4_t*>(dense + c * N + n0 + 4 * q);
      else
        bv[u] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], bv[u][j], acc[j], 0, 0, 0);
    }
  }
  if (col_ok) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float4_t v = float4_t{acc[0][e], acc[1][e], acc[2][e], acc[3][e]};
      *reinterpret_cast<float4_t*>(tile + (4 * kg + e) * N + n0 + 4 * q) = v;
    }
  }
}

template <typename T, typename I>
__global__ __launch_bounds__(256) void block_windows(
    const I* __restrict__ Crowptr, const I* __restrict__ Ccol, const T* __restrict__ Cvalue,
    int64_t windows, int64_t block_limit, const I* __restrict__ Vrowptr,
    const I* __restrict__ Vcol, const T* __restrict__ Vvalue, int64_t vector_rows,
    int64_t vector_nnz, const T* __restrict__ dense, int64_t K, int64_t N, T* __restrict__ out,
    int64_t per_xcd) {
  extern __shared__ float tile[];  // [16][N] fp32
  const int64_t s = static_cast<int64_t>(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  if (s >= windows) return;  // uniform over the work-group

  const int64_t b0 = clampi(static_cast<int64_t>(Crowptr[s]), 0, block_limit);
  const int64_t b1 = clampi(static_cast<int64_t>(Crowptr[s + 1]), b0, block_limit);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int64_t groups = (N + 63) / 64;
  for (int64_t g = wave; g < groups; g += waves) {
    if constexpr (sizeof(T) == 2)
      window_group_f16<I>(tile, Ccol, Cvalue, b0, b1, dense, K, N, 64 * g, lane);
    else
      window_group_f32<I>(tile, Ccol, Cvalue, b0, b1, dense, K, N, 64 * g, lane);
  }
  __syncthreads();

  constexpr int V = LaneVec<T>::V;
  const int64_t chunks = N / V;
  for (int64_t it = threadIdx.x; it < 16 * chunks; it += blockDim.x) {
    const int64_t r = it / chunks;
    const int64_t c0 = (it - r * chunks) * V;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = tile[r * N + c0 + i];
    const int64_t row = 16 * s + r;
    if (row < vector_rows) {
      const int64_t a = clampi(static_cast<int64_t>(Vrowptr[row]), 0, vector_nnz);
      const int64_t b = clampi(static_cast<int64_t>(Vrowptr[row + 1]), 0, vector_nnz);
      accumulate<T, I>(acc, a, b, Vcol, Vvalue, dense, K, N, c0);
    }
    LaneVec<T>::store(out + row * N + c0, acc);
  }
}

template <typename T, typename I>
spmm_status block_typed(const void* Crowptr, const void* Ccol, const void* Cvalue,
                        int64_t windows, int64_t block_count, int64_t block_values,
                        const void* Vrowptr, const void* Vcol, const void* Vvalue,
                        int64_t vector_rows, int64_t vector_nnz, const void* dense, int64_t K,
                        int64_t N, void* out, hipStream_t stream) {
  if (windows <= 0) return SPMM_OK;
  const int64_t limit = block_count < block_values / 16 ? block_count : block_values / 16;
  const int64_t groups = (N + 63) / 64;
  const int waves = groups < 4 ? static_cast<int>(groups) : 4;
  const int64_t per_xcd = ceil_div(windows, kXcds);
  const int64_t grid = per_xcd * kXcds;
  const size_t lds = static_cast<size_t>(16) * N * sizeof(float);
  hipLaunchKernelGGL((block_windows<T, I>), dim3(static_cast<unsigned>(grid)), dim3(64 * waves),
                     lds, stream, static_cast<const I*>(Crowptr), static_cast<const I*>(Ccol),
                     static_cast<const T*>(Cvalue), windows, limit < 0 ? 0 : limit,
                     static_cast<const I*>(Vrowptr), static_cast<const I*>(Vcol),
                     static_cast<const T*>(Vvalue), vector_rows, vector_nnz,
                     static_cast<const T*>(dense), K, N, static_cast<T*>(out), per_xcd);
  return check_launch("block_windows");
}

}  // namespace

spmm_status launch_block(int32_t index_type, int32_t value_type, const void* Crowptr,
                         const void* Ccol, const void* Cvalue, int64_t windows,
                         int64_t block_count, int64_t block_values, const void* Vrowptr,
                         const void* Vcol, const void* Vvalue, int64_t vector_rows,
                         int64_t vector_nnz, const void* dense, int64_t dense_rows,
                         int64_t width, void* out, hipStream_t stream) {
#define SPMM_BLOCK_CALL(T, I)                                                                 \
  return block_typed<T, I>(Crowptr, Ccol, Cvalue, windows, block_count, block_values, Vrowptr, \
                           Vcol, Vvalue, vector_rows, vector_nnz, dense, dense_rows, width, out, \
                           stream)
  if (value_type == SPMM_VALUE_F16) {
    if (index_type == SPMM_INDEX_I32) SPMM_BLOCK_CALL(_Float16, int32_t);
    SPMM_BLOCK_CALL(_Float16, int64_t);
  }
  if (index_type == SPMM_INDEX_I32) SPMM_BLOCK_CALL(float, int32_t);
  SPMM_BLOCK_CALL(float, int64_t);
#undef SPMM_BLOCK_CALL
}

}  // namespace spmm
