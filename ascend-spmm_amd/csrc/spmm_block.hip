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
//  * Windows longer than a fixed chunk (block_chunk: 512 blocks fp16, 256
//    fp32) are cut at fixed block positions: the window's own work-group
//    takes its first chunk, and "overflow" work-groups take the rest in fixed
//    global block ranges (only one window can overflow into a range).  A
//    combine kernel adds the pieces in order, so the split is deterministic.
//  * Vector (CSR) nonzeros of rows inside block windows are summed by the CSR
//    gather kernel first (so long rows get its load balance) and left in an
//    fp32 workspace; the block kernel adds them after the block sum and
//    rounds once.
//  * blockIdx -> window is XCD-aware: consecutive windows land on the same XCD
//    (work-groups are dealt round-robin over the 8 XCDs), so neighbouring
//    windows that gather the same dense rows share that XCD's L2.
#include "common.h"
#include "lanevec.h"
#include "wgsearch.h"

namespace spmm {
namespace {

using lanes::LaneVec;
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

// Arguments shared by the block kernels.
template <typename T, typename I>
struct BlockArgs {
  const I* Crowptr;
  const I* Ccol;
  const T* Cvalue;
  int64_t windows, limit;  // block windows; usable blocks = min(Ccol, Cvalue/16)
  const I* Vrowptr;
  int64_t vrows, vnnz;     // vector part: rows and nonzeros
  const T* dense;
  int64_t K, N;
  T* out;
  const float* vpart;      // [16*windows][N] fp32 vector sums of block-window rows (gather pass)
  float* slots;            // [noverflow][2][16][N] fp32 partials of windows longer than kbig
  int64_t kbig, noverflow, per_xcd;

  __device__ inline int64_t crp(int64_t s) const { return clampi(static_cast<int64_t>(Crowptr[s]), 0, limit); }
  __device__ inline int64_t vrp(int64_t r) const {
    return clampi(static_cast<int64_t>(Vrowptr[r < vrows ? r : vrows]), 0, vnnz);
  }
  // Row r has vector-part nonzeros (then the gather pass left their sum in vpart).
  __device__ inline bool row_has_vector(int64_t r) const { return r < vrows && vrp(r) != vrp(r + 1); }
};

// Fills the LDS tile with the MFMA sum of blocks [b0, b1) of window s.
template <typename T, typename I>
__device__ inline void window_tile(const BlockArgs<T, I>& a, float* tile, int64_t b0, int64_t b1) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int64_t groups = (a.N + 63) / 64;
  for (int64_t g = wave; g < groups; g += waves) {
    if constexpr (sizeof(T) == 2)
      window_group_f16<I>(tile, a.Ccol, a.Cvalue, b0, b1, a.dense, a.K, a.N, 64 * g, lane);
    else
      window_group_f32<I>(tile, a.Ccol, a.Cvalue, b0, b1, a.dense, a.K, a.N, 64 * g, lane);
  }
}

// Finishes window s from its fp32 block sum (LDS tile or `src`): adds the
// vector sums of rows that have them (block first, then vector part), rounds
// once and writes rows 16*s .. 16*s+15.
template <typename T, typename I>
__device__ inline void finish_window(const BlockArgs<T, I>& a, int64_t s, const float* src) {
  constexpr int V = LaneVec<T>::V;
  __shared__ unsigned s_vec;  // bit r: row 16*s + r has vector nonzeros
  if (threadIdx.x == 0) s_vec = 0;
  __syncthreads();
  if (threadIdx.x < 16 && a.row_has_vector(16 * s + threadIdx.x)) atomicOr(&s_vec, 1u << threadIdx.x);
  __syncthreads();
  const unsigned vec = s_vec;
  const int64_t chunks = a.N / V;
  for (int64_t it = threadIdx.x; it < 16 * chunks; it += blockDim.x) {
    const int64_t r = it / chunks;
    const int64_t c0 = (it - r * chunks) * V;
    const int64_t row = 16 * s + r;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = src[r * a.N + c0 + i];
    if (vec >> r & 1u) {
      const float* vp = a.vpart + row * a.N + c0;
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = acc[i] + vp[i];
    }
    LaneVec<T>::store(a.out + row * a.N + c0, acc);
  }
}

// Copies the 16 x N fp32 tile to a workspace slot.
__device__ inline void save_tile(const float* tile, int64_t N, float* dst) {
  for (int64_t i = threadIdx.x; i < 16 * N; i += blockDim.x) dst[i] = tile[i];
}

// Work-groups [0, 8*per_xcd): window s (XCD-aware order) computes its first
// kbig blocks; a window with at most kbig blocks is finished here.  A longer
// window leaves its first-chunk sum in slot (k0, 1), k0 = (b0 + kbig) / kbig.
// Work-groups 8*per_xcd + k: overflow range k = blocks [k*kbig, (k+1)*kbig).
// Only the window holding block k*kbig can have blocks past its first chunk
// in that range; that segment's sum goes to slot (k, 0).
template <typename T, typename I>
__global__ __launch_bounds__(256) void block_windows(BlockArgs<T, I> a) {
  extern __shared__ float tile[];  // [16][N] fp32
  const int64_t lead = a.per_xcd * kXcds;
  const int64_t g = blockIdx.x;
  if (g < lead) {
    const int64_t s = (g % kXcds) * a.per_xcd + g / kXcds;
    if (s >= a.windows) return;  // uniform over the work-group
    const int64_t b0 = a.crp(s);
    int64_t b1 = a.crp(s + 1);
    if (b1 <= b0) return;  // empty window: rows handled by the vector pass
    const bool single = b1 - b0 <= a.kbig;
    if (!single) b1 = b0 + a.kbig;
    window_tile(a, tile, b0, b1);
    __syncthreads();
    if (single)
      finish_window(a, s, tile);
    else
      save_tile(tile, a.N, a.slots + (2 * ((b0 + a.kbig) / a.kbig) + 1) * 16 * a.N);
    return;
  }
  const int64_t k = g - lead;
  if (k >= a.noverflow) return;
  const int64_t bk = k * a.kbig;
  // s = window holding block bk: last s with crp(s) <= bk.
  int64_t first_above, unused;
  wg_lower_bound2([&](int64_t i) { return a.crp(i); }, 0, a.windows, bk + 1, bk + 1, first_above, unused);
  const int64_t s = first_above - 1;
  if (s < 0 || s >= a.windows) return;
  const int64_t b0 = a.crp(s), b1 = a.crp(s + 1);
  if (!(b0 < bk && b1 > b0 + a.kbig)) return;
  const int64_t lo = b0 + a.kbig > bk ? b0 + a.kbig : bk;
  const int64_t hi = b1 < bk + a.kbig ? b1 : bk + a.kbig;
  if (lo >= hi) return;
  window_tile(a, tile, lo, hi);
  __syncthreads();
  save_tile(tile, a.N, a.slots + (2 * k) * 16 * a.N);
}

// Work-group k: if a window's blocks past its first chunk start in overflow
// range k, add first chunk + segments k, k+1, ... in order (into LDS) and
// finish the window.
template <typename T, typename I>
__global__ __launch_bounds__(256) void block_combine(BlockArgs<T, I> a) {
  extern __shared__ float tile[];  // [16][N] fp32
  const int64_t k = blockIdx.x;
  const int64_t bk = k * a.kbig;
  int64_t first_above, unused;
  wg_lower_bound2([&](int64_t i) { return a.crp(i); }, 0, a.windows, bk + 1, bk + 1, first_above, unused);
  const int64_t s = first_above - 1;
  if (s < 0 || s >= a.windows) return;
  const int64_t b0 = a.crp(s), b1 = a.crp(s + 1);
  if (!(b1 - b0 > a.kbig && (b0 + a.kbig) / a.kbig == k)) return;
  const int64_t k_end = (b1 - 1) / a.kbig;
  const int64_t n = 16 * a.N;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    float acc = a.slots[(2 * k + 1) * n + i];
    for (int64_t kk = k; kk <= k_end; ++kk) acc = acc + a.slots[(2 * kk) * n + i];
    tile[i] = acc;
  }
  __syncthreads();
  finish_window(a, s, tile);
}

template <typename T, typename I>
spmm_status block_typed(const void* Crowptr, const void* Ccol, const void* Cvalue, int64_t windows,
                        int64_t block_count, int64_t block_values, const void* Vrowptr,
                        int64_t vector_rows, int64_t vector_nnz, const void* dense, int64_t K,
                        int64_t N, void* out, const float* vpart, float* slots, hipStream_t stream) {
  if (windows <= 0) return SPMM_OK;
  BlockArgs<T, I> a;
  a.Crowptr = static_cast<const I*>(Crowptr);
  a.Ccol = static_cast<const I*>(Ccol);
  a.Cvalue = static_cast<const T*>(Cvalue);
  a.windows = windows;
  const int64_t limit = block_count < block_values / 16 ? block_count : block_values / 16;
  a.limit = limit < 0 ? 0 : limit;
  a.Vrowptr = static_cast<const I*>(Vrowptr);
  a.vrows = vector_rows;
  a.vnnz = vector_nnz;
  a.dense = static_cast<const T*>(dense);
  a.K = K;
  a.N = N;
  a.out = static_cast<T*>(out);
  a.vpart = vpart;
  a.slots = slots;
  a.kbig = block_chunk<T>();
  a.noverflow = block_overflow_ranges(a.limit, a.kbig);
  a.per_xcd = ceil_div(windows, kXcds);
  const int64_t groups = (N + 63) / 64;
  const int waves = groups < 4 ? static_cast<int>(groups) : 4;
  const size_t lds = static_cast<size_t>(16) * N * sizeof(float);
  const int64_t grid = a.per_xcd * kXcds + a.noverflow;
  hipLaunchKernelGGL((block_windows<T, I>), dim3(static_cast<unsigned>(grid)), dim3(64 * waves), lds,
                     stream, a);
  if (spmm_status st = check_launch("block_windows")) return st;
  if (a.noverflow == 0) return SPMM_OK;
  hipLaunchKernelGGL((block_combine<T, I>), dim3(static_cast<unsigned>(a.noverflow)), dim3(256), lds, stream,
                     a);
  return check_launch("block_combine");
}

}  // namespace

int64_t block_overflow_ranges(int64_t blocks, int64_t kbig) {
  return blocks > kbig ? ceil_div(blocks, kbig) : 0;
}

spmm_status launch_block(int32_t index_type, int32_t value_type, const void* Crowptr,
                         const void* Ccol, const void* Cvalue, int64_t windows,
                         int64_t block_count, int64_t block_values, const void* Vrowptr,
                         int64_t vector_rows, int64_t vector_nnz, const void* dense,
                         int64_t dense_rows, int64_t width, void* out, const float* vpart,
                         float* slots, hipStream_t stream) {
#define SPMM_BLOCK_CALL(T, I)                                                                   \
  return block_typed<T, I>(Crowptr, Ccol, Cvalue, windows, block_count, block_values, Vrowptr, \
                           vector_rows, vector_nnz, dense, dense_rows, width, out, vpart, slots, \
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
