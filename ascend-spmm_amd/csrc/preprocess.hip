// GPU preprocessing of the MI355X SpMM library: the reference's host-side
// layout converters and work partitioners rewritten as device pipelines whose
// integer outputs (and copied values) are bit-identical to the reference's.
//
//   csr_to_bcsr        ToBCSR              (extension/custom_op.cpp:594-746)
//   csr_to_ascend_cube your_logic_kernel   (extension/custom_op.cpp:429-592)
//   block_level_split  hybrid_split_impl   (extension/custom_op.cpp:1139-1348, 1390-1412)
//   preprocess         taskmapping         (extension/custom_op.cpp:749-1137), with
//                      the graph layout (packed_column_reindex.h, pack_fixed_layout
//                      :1350-1384) and the marginal bucket sort (boundary_bucket_sort.h)
//
// Shared stage ("window sort"): every nonzero gets the key (window, column)
// and is radix-sorted stably, so equal keys keep position order.  A run of
// equal keys is a block (a window's 16x1 column strip): the sorted order is
// window-major with ascending columns, each block's first element is its
// first-seen position and its run length is its occupancy.  Within a block the
// entries of one row are adjacent, so "last write wins" for duplicate
// coordinates is "skip an entry followed by one of the same row".
//
// The reference's host sorts and argmins become device sorts and reductions
// that reproduce its tie rules exactly: stable radix sorts with the
// tie-breaking id in the key or value order, double-precision costs computed
// with the same IEEE expressions, and first-minimum selection done with two
// atomic-min passes on the bit patterns of the (non-negative) doubles.
//
// Every pipeline runs in two calls: *_plan computes all intermediate arrays in
// the caller's workspace and reads the output sizes back (it synchronises the
// stream); *_fill writes the outputs into caller buffers of those sizes.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <string>

#include "common.h"

namespace spmm {
namespace pre {

constexpr int kT = 256;

enum ErrorBit : int {
  kBadRowptr = 1,     // row pointer not monotone / outside the nonzero arrays
  kBadColumn = 2,     // column id outside [0, ncols)
  kUnsortedRow = 4,   // a row's column ids are not ascending
  kBadOccupancy = 8,  // marginal block occupancy outside [1, window_size]
};

inline unsigned grid_for(int64_t n) {
  int64_t g = (n + kT - 1) / kT;
  if (g < 1) g = 1;
  if (g > 65535 * 16) g = 65535 * 16;
  return static_cast<unsigned>(g);
}

#define GRID_STRIDE(i, n)                                                                \
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (n); \
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)

// ---------------------------------------------------------------- workspace

// Bump allocator over the caller's workspace.  With base == nullptr it only
// adds up sizes (the *_workspace queries run the same allocation sequence).
struct Arena {
  char* base = nullptr;
  size_t used = 0;
  template <typename T>
  T* take(int64_t n) {
    const size_t bytes = align_up(static_cast<size_t>(n > 0 ? n : 1) * sizeof(T), 256);
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += bytes;
    return p;
  }
};

// Device-wide sort and scan (rocPRIM) with one shared temporary buffer sized
// for the largest call.
struct Prims {
  void* temp = nullptr;
  size_t temp_bytes = 0;
  hipStream_t stream = nullptr;

  static size_t temp_needed(int64_t n) {
    size_t a = 0, b = 0, c = 0;
    const size_t m = static_cast<size_t>(n > 0 ? n : 1);
    (void)rocprim::radix_sort_pairs(nullptr, a, static_cast<const uint64_t*>(nullptr),
                              static_cast<uint64_t*>(nullptr), static_cast<const int64_t*>(nullptr),
                              static_cast<int64_t*>(nullptr), m, 0, 64);
    (void)rocprim::exclusive_scan(nullptr, b, static_cast<const int64_t*>(nullptr),
                            static_cast<int64_t*>(nullptr), int64_t(0), m,
                            rocprim::plus<int64_t>());
    (void)rocprim::inclusive_scan(nullptr, c, static_cast<const int64_t*>(nullptr),
                            static_cast<int64_t*>(nullptr), m, rocprim::plus<int64_t>());
    size_t t = a > b ? a : b;
    return t > c ? t : c;
  }
  hipError_t sort_pairs(const uint64_t* kin, uint64_t* kout, const int64_t* vin, int64_t* vout,
                        int64_t n, int end_bit) {
    if (n <= 0) return hipSuccess;
    size_t bytes = temp_bytes;
    return rocprim::radix_sort_pairs(temp, bytes, kin, kout, vin, vout, static_cast<size_t>(n), 0,
                                     end_bit < 1 ? 1 : end_bit, stream);
  }
  hipError_t exclusive_sum(const int64_t* in, int64_t* out, int64_t n) {
    if (n <= 0) return hipSuccess;
    size_t bytes = temp_bytes;
    return rocprim::exclusive_scan(temp, bytes, in, out, int64_t(0), static_cast<size_t>(n),
                                   rocprim::plus<int64_t>(), stream);
  }
  hipError_t inclusive_sum(const int64_t* in, int64_t* out, int64_t n) {
    if (n <= 0) return hipSuccess;
    size_t bytes = temp_bytes;
    return rocprim::inclusive_scan(temp, bytes, in, out, static_cast<size_t>(n),
                                   rocprim::plus<int64_t>(), stream);
  }
};

// Most blocks the marginal window can hold: distinct columns of one window.
inline int64_t marginal_capacity(int64_t nb, int64_t ncols) {
  const int64_t m = nb < ncols ? nb : ncols;
  return m > 0 ? m : 1;
}

inline int bits_for(uint64_t max_value) {
  int b = 0;
  while (b < 64 && (max_value >> b) != 0) ++b;
  return b < 1 ? 1 : b;
}

// ------------------------------------------------------------ small kernels

template <typename T>
__global__ void fill_kernel(T* __restrict__ p, int64_t n, T v) {
  GRID_STRIDE(i, n) p[i] = v;
}

__global__ void fill_bytes(unsigned char* __restrict__ p, int64_t n) {
  GRID_STRIDE(i, n) p[i] = 0;
}

__global__ void fill_zero16(uint4* __restrict__ p, int64_t n) {
  GRID_STRIDE(i, n) p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// dst[i] = src[i] converted to the output index type.
template <typename O>
__global__ void convert_index(const int64_t* __restrict__ src, O* __restrict__ dst, int64_t n) {
  GRID_STRIDE(i, n) dst[i] = static_cast<O>(src[i]);
}

// dst[i] = src[idx[i]] converted (gather).
template <typename O>
__global__ void gather_index(const int64_t* __restrict__ src, const int64_t* __restrict__ idx,
                             O* __restrict__ dst, int64_t n) {
  GRID_STRIDE(i, n) dst[i] = static_cast<O>(src[idx[i]]);
}

// ----------------------------------------------------- stage A: validation

// Checks row pointer monotonicity and bounds.
template <typename I>
__global__ void check_rowptr(const I* __restrict__ rowptr, int64_t nrows, int64_t nnz,
                             int* __restrict__ err) {
  GRID_STRIDE(r, nrows) {
    const int64_t a = static_cast<int64_t>(rowptr[r]), b = static_cast<int64_t>(rowptr[r + 1]);
    if (a < 0 || b < a || b > nnz) atomicOr(err, kBadRowptr);
  }
}

// The scalars the host needs after validation, gathered for one read-back:
// rowptr[0], rowptr[rows] and the error bits.
template <typename I>
__global__ void collect_ends(const I* __restrict__ rowptr, int64_t rows, const int* __restrict__ err,
                             int64_t* __restrict__ scal) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    scal[0] = static_cast<int64_t>(rowptr[0]);
    scal[1] = static_cast<int64_t>(rowptr[rows]);
    scal[2] = *err;
  }
}

// The block count (last inclusive block id) and the error bits, for one read-back.
__global__ void collect_blocks(const int64_t* __restrict__ bid, int64_t n, const int* __restrict__ err,
                               int64_t* __restrict__ scal) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    scal[0] = n > 0 ? bid[n - 1] : 0;
    scal[1] = *err;
  }
}

// Expands rows: for element e (position p = p_begin + e) records its row and
// 64-bit column, checking column range and (optionally) ascending order.
// Element-parallel, so a row of any length costs the same per element: each
// work-group takes kExpandChunk consecutive positions, two of its threads
// bracket the chunk's rows with binary searches over the whole row pointer,
// and every thread then searches only that bracket (empty when the chunk lies
// inside one long row).  The row pointer was checked monotone beforehand.
constexpr int64_t kExpandChunk = 4 * kT;

template <typename I>
__device__ inline int64_t row_of_position(const I* __restrict__ rowptr, int64_t lo, int64_t hi, int64_t p) {
  // largest r in [lo, hi] with rowptr[r] <= p (rowptr[lo] <= p holds)
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo + 1) / 2;
    if (static_cast<int64_t>(rowptr[mid]) <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <typename I>
__global__ void expand_rows(const I* __restrict__ rowptr, const I* __restrict__ col, int64_t nrows,
                            int64_t ncols, int64_t p_begin, int64_t n, int64_t* __restrict__ row_of,
                            int64_t* __restrict__ col64, int check_sorted, int* __restrict__ err) {
  __shared__ int64_t bracket[2];
  const int64_t chunks = (n + kExpandChunk - 1) / kExpandChunk;
  for (int64_t k = blockIdx.x; k < chunks; k += gridDim.x) {
    const int64_t e0 = k * kExpandChunk;
    const int64_t e1 = e0 + kExpandChunk < n ? e0 + kExpandChunk : n;
    if (threadIdx.x < 2)
      bracket[threadIdx.x] = row_of_position(rowptr, 0, nrows - 1, p_begin + (threadIdx.x ? e1 - 1 : e0));
    __syncthreads();
    const int64_t r_lo = bracket[0], r_hi = bracket[1];
    int bad = 0;
    for (int64_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
      const int64_t p = p_begin + e;
      const int64_t r = row_of_position(rowptr, r_lo, r_hi, p);
      const int64_t c = static_cast<int64_t>(col[p]);
      row_of[e] = r;
      col64[e] = c;
      if (c < 0 || c >= ncols) bad |= kBadColumn;
      if (check_sorted && p > static_cast<int64_t>(rowptr[r]) && c < static_cast<int64_t>(col[p - 1]))
        bad |= kUnsortedRow;
    }
    if (bad) atomicOr(err, bad);
    __syncthreads();
  }
}

// ----------------------------------------------------- stage B: window sort

__global__ void window_keys(const int64_t* __restrict__ row_of, const int64_t* __restrict__ col64,
                            int64_t n, int64_t W, int64_t ncols, uint64_t* __restrict__ key,
                            int64_t* __restrict__ elem) {
  GRID_STRIDE(e, n) {
    key[e] = static_cast<uint64_t>(row_of[e] / W) * static_cast<uint64_t>(ncols) +
             static_cast<uint64_t>(col64[e]);
    elem[e] = e;
  }
}

__global__ void run_heads(const uint64_t* __restrict__ skey, int64_t n, int64_t* __restrict__ head) {
  GRID_STRIDE(i, n) head[i] = (i == 0 || skey[i] != skey[i - 1]) ? 1 : 0;
}

// Block table from the sorted keys: blk_key, first element, run start.
__global__ void block_table(const uint64_t* __restrict__ skey, const int64_t* __restrict__ selem,
                            const int64_t* __restrict__ bid, int64_t n,
                            uint64_t* __restrict__ blk_key, int64_t* __restrict__ blk_first,
                            int64_t* __restrict__ blk_start, int64_t* __restrict__ elem_block) {
  GRID_STRIDE(i, n) {
    const int64_t b = bid[i] - 1;
    elem_block[selem[i]] = b;
    if (i == 0 || skey[i] != skey[i - 1]) {
      blk_key[b] = skey[i];
      blk_first[b] = selem[i];
      blk_start[b] = i;
    }
  }
}

__global__ void block_counts(const int64_t* __restrict__ blk_start, int64_t nb, int64_t n,
                             int64_t* __restrict__ blk_cnt) {
  GRID_STRIDE(b, nb) blk_cnt[b] = (b + 1 < nb ? blk_start[b + 1] : n) - blk_start[b];
}

// win_start[w] = first block of window >= w (nb past the end), w in [0, nwin].
__global__ void window_starts(const uint64_t* __restrict__ blk_key, int64_t nb, int64_t ncols,
                              int64_t nwin, int64_t* __restrict__ win_start) {
  GRID_STRIDE(b, nb + 1) {
    const int64_t wprev = b > 0 ? static_cast<int64_t>(blk_key[b - 1] / ncols) : -1;
    const int64_t wcur = b < nb ? static_cast<int64_t>(blk_key[b] / ncols) : nwin;
    for (int64_t w = wprev + 1; w <= wcur; ++w) win_start[w] = b;
  }
}

// ------------------------------------------------------ value scatter

// Copies the value of sorted element i to dst[slot(i)] unless the next sorted
// element is the same block and row (then that one, later in position order,
// wins), i.e. the reference's "last write wins" for duplicate coordinates.
// slot(i) = out_block(b) * stride + (row - window*W) + column offset, where
// out_block(b) < 0 drops the element.
template <typename U>
__global__ void scatter_values(const int64_t* __restrict__ selem, const int64_t* __restrict__ bid,
                               const int64_t* __restrict__ row_of, int64_t n, int64_t W,
                               const int64_t* __restrict__ out_block, int64_t stride,
                               int64_t tile_mode, const int64_t* __restrict__ win_start,
                               const uint64_t* __restrict__ blk_key, int64_t ncols,
                               const U* __restrict__ val, int64_t p_begin, U* __restrict__ dst) {
  GRID_STRIDE(i, n) {
    const int64_t e = selem[i];
    const int64_t b = bid[i] - 1;
    const int64_t r = row_of[e];
    if (i + 1 < n && bid[i + 1] == bid[i] && row_of[selem[i + 1]] == r) continue;
    const int64_t w = r / W;
    const int64_t rr = r - w * W;
    int64_t slot;
    if (tile_mode) {  // 16x16 tiles: value[256*t + 16*row + c]
      const int64_t k = b - win_start[w];
      const int64_t t = out_block[w] + k / 16;
      slot = 256 * t + 16 * rr + (k % 16);
    } else {
      const int64_t ob = out_block ? out_block[b] : b;
      if (ob < 0) continue;
      slot = ob * stride + rr;
    }
    dst[slot] = val[p_begin + e];
  }
}

// ------------------------------------------------------------- ToBCSR

template <typename O>
__global__ void block_columns(const uint64_t* __restrict__ blk_key, const int64_t* __restrict__ out_block,
                              int64_t nb, int64_t ncols, O* __restrict__ dst) {
  GRID_STRIDE(b, nb) {
    const int64_t ob = out_block ? out_block[b] : b;
    if (ob >= 0) dst[ob] = static_cast<O>(blk_key[b] % ncols);
  }
}

// ---------------------------------------------------- your_logic_kernel

__global__ void tile_counts(const int64_t* __restrict__ win_start, int64_t nwin,
                            int64_t* __restrict__ tiles) {
  GRID_STRIDE(w, nwin + 1) tiles[w] = w < nwin ? (win_start[w + 1] - win_start[w] + 15) / 16 : 0;
}

template <typename O>
__global__ void tile_columns(const uint64_t* __restrict__ blk_key, const int64_t* __restrict__ win_start,
                             const int64_t* __restrict__ tile_ptr, int64_t nb, int64_t ncols,
                             O* __restrict__ dst) {
  GRID_STRIDE(b, nb) {
    const int64_t w = static_cast<int64_t>(blk_key[b] / ncols);
    const int64_t k = b - win_start[w];
    dst[16 * (tile_ptr[w] + k / 16) + k % 16] = static_cast<O>(blk_key[b] % ncols);
  }
}

// ------------------------------------------------------- hybrid split

// One key for the block order of the split: occupancy ascending, ties in
// first-seen order (first element ascending), the order the two stable sorts
// below give: key = occupancy << pbits | first element (first < 2^pbits).
// An occupancy of 2^cbits or more (only duplicate CSR entries make one larger
// than the window) does not fit: *wide is set and the caller takes the
// two-sort path instead.
__global__ void split_keys(const int64_t* __restrict__ blk_first, const int64_t* __restrict__ blk_cnt,
                           int64_t nb, int pbits, int cbits, uint64_t* __restrict__ key,
                           int64_t* __restrict__ id, int* __restrict__ wide) {
  const int64_t cmax = (int64_t(1) << cbits) - 1;
  GRID_STRIDE(b, nb) {
    const int64_t cnt = blk_cnt[b];
    if (cnt < 0 || cnt > cmax) atomicOr(wide, 1);
    const int64_t cc = cnt < 0 ? 0 : (cnt > cmax ? cmax : cnt);
    key[b] = (static_cast<uint64_t>(cc) << pbits) | static_cast<uint64_t>(blk_first[b]);
    id[b] = b;
  }
}

__global__ void collect_three(const int64_t* __restrict__ a, const int64_t* __restrict__ b,
                              const int* __restrict__ c, int64_t* __restrict__ scal) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    scal[0] = *a;
    scal[1] = *b;
    scal[2] = *c;
  }
}

// Keys for the first-seen order of blocks (first element = first position).
__global__ void first_seen_keys(const int64_t* __restrict__ blk_first, int64_t nb,
                                uint64_t* __restrict__ key, int64_t* __restrict__ id) {
  GRID_STRIDE(b, nb) {
    key[b] = static_cast<uint64_t>(blk_first[b]);
    id[b] = b;
  }
}

__global__ void count_keys(const int64_t* __restrict__ order, const int64_t* __restrict__ blk_cnt,
                           int64_t nb, uint64_t* __restrict__ key) {
  GRID_STRIDE(i, nb) key[i] = static_cast<uint64_t>(blk_cnt[order[i]]);
}

__global__ void gather_counts(const int64_t* __restrict__ order, const int64_t* __restrict__ blk_cnt,
                              int64_t nb, int64_t* __restrict__ cnt_sorted) {
  GRID_STRIDE(i, nb + 1) cnt_sorted[i] = i < nb ? blk_cnt[order[i]] : 0;
}

// Grid-wide minima.  Same-address device-scope atomics serialise (measured
// about 11 ns apiece on MI355X, so one per wave made a 1.9M-candidate minimum
// take 0.33 ms): the kernels that use this run a grid capped at kReduceGroups
// work-groups whose threads loop, reduce over the work-group, and issue one
// atomicMin per work-group.  Every thread of the work-group must call it;
// ~0 means "no candidate".
constexpr unsigned kReduceGroups = 512;

__device__ inline void group_atomic_min(unsigned long long* dst, unsigned long long v) {
  __shared__ unsigned long long part[kT / 64];
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long u = __shfl_xor(v, o);
    v = u < v ? u : v;
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kT / 64; ++w) v = part[w] < v ? part[w] : v;
    if (v != ~0ull) atomicMin(dst, v);
  }
}

__device__ inline uint64_t nonneg_bits(double d) {
  // Non-negative doubles order like their bit patterns; NaN is never chosen.
  if (!(d >= 0.0)) return 0x7ff0000000000000ull;  // +inf
  return __double_as_longlong(d);
}

// |ratio(k) - a| of hybrid_split_impl (custom_op.cpp:1207-1220).
__device__ inline double split_diff(int64_t k, int64_t nb, const int64_t* prefix, double a) {
  const int64_t rem = nb - k;
  const int64_t nz = prefix[k];
  const double ratio = (nz == 0) ? (rem > 0 ? INFINITY : 0.0)
                                 : static_cast<double>(rem) / static_cast<double>(nz);
  return fabs(ratio - a);
}

__global__ void split_min(const int64_t* __restrict__ prefix, int64_t nb, double a,
                          unsigned long long* __restrict__ best) {
  unsigned long long m = ~0ull;
  GRID_STRIDE(k, nb + 1) {
    const unsigned long long v = nonneg_bits(split_diff(k, nb, prefix, a));
    m = v < m ? v : m;
  }
  group_atomic_min(best, m);
}

__global__ void split_first(const int64_t* __restrict__ prefix, int64_t nb, double a,
                            const unsigned long long* __restrict__ best,
                            unsigned long long* __restrict__ kbest) {
  const unsigned long long target = *best;
  unsigned long long m = ~0ull;
  GRID_STRIDE(k, nb + 1) {
    if (m == ~0ull && nonneg_bits(split_diff(k, nb, prefix, a)) == target) m = static_cast<unsigned long long>(k);
  }
  group_atomic_min(kbest, m);
}

// Moved blocks: the first k* of the count order (k* = 0 when no finite minimum).
__global__ void mark_moved(const int64_t* __restrict__ order, int64_t nb,
                           const unsigned long long* __restrict__ best,
                           const unsigned long long* __restrict__ kbest, int64_t* __restrict__ kept) {
  const int64_t k = (*best == 0x7ff0000000000000ull) ? 0 : static_cast<int64_t>(*kbest);
  GRID_STRIDE(i, nb) kept[order[i]] = i < k ? 0 : 1;
}

__global__ void kept_index(const int64_t* __restrict__ kept, const int64_t* __restrict__ kscan,
                           int64_t nb, int64_t* __restrict__ out_block) {
  GRID_STRIDE(b, nb) out_block[b] = kept[b] ? kscan[b] : -1;
}

// Flag per element: 1 if its block goes to the CSR part.
__global__ void moved_elements(const int64_t* __restrict__ elem_block, const int64_t* __restrict__ kept,
                               int64_t n, int64_t* __restrict__ flag) {
  GRID_STRIDE(e, n + 1) flag[e] = e < n ? 1 - kept[elem_block[e]] : 0;
}

template <typename O>
__global__ void residual_rowptr(const int64_t* __restrict__ row_first_elem, const int64_t* __restrict__ vdst,
                                int64_t nrows, int64_t m_pad, O* __restrict__ vrow) {
  GRID_STRIDE(r, m_pad + 1) {
    const int64_t e = r < nrows ? row_first_elem[r] : -1;
    vrow[r] = static_cast<O>(e >= 0 ? vdst[e] : vdst[row_first_elem[nrows]]);
  }
}

template <typename I>
__global__ void row_first_elements(const I* __restrict__ rowptr, int64_t nrows, int64_t p_begin,
                                   int64_t* __restrict__ out) {
  GRID_STRIDE(r, nrows + 1) out[r] = static_cast<int64_t>(rowptr[r]) - p_begin;
}

template <typename O, typename U>
__global__ void scatter_residual(const int64_t* __restrict__ flag, const int64_t* __restrict__ vdst,
                                 const int64_t* __restrict__ col64, const U* __restrict__ val,
                                 int64_t p_begin, int64_t n, O* __restrict__ vcol, U* __restrict__ vval) {
  GRID_STRIDE(e, n) {
    if (flag[e]) {
      vcol[vdst[e]] = static_cast<O>(col64[e]);
      vval[vdst[e]] = val[p_begin + e];
    }
  }
}

// ------------------------------------------------------------- taskmapping

// Per window: nnz (from the row pointer), blocks, density key.
template <typename I>
__global__ void window_stats(const I* __restrict__ rowptr, const int64_t* __restrict__ win_start,
                             int64_t nwin, int64_t nrows, int64_t* __restrict__ wnnz,
                             int64_t* __restrict__ wnb, uint64_t* __restrict__ dkey,
                             int64_t* __restrict__ wid) {
  GRID_STRIDE(w, nwin) {
    const int64_t r0 = 16 * w;
    const int64_t r1 = r0 + 16 < nrows ? r0 + 16 : nrows;
    const int64_t nz = static_cast<int64_t>(rowptr[r1]) - static_cast<int64_t>(rowptr[r0]);
    const int64_t nb = win_start[w + 1] - win_start[w];
    const double density = nb ? static_cast<double>(nz) / static_cast<double>(nb) : 0.0;
    wnnz[w] = nz;
    wnb[w] = nb;
    // descending density == ascending complement of the (non-negative) bits
    dkey[w] = ~static_cast<uint64_t>(__double_as_longlong(density));
    wid[w] = w;
  }
}

__global__ void gather_i64(const int64_t* __restrict__ src, const int64_t* __restrict__ idx, int64_t n,
                           int64_t* __restrict__ dst) {
  GRID_STRIDE(i, n) dst[i] = src[idx[i]];
}

// First sorted position with (prefix+nb)/295 >= (remaining-nnz_w)/505 (custom_op.cpp:813-826).
__global__ void boundary_search(const int64_t* __restrict__ snb, const int64_t* __restrict__ snnz,
                                const int64_t* __restrict__ pnb, const int64_t* __restrict__ pnnz,
                                int64_t nwin, int64_t nnz, unsigned long long* __restrict__ bpos) {
  unsigned long long m = ~0ull;
  GRID_STRIDE(pos, nwin) {
    const double aic_after = static_cast<double>(pnb[pos] + snb[pos]) / 295.0;
    const double aiv_after = static_cast<double>(nnz - pnnz[pos] - snnz[pos]) / 505.0;
    if (m == ~0ull && aic_after >= aiv_after) m = static_cast<unsigned long long>(pos);
  }
  group_atomic_min(bpos, m);
}

// Scalars shared by the taskmapping kernels (device resident).
// Host values a plan hands to its fill, kept at the head of the workspace.
struct Header {
  int64_t magic;
  int64_t p_begin, n, nb;
  int64_t a0, a1, a2, a3;  // pipeline-specific
};
constexpr int64_t kMagic = 0x5350'4d4d'5052'4531LL;

struct TaskState {
  unsigned long long bpos;       // marginal sorted position, or ~0 (none)
  unsigned long long best_bits;  // min max-cost bits
  unsigned long long best_q;     // first q with that cost
  int64_t bwin, bblocks, prefix_blocks, remaining, wnnz_b, baic, shared, naic;
  int64_t aic_real, out_rows, real_extent, layout;
  int64_t n_aic_blocks, vnnz, err_bits;
  double est_aic, est_aiv, est_max;
};

// The AIC block count, the vector nonzero count and the error bits, stored in
// the task state, which is then read back in one copy; and the plan's header
// for the fill (h holds the values the host already has), written before that
// read-back so that its synchronisation covers it.
__global__ void collect_taskmap(TaskState* __restrict__ st, const int64_t* __restrict__ slot_ptr,
                                const int64_t* __restrict__ vrow64, const int* __restrict__ err,
                                Header* __restrict__ header, Header h) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    st->n_aic_blocks = slot_ptr[st->naic];
    st->vnnz = vrow64[st->out_rows];
    st->err_bits = *err;
    h.a0 = st->n_aic_blocks;
    h.a1 = st->vnnz;
    h.a2 = st->out_rows;
    h.a3 = st->naic;
    *header = h;
  }
}

__global__ void task_init(TaskState* __restrict__ s) {
  s->bpos = ~0ull;
  s->best_bits = ~0ull;
  s->best_q = ~0ull;
}

// Resolves the marginal window from bpos.
__global__ void task_marginal(TaskState* __restrict__ s, const int64_t* __restrict__ swin,
                              const int64_t* __restrict__ snb, const int64_t* __restrict__ snnz,
                              const int64_t* __restrict__ pnb, const int64_t* __restrict__ pnnz,
                              int64_t nnz) {
  if (s->bpos == ~0ull) {
    s->bwin = -1;
    s->bblocks = 0;
    s->prefix_blocks = 0;
    s->remaining = 0;
    s->wnnz_b = 0;
    return;
  }
  const int64_t p = static_cast<int64_t>(s->bpos);
  s->bwin = swin[p];
  s->bblocks = snb[p];
  s->prefix_blocks = pnb[p];
  s->remaining = nnz - pnnz[p];
  s->wnnz_b = snnz[p];
}

// Marginal blocks sorted by occupancy descending, first-seen ascending
// (stable_bucket_sort_by_occupancy_desc, boundary_bucket_sort.h:13-56).
// The marginal window's blocks [b0, b1) are distinct columns of one window,
// so at most mcap = min(nb, ncols) of them: entry q < mcap is block b0 + q,
// key = (16 - occupancy) << pbits | first element (every first element is
// below 2^pbits); entries past b1 get 16 << pbits and sort last, so the sort
// needs pbits + 5 key bits over mcap entries, not over every block.
__global__ void marginal_keys(const TaskState* __restrict__ s, const int64_t* __restrict__ win_start,
                              const int64_t* __restrict__ blk_first, const int64_t* __restrict__ blk_cnt,
                              int64_t mcap, int pbits, uint64_t* __restrict__ key, int64_t* __restrict__ id,
                              int* __restrict__ err) {
  const int64_t bw = s->bwin;
  const int64_t b0 = bw >= 0 ? win_start[bw] : 0, b1 = bw >= 0 ? win_start[bw + 1] : 0;
  GRID_STRIDE(q, mcap) {
    const int64_t b = b0 + q;
    id[q] = b;
    if (b < b1) {
      const int64_t occ = blk_cnt[b];
      if (occ < 1 || occ > 16) atomicOr(err, kBadOccupancy);
      const int64_t o = occ < 1 ? 1 : (occ > 16 ? 16 : occ);
      key[q] = (static_cast<uint64_t>(16 - o) << pbits) | static_cast<uint64_t>(blk_first[b]);
    } else {
      key[q] = uint64_t(16) << pbits;  // after every marginal block
    }
  }
}

__global__ void marginal_occ(const int64_t* __restrict__ order, const int64_t* __restrict__ blk_cnt,
                             const TaskState* __restrict__ s, int64_t mcap, int64_t* __restrict__ occ) {
  const int64_t c = s->bblocks;
  GRID_STRIDE(q, mcap + 1) occ[q] = q < c ? blk_cnt[order[q]] : 0;
}

// max(aic, aiv) for the first q marginal blocks on AIC (custom_op.cpp:855-885).
__device__ inline void marginal_cost(const TaskState* s, int64_t q, const int64_t* assigned,
                                     double& aic, double& aiv, double& mx) {
  aic = static_cast<double>(s->prefix_blocks + q) / 295.0;
  const int64_t suffix = s->remaining - s->wnnz_b;
  aiv = static_cast<double>(suffix + s->wnnz_b - assigned[q]) / 505.0;
  mx = (aic < aiv) ? aiv : aic;  // std::max(aic, aiv)
}

__global__ void marginal_min(TaskState* __restrict__ s, const int64_t* __restrict__ assigned, int64_t nb) {
  if (s->bwin < 0) return;
  const int64_t c = s->bblocks;
  unsigned long long m = ~0ull;
  GRID_STRIDE(q, c + 1) {
    double aic, aiv, mx;
    marginal_cost(s, q, assigned, aic, aiv, mx);
    const unsigned long long v = nonneg_bits(mx);
    m = v < m ? v : m;
  }
  group_atomic_min(&s->best_bits, m);
  (void)nb;
}

__global__ void marginal_first(TaskState* __restrict__ s, const int64_t* __restrict__ assigned) {
  if (s->bwin < 0) return;
  const int64_t c = s->bblocks;
  const unsigned long long target = s->best_bits;
  unsigned long long m = ~0ull;
  GRID_STRIDE(q, c + 1) {
    double aic, aiv, mx;
    marginal_cost(s, q, assigned, aic, aiv, mx);
    if (m == ~0ull && nonneg_bits(mx) == target) m = static_cast<unsigned long long>(q);
  }
  group_atomic_min(&s->best_q, m);
}

__global__ void marginal_finish(TaskState* __restrict__ s, const int64_t* __restrict__ assigned,
                                int64_t nwin) {
  if (s->bwin < 0) {
    s->baic = 0;
    s->shared = 0;
    s->est_aic = s->est_aiv = s->est_max = 0.0;
    s->naic = 0;
    return;
  }
  const int64_t q = static_cast<int64_t>(s->best_q);
  double aic, aiv, mx;
  marginal_cost(s, q, assigned, aic, aiv, mx);
  s->est_aic = aic;
  s->est_aiv = aiv;
  s->est_max = mx;
  s->baic = q;
  s->shared = (q > 0 && q < s->bblocks) ? 1 : 0;
  s->naic = static_cast<int64_t>(s->bpos) + (q > 0 ? 1 : 0);
  (void)nwin;
}

// to_aic per block of the marginal window (the only blocks it is read for):
// the first baic blocks of the marginal order.
__global__ void marginal_to_aic(const TaskState* __restrict__ s, const int64_t* __restrict__ order,
                                int64_t mcap, int64_t* __restrict__ to_aic) {
  const int64_t c = s->bwin >= 0 ? s->bblocks : 0;
  GRID_STRIDE(i, mcap) {
    if (i < c) to_aic[order[i]] = i < s->baic ? 1 : 0;
  }
}

// Window roles: slot (AIC) or AIV rank, in sorted-position order.
__global__ void window_roles(const TaskState* __restrict__ s, const int64_t* __restrict__ swin,
                             int64_t nwin, int64_t* __restrict__ slot_of, int64_t* __restrict__ aiv_win,
                             int64_t* __restrict__ aic_win) {
  const bool none = s->bwin < 0;
  const int64_t bp = none ? 0 : static_cast<int64_t>(s->bpos);
  const bool m_aic = !none && s->baic > 0;
  GRID_STRIDE(i, nwin) {
    const int64_t w = swin[i];
    int64_t slot = -1, rank = -1;
    if (none) {
      rank = i;
    } else if (i < bp) {
      slot = i;
    } else if (i == bp) {
      if (m_aic) slot = bp; else rank = 0;
    } else {
      rank = i - bp - 1 + (m_aic ? 0 : 1);
    }
    slot_of[w] = slot;
    if (slot >= 0) aic_win[slot] = w;
    if (rank >= 0) aiv_win[rank] = w;
  }
}

__global__ void aiv_row_counts(const TaskState* __restrict__ s, const int64_t* __restrict__ aiv_win,
                               int64_t nwin, int64_t nrows, int64_t* __restrict__ cnt) {
  const int64_t naiv = nwin - s->naic;
  GRID_STRIDE(k, nwin + 1) {
    int64_t c = 0;
    if (k < naiv) {
      const int64_t w = aiv_win[k];
      c = (16 * w + 16 < nrows ? 16 * w + 16 : nrows) - 16 * w;
    }
    cnt[k] = c;
  }
}

__global__ void task_rows(TaskState* __restrict__ s, const int64_t* __restrict__ aiv_off, int64_t nwin,
                          int64_t nrows, int64_t ncols, int graph_layout) {
  const int64_t naiv = nwin - s->naic;
  const int64_t aiv_rows = aiv_off[naiv];  // exclusive scan total
  s->aic_real = nrows - aiv_rows;
  s->real_extent = 16 * s->naic + aiv_rows;
  s->layout = (graph_layout && nrows == ncols) ? 1 : 0;
  s->out_rows = s->layout ? 16 * nwin : s->real_extent;
}

// permutation[out] = original row, inv_permutation[row] = out (custom_op.cpp:917-940).
__global__ void task_permutation(const TaskState* __restrict__ s, const int64_t* __restrict__ slot_of,
                                 const int64_t* __restrict__ aiv_rank, const int64_t* __restrict__ aiv_off,
                                 int64_t nrows, int64_t* __restrict__ perm, int64_t* __restrict__ inv) {
  GRID_STRIDE(r, nrows) {
    const int64_t w = r / 16;
    const int64_t sl = slot_of[w];
    const int64_t o = sl >= 0 ? 16 * sl + (r - 16 * w) : 16 * s->naic + aiv_off[aiv_rank[w]] + (r - 16 * w);
    perm[o] = r;
    inv[r] = o;
  }
}

__global__ void aiv_ranks(const int64_t* __restrict__ aiv_win, const TaskState* __restrict__ s,
                          int64_t nwin, int64_t* __restrict__ aiv_rank) {
  const int64_t naiv = nwin - s->naic;
  GRID_STRIDE(k, naiv) aiv_rank[aiv_win[k]] = k;
}

// AIC-kept blocks: blocks of AIC windows, minus the non-AIC blocks of a shared
// marginal window (custom_op.cpp:942-979).
__global__ void aic_kept(const TaskState* __restrict__ s, const uint64_t* __restrict__ blk_key,
                         const int64_t* __restrict__ slot_of, const int64_t* __restrict__ to_aic,
                         int64_t nb, int64_t ncols, int64_t* __restrict__ kept) {
  GRID_STRIDE(b, nb + 1) {
    int64_t k = 0;
    if (b < nb) {
      const int64_t w = static_cast<int64_t>(blk_key[b] / ncols);
      k = slot_of[w] >= 0 && !(s->shared && w == s->bwin && !to_aic[b]) ? 1 : 0;
    }
    kept[b] = k;
  }
}

// Blocks kept per slot (slot order), for the AIC block pointer.
__global__ void slot_counts(const TaskState* __restrict__ s, const int64_t* __restrict__ aic_win,
                            const int64_t* __restrict__ win_start, const int64_t* __restrict__ kscan,
                            int64_t nwin, int64_t* __restrict__ cnt) {
  GRID_STRIDE(k, nwin + 1) {
    int64_t c = 0;
    if (k < s->naic) {
      const int64_t w = aic_win[k];
      c = kscan[win_start[w + 1]] - kscan[win_start[w]];
    }
    cnt[k] = c;
  }
}

__global__ void aic_block_index(const uint64_t* __restrict__ blk_key, const int64_t* __restrict__ kept,
                                const int64_t* __restrict__ kscan, const int64_t* __restrict__ win_start,
                                const int64_t* __restrict__ slot_of, const int64_t* __restrict__ slot_ptr,
                                int64_t nb, int64_t ncols, int64_t* __restrict__ out_block) {
  GRID_STRIDE(b, nb) {
    const int64_t w = static_cast<int64_t>(blk_key[b] / ncols);
    out_block[b] = kept[b] ? slot_ptr[slot_of[w]] + (kscan[b] - kscan[win_start[w]]) : -1;
  }
}

// AIV nonzeros: all of AIV-window rows, plus the non-AIC entries of a shared
// marginal window (custom_op.cpp:981-1001).  Flag per element.
__global__ void aiv_elements(const TaskState* __restrict__ s, const int64_t* __restrict__ row_of,
                             const int64_t* __restrict__ elem_block, const int64_t* __restrict__ slot_of,
                             const int64_t* __restrict__ to_aic, int64_t n, int64_t* __restrict__ flag) {
  GRID_STRIDE(e, n + 1) {
    int64_t f = 0;
    if (e < n) {
      const int64_t w = row_of[e] / 16;
      if (slot_of[w] < 0) f = 1;
      else if (s->shared && w == s->bwin && !to_aic[elem_block[e]]) f = 1;
    }
    flag[e] = f;
  }
}

// Per output row: count of its AIV entries (0 for padding rows).
__global__ void aiv_out_counts(const TaskState* __restrict__ s, const int64_t* __restrict__ perm,
                               const int64_t* __restrict__ row_first, const int64_t* __restrict__ escan,
                               int64_t max_rows, int64_t* __restrict__ cnt) {
  const int64_t out_rows = s->out_rows;
  GRID_STRIDE(o, max_rows + 1) {
    int64_t c = 0;
    if (o < out_rows) {
      const int64_t r = perm[o];
      if (r >= 0) c = escan[row_first[r + 1]] - escan[row_first[r]];
    }
    cnt[o] = c;
  }
}

template <typename O, typename U>
__global__ void scatter_aiv(const int64_t* __restrict__ flag, const int64_t* __restrict__ escan,
                            const int64_t* __restrict__ row_of, const int64_t* __restrict__ row_first,
                            const int64_t* __restrict__ inv, const int64_t* __restrict__ vrow,
                            const int64_t* __restrict__ col64, const U* __restrict__ val, int64_t p_begin,
                            int64_t n, O* __restrict__ vcol, U* __restrict__ vval,
                            int64_t* __restrict__ vcol64) {
  GRID_STRIDE(e, n) {
    if (flag[e]) {
      const int64_t r = row_of[e];
      const int64_t d = vrow[inv[r]] + (escan[e] - escan[row_first[r]]);
      vcol[d] = static_cast<O>(col64[e]);
      vval[d] = val[p_begin + e];
      vcol64[d] = col64[e];
    }
  }
}

// inv[col] with the checks of renumber_columns_for_packed_layout
// (packed_column_reindex.h:22-37); err bits: 16 range, 32 unmapped, 64 overflow.
template <typename O>
__global__ void renumber(const int64_t* __restrict__ cols, int64_t n, const int64_t* __restrict__ inv,
                         int64_t ninv, int64_t index_max, O* __restrict__ out, int* __restrict__ err) {
  GRID_STRIDE(i, n) {
    const int64_t c = cols[i];
    if (c < 0 || c >= ninv) {
      atomicOr(err, 16);
      continue;
    }
    const int64_t pc = inv[c];
    if (pc < 0) {
      atomicOr(err, 32);
      continue;
    }
    if (static_cast<uint64_t>(pc) > static_cast<uint64_t>(index_max)) {
      atomicOr(err, 64);
      continue;
    }
    out[i] = static_cast<O>(pc);
  }
}

// Transpose keys: entry e goes to packed row inv[col] (stable in position order).
// The transposed entry of element e goes to row inv[col] at column
// inv[row]; the sort value carries both e and inv[row] when they fit 32 bits
// each (packed), so transpose_entries reads no row or inverse: the elements
// run in row order here, so these inv[row] reads are nearly sequential.
__global__ void transpose_keys(const int64_t* __restrict__ col64, const int64_t* __restrict__ row_of,
                               const int64_t* __restrict__ inv, int64_t n, int packed,
                               uint64_t* __restrict__ key, int64_t* __restrict__ id) {
  GRID_STRIDE(e, n) {
    key[e] = static_cast<uint64_t>(inv[col64[e]]);
    id[e] = packed ? static_cast<int64_t>((static_cast<uint64_t>(inv[row_of[e]]) << 32) | static_cast<uint64_t>(e))
                   : e;
  }
}

__global__ void transpose_rowptr(const uint64_t* __restrict__ skey, int64_t n, int64_t rows,
                                 int64_t* __restrict__ rp) {
  GRID_STRIDE(i, n + 1) {
    const int64_t prev = i > 0 ? static_cast<int64_t>(skey[i - 1]) : -1;
    const int64_t cur = i < n ? static_cast<int64_t>(skey[i]) : rows;
    for (int64_t r = prev + 1; r <= cur; ++r) rp[r] = i;
  }
}

template <typename U>
__global__ void transpose_entries(const int64_t* __restrict__ sid, const int64_t* __restrict__ row_of,
                                  const int64_t* __restrict__ inv, const U* __restrict__ val, int64_t p_begin,
                                  int64_t n, int packed, int64_t* __restrict__ colT, U* __restrict__ valT) {
  GRID_STRIDE(i, n) {
    const int64_t v = sid[i];
    const int64_t e = packed ? static_cast<int64_t>(static_cast<uint64_t>(v) & 0xFFFFFFFFu) : v;
    colT[i] = packed ? static_cast<int64_t>(static_cast<uint64_t>(v) >> 32) : inv[row_of[e]];
    valT[i] = val[p_begin + e];
  }
}

}  // namespace pre
}  // namespace spmm

// ======================================================================
// Host orchestration
// ======================================================================
namespace spmm {
namespace pre {
namespace {

template <typename K, typename... Args>
inline void launch(K kernel, int64_t n, hipStream_t s, Args... args) {
  hipLaunchKernelGGL(kernel, dim3(grid_for(n)), dim3(kT), 0, s, args...);
}

// Launch of a kernel that ends in group_atomic_min (capped grid).
template <typename K, typename... Args>
inline void launch_reduce(K kernel, int64_t n, hipStream_t s, Args... args) {
  const unsigned g = grid_for(n);
  hipLaunchKernelGGL(kernel, dim3(g < kReduceGroups ? g : kReduceGroups), dim3(kT), 0, s, args...);
}

struct Csr {
  int64_t rows, cols, nnz;
  int32_t it, vt;
  const void* rowptr;
  const void* col;
  const void* val;
  int64_t vs() const { return vt == SPMM_VALUE_F16 ? 2 : (vt == SPMM_VALUE_F32 ? 4 : 8); }
};

Csr from_matrix(const spmm_csr_matrix* m) {
  return Csr{m->rows, m->cols, m->nnz, m->index_type, m->value_type, m->rowptr, m->col, m->value};
}


// Arrays of the window sort (upper bounds from the sizes only).
struct WinSort {
  int64_t nmax = 0, nrows = 0, nwin = 0;
  int* err = nullptr;
  int64_t* scal = nullptr;  // scalars read back to the host in one copy
  int64_t *row_of, *col64, *elem, *selem, *head, *bid, *blk_first, *blk_start, *blk_cnt,
      *elem_block, *win_start, *row_first;
  uint64_t *key, *skey, *blk_key;
  int64_t p_begin = 0, n = 0, nb = 0;

  void lay(Arena& a, int64_t rows, int64_t nnz, int64_t W) {
    nrows = rows;
    nmax = nnz;
    nwin = (rows + W - 1) / W;
    err = a.take<int>(4);
    scal = a.take<int64_t>(4);
    row_of = a.take<int64_t>(nmax);
    col64 = a.take<int64_t>(nmax);
    key = a.take<uint64_t>(nmax);
    elem = a.take<int64_t>(nmax);
    skey = a.take<uint64_t>(nmax);
    selem = a.take<int64_t>(nmax);
    head = a.take<int64_t>(nmax + 1);
    bid = a.take<int64_t>(nmax + 1);
    blk_key = a.take<uint64_t>(nmax);
    blk_first = a.take<int64_t>(nmax);
    blk_start = a.take<int64_t>(nmax);
    blk_cnt = a.take<int64_t>(nmax);
    elem_block = a.take<int64_t>(nmax);
    win_start = a.take<int64_t>(nwin + 1);
    row_first = a.take<int64_t>(rows + 1);
  }
};

struct Ctx {
  Arena arena;
  Prims prims;
  Header* header = nullptr;
  hipStream_t stream = nullptr;

  // Reserves the header and the rocPRIM temporary (sized for n elements).
  void begin(void* ws, int64_t n_for_temp) {
    arena.base = static_cast<char*>(ws);
    arena.used = 0;
    header = arena.take<Header>(1);
    prims.temp_bytes = Prims::temp_needed(n_for_temp + 1);
    prims.temp = arena.take<char>(static_cast<int64_t>(prims.temp_bytes));
  }
};

template <typename T>
spmm_status read_back(T* host, const T* dev, int64_t count, hipStream_t s) {
  if (count <= 0) return SPMM_OK;
  hipError_t e = hipMemcpyAsync(host, dev, sizeof(T) * count, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return check_hip(e, "reading preprocessing results");
}

// Zeroes `bytes` bytes at p: 16-byte stores over the aligned body, byte
// stores for the unaligned head and the tail.
spmm_status zero(void* p, int64_t bytes, hipStream_t s) {
  if (bytes <= 0) return SPMM_OK;
  unsigned char* b = static_cast<unsigned char*>(p);
  const int64_t head = std::min<int64_t>(bytes, (16 - reinterpret_cast<uintptr_t>(b) % 16) % 16);
  const int64_t body = (bytes - head) / 16;
  const int64_t tail = bytes - head - 16 * body;
  if (head) launch(fill_bytes, head, s, b, head);
  if (body) launch(fill_zero16, body, s, reinterpret_cast<uint4*>(b + head), body);
  if (tail) launch(fill_bytes, tail, s, b + head + 16 * body, tail);
  return check_launch("zero fill");
}

template <typename I>
spmm_status run_window_sort(const Csr& c, int64_t W, bool check_sorted, WinSort& S, Ctx& x) {
  hipStream_t s = x.stream;
  launch(fill_kernel<int>, 4, s, S.err, int64_t(4), 0);
  if (c.rows > 0)
    launch(check_rowptr<I>, c.rows, s, static_cast<const I*>(c.rowptr), c.rows, c.nnz, S.err);
  if (spmm_status st = check_launch("check_rowptr")) return st;
  hipLaunchKernelGGL(collect_ends<I>, dim3(1), dim3(64), 0, s, static_cast<const I*>(c.rowptr), c.rows, S.err,
                     S.scal);
  int64_t v[3] = {0, 0, 0};
  if (spmm_status st = read_back(v, S.scal, 3, s)) return st;
  if (v[2] & kBadRowptr)
    return fail(SPMM_ERR_INVALID_ARGUMENT,
                "invalid CSR row pointer: entries must be non-decreasing within [0, nnz]");
  S.p_begin = v[0];
  S.n = v[1] - S.p_begin;

  if (c.rows > 0 && S.n > 0)
    launch(expand_rows<I>, (S.n + kExpandChunk - 1) / kExpandChunk * kT, s,
           static_cast<const I*>(c.rowptr), static_cast<const I*>(c.col), c.rows, c.cols, S.p_begin, S.n,
           S.row_of, S.col64, check_sorted ? 1 : 0, S.err);
  launch(window_keys, S.n, s, S.row_of, S.col64, S.n, W, c.cols, S.key, S.elem);
  if (spmm_status st = check_launch("window_keys")) return st;
  const uint64_t maxkey = static_cast<uint64_t>(S.nwin > 0 ? S.nwin : 1) * static_cast<uint64_t>(c.cols > 0 ? c.cols : 1);
  if (hipError_t e = x.prims.sort_pairs(S.key, S.skey, S.elem, S.selem, S.n, bits_for(maxkey)))
    return check_hip(e, "window sort");
  launch(run_heads, S.n, s, S.skey, S.n, S.head);
  if (hipError_t e = x.prims.inclusive_sum(S.head, S.bid, S.n)) return check_hip(e, "block scan");
  hipLaunchKernelGGL(collect_blocks, dim3(1), dim3(64), 0, s, S.bid, S.n, S.err, S.scal);
  int64_t b[2] = {0, 0};
  if (spmm_status st = read_back(b, S.scal, 2, s)) return st;
  S.nb = b[0];
  const int64_t herr = b[1];
  if (herr & kBadColumn) return fail(SPMM_ERR_CONTRACT, "column index out of range");
  if (herr & kUnsortedRow)
    return fail(SPMM_ERR_INVALID_ARGUMENT,
                "each row's col_indices must be sorted in ascending order");
  launch(block_table, S.n, s, S.skey, S.selem, S.bid, S.n, S.blk_key, S.blk_first, S.blk_start,
         S.elem_block);
  launch(block_counts, S.nb, s, S.blk_start, S.nb, S.n, S.blk_cnt);
  launch(window_starts, S.nb + 1, s, S.blk_key, S.nb, c.cols, S.nwin, S.win_start);
  launch(row_first_elements<I>, c.rows + 1, s, static_cast<const I*>(c.rowptr), c.rows, S.p_begin,
         S.row_first);
  return check_launch("block table");
}

// Value copy kernels by element size.
template <typename F>
spmm_status by_value_size(int64_t vs, F f) {
  if (vs == 2) return f(uint16_t{});
  if (vs == 4) return f(uint32_t{});
  return f(uint64_t{});
}

// ------------------------------------------------------------ BCSR / cube

struct CubeExtra {
  int64_t* tiles;
  int64_t* tile_ptr;
  void lay(Arena& a, int64_t nwin) {
    tiles = a.take<int64_t>(nwin + 1);
    tile_ptr = a.take<int64_t>(nwin + 1);
  }
};

void lay_bcsr(Ctx& x, WinSort& S, CubeExtra* cube, const Csr& c, int64_t W, void* ws) {
  x.begin(ws, c.nnz);
  S.lay(x.arena, c.rows, c.nnz, W);
  if (cube) cube->lay(x.arena, S.nwin);
}

template <typename I>
spmm_status bcsr_plan(const Csr& c, int64_t W, void* ws, size_t ws_bytes, hipStream_t s,
                      bool tiles, int64_t* count) {
  Ctx x;
  WinSort S;
  CubeExtra cube;
  x.stream = s;
  x.prims.stream = s;
  lay_bcsr(x, S, tiles ? &cube : nullptr, c, W, ws);
  if (x.arena.used > ws_bytes) return fail(SPMM_ERR_CONTRACT, "preprocessing workspace too small");
  if (spmm_status st = run_window_sort<I>(c, W, true, S, x)) return st;
  Header h{kMagic, S.p_begin, S.n, S.nb, 0, 0, 0, 0};
  if (tiles) {
    launch(tile_counts, S.nwin + 1, s, S.win_start, S.nwin, cube.tiles);
    if (hipError_t e = x.prims.exclusive_sum(cube.tiles, cube.tile_ptr, S.nwin + 1))
      return check_hip(e, "tile scan");
    if (spmm_status st = read_back(&h.a0, cube.tile_ptr + S.nwin, 1, s)) return st;
    *count = h.a0;
  } else {
    *count = S.nb;
  }
  hipError_t e = hipMemcpyAsync(x.header, &h, sizeof h, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return check_hip(e, "storing the plan");
}

spmm_status load_header(Header& h, const Ctx& x) {
  if (spmm_status st = read_back(&h, x.header, 1, x.stream)) return st;
  if (h.magic != kMagic) return fail(SPMM_ERR_CONTRACT, "workspace does not hold a plan for this call");
  return SPMM_OK;
}

template <typename I>
spmm_status bcsr_fill(const Csr& c, int64_t W, void* ws, size_t ws_bytes, hipStream_t s, bool tiles,
                      void* crow_out, void* uniq_out, void* val_out) {
  Ctx x;
  WinSort S;
  CubeExtra cube;
  x.stream = s;
  lay_bcsr(x, S, tiles ? &cube : nullptr, c, W, ws);
  if (x.arena.used > ws_bytes) return fail(SPMM_ERR_CONTRACT, "preprocessing workspace too small");
  Header h;
  if (spmm_status st = load_header(h, x)) return st;
  S.p_begin = h.p_begin;
  S.n = h.n;
  S.nb = h.nb;
  const int64_t vs = c.vs();
  if (!tiles) {
    launch(convert_index<I>, S.nwin + 1, s, S.win_start, static_cast<I*>(crow_out), S.nwin + 1);
    launch(block_columns<I>, S.nb, s, S.blk_key, static_cast<const int64_t*>(nullptr), S.nb, c.cols,
           static_cast<I*>(uniq_out));
    if (spmm_status st = zero(val_out, 16 * S.nb * vs, s)) return st;
    return by_value_size(vs, [&](auto u) {
      using U = decltype(u);
      launch(scatter_values<U>, S.n, s, S.selem, S.bid, S.row_of, S.n, W,
             static_cast<const int64_t*>(nullptr), int64_t(16), int64_t(0), S.win_start, S.blk_key,
             c.cols, static_cast<const U*>(c.val), S.p_begin, static_cast<U*>(val_out));
      return check_launch("scatter_values");
    });
  }
  const int64_t ntiles = h.a0;
  launch(convert_index<I>, S.nwin + 1, s, cube.tile_ptr, static_cast<I*>(crow_out), S.nwin + 1);
  if (spmm_status st = zero(uniq_out, 16 * ntiles * static_cast<int64_t>(sizeof(I)), s)) return st;
  launch(tile_columns<I>, S.nb, s, S.blk_key, S.win_start, cube.tile_ptr, S.nb, c.cols,
         static_cast<I*>(uniq_out));
  if (spmm_status st = zero(val_out, 256 * ntiles * vs, s)) return st;
  return by_value_size(vs, [&](auto u) {
    using U = decltype(u);
    launch(scatter_values<U>, S.n, s, S.selem, S.bid, S.row_of, S.n, W,
           static_cast<const int64_t*>(cube.tile_ptr), int64_t(0), int64_t(1), S.win_start,
           S.blk_key, c.cols, static_cast<const U*>(c.val), S.p_begin, static_cast<U*>(val_out));
    return check_launch("scatter_values");
  });
}

// ------------------------------------------------------------ hybrid split

struct HybridArrays {
  WinSort S;
  uint64_t *fkey, *fskey, *ckey, *cskey;
  int64_t *fid, *forder, *corder, *cnt_sorted, *prefix, *kept, *kscan, *out_block, *eflag, *vdst;
  unsigned long long* best;  // [2]: min bits, first k
  int* wide;                 // an occupancy does not fit split_keys' key
  void lay(Arena& a, int64_t rows, int64_t nnz, int64_t W) {
    S.lay(a, rows, nnz, W);
    wide = a.take<int>(1);
    fkey = a.take<uint64_t>(nnz);
    fskey = a.take<uint64_t>(nnz);
    ckey = a.take<uint64_t>(nnz);
    cskey = a.take<uint64_t>(nnz);
    fid = a.take<int64_t>(nnz);
    forder = a.take<int64_t>(nnz);
    corder = a.take<int64_t>(nnz);
    cnt_sorted = a.take<int64_t>(nnz + 1);
    prefix = a.take<int64_t>(nnz + 1);
    kept = a.take<int64_t>(nnz + 1);
    kscan = a.take<int64_t>(nnz + 1);
    out_block = a.take<int64_t>(nnz);
    eflag = a.take<int64_t>(nnz + 1);
    vdst = a.take<int64_t>(nnz + 1);
    best = a.take<unsigned long long>(2);
  }
};

// Runs hybrid_split_impl up to the output sizes (kept blocks, vector nnz).
template <typename I>
spmm_status hybrid_run(const Csr& c, double a, int64_t W, HybridArrays& H, Ctx& x, int64_t* kept_out,
                       int64_t* vnnz_out) {
  hipStream_t s = x.stream;
  WinSort& S = H.S;
  if (spmm_status st = run_window_sort<I>(c, W, false, S, x)) return st;
  const int64_t nb = S.nb;
  // Block order: one sort on split_keys (occupancy, then first element),
  // unless an occupancy needs more than cbits; then (second round) the
  // first-seen sort followed by the stable occupancy sort.
  const int pbits = bits_for(static_cast<uint64_t>(S.n));
  const int cbits = bits_for(static_cast<uint64_t>(W > 0 ? W : 1));
  int64_t v[3] = {0, 0, 0};
  for (int round = 0; round < 2; ++round) {
    if (round == 0) {
      launch(fill_kernel<int>, 1, s, H.wide, int64_t(1), 0);
      launch(split_keys, nb, s, S.blk_first, S.blk_cnt, nb, pbits, cbits, H.ckey, H.fid, H.wide);
      if (hipError_t e = x.prims.sort_pairs(H.ckey, H.cskey, H.fid, H.corder, nb, pbits + cbits))
        return check_hip(e, "block order sort");
    } else {
      launch(first_seen_keys, nb, s, S.blk_first, nb, H.fkey, H.fid);
      if (hipError_t e = x.prims.sort_pairs(H.fkey, H.fskey, H.fid, H.forder, nb, pbits))
        return check_hip(e, "first-seen sort");
      launch(count_keys, nb, s, H.forder, S.blk_cnt, nb, H.ckey);
      if (hipError_t e = x.prims.sort_pairs(H.ckey, H.cskey, H.forder, H.corder, nb, pbits))
        return check_hip(e, "count sort");
    }
    launch(gather_counts, nb + 1, s, H.corder, S.blk_cnt, nb, H.cnt_sorted);
    if (hipError_t e = x.prims.exclusive_sum(H.cnt_sorted, H.prefix, nb + 1)) return check_hip(e, "prefix");
    launch(fill_kernel<unsigned long long>, 2, s, H.best, int64_t(2), ~0ull);
    launch_reduce(split_min, nb + 1, s, H.prefix, nb, a, H.best);
    launch_reduce(split_first, nb + 1, s, H.prefix, nb, a, H.best, H.best + 1);
    launch(mark_moved, nb, s, H.corder, nb, H.best, H.best + 1, H.kept);
    launch(fill_kernel<int64_t>, 1, s, H.kept + nb, int64_t(1), int64_t(0));
    if (hipError_t e = x.prims.exclusive_sum(H.kept, H.kscan, nb + 1)) return check_hip(e, "kept scan");
    launch(kept_index, nb, s, H.kept, H.kscan, nb, H.out_block);
    launch(moved_elements, S.n + 1, s, S.elem_block, H.kept, S.n, H.eflag);
    if (hipError_t e = x.prims.exclusive_sum(H.eflag, H.vdst, S.n + 1)) return check_hip(e, "residual scan");
    if (spmm_status st = check_launch("hybrid split")) return st;
    hipLaunchKernelGGL(collect_three, dim3(1), dim3(64), 0, s, H.kscan + nb, H.vdst + S.n, H.wide, S.scal);
    if (spmm_status st = read_back(v, S.scal, 3, s)) return st;
    if (round == 1 || v[2] == 0) break;
  }
  *kept_out = v[0];
  *vnnz_out = v[1];
  return SPMM_OK;
}

template <typename O>
spmm_status hybrid_write(const Csr& c, int64_t W, HybridArrays& H, int64_t n_kept, Ctx& x, void* crow,
                         void* uniq, void* val, void* vrow, void* vcol, void* vval) {
  hipStream_t s = x.stream;
  WinSort& S = H.S;
  const int64_t m_pad = S.nwin * W;
  launch(gather_index<O>, S.nwin + 1, s, H.kscan, S.win_start, static_cast<O*>(crow), S.nwin + 1);
  launch(block_columns<O>, S.nb, s, S.blk_key, static_cast<const int64_t*>(H.out_block), S.nb, c.cols,
         static_cast<O*>(uniq));
  launch(residual_rowptr<O>, m_pad + 1, s, S.row_first, H.vdst, c.rows, m_pad, static_cast<O*>(vrow));
  const int64_t vs = c.vs();
  if (spmm_status st = zero(val, W * n_kept * vs, s)) return st;
  return by_value_size(vs, [&](auto u) {
    using U = decltype(u);
    launch(scatter_values<U>, S.n, s, S.selem, S.bid, S.row_of, S.n, W,
           static_cast<const int64_t*>(H.out_block), W, int64_t(0), S.win_start, S.blk_key, c.cols,
           static_cast<const U*>(c.val), S.p_begin, static_cast<U*>(val));
    launch(scatter_residual<O, U>, S.n, s, H.eflag, H.vdst, S.col64, static_cast<const U*>(c.val),
           S.p_begin, S.n, static_cast<O*>(vcol), static_cast<U*>(vval));
    return check_launch("hybrid outputs");
  });
}

void lay_hybrid(Ctx& x, HybridArrays& H, const Csr& c, int64_t W, void* ws) {
  x.begin(ws, c.nnz);
  H.lay(x.arena, c.rows, c.nnz, W);
}

template <typename I>
spmm_status hybrid_plan(const Csr& c, double a, int64_t W, void* ws, size_t ws_bytes, hipStream_t s,
                        int64_t* kept, int64_t* vnnz) {
  Ctx x;
  HybridArrays H;
  x.stream = s;
  x.prims.stream = s;
  lay_hybrid(x, H, c, W, ws);
  if (x.arena.used > ws_bytes) return fail(SPMM_ERR_CONTRACT, "preprocessing workspace too small");
  if (spmm_status st = hybrid_run<I>(c, a, W, H, x, kept, vnnz)) return st;
  Header h{kMagic, H.S.p_begin, H.S.n, H.S.nb, *kept, *vnnz, 0, 0};
  hipError_t e = hipMemcpyAsync(x.header, &h, sizeof h, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return check_hip(e, "storing the plan");
}

template <typename I>
spmm_status hybrid_fill(const Csr& c, int64_t W, void* ws, size_t ws_bytes, hipStream_t s, void* crow,
                        void* uniq, void* val, void* vrow, void* vcol, void* vval) {
  Ctx x;
  HybridArrays H;
  x.stream = s;
  lay_hybrid(x, H, c, W, ws);
  if (x.arena.used > ws_bytes) return fail(SPMM_ERR_CONTRACT, "preprocessing workspace too small");
  Header h;
  if (spmm_status st = load_header(h, x)) return st;
  H.S.p_begin = h.p_begin;
  H.S.n = h.n;
  H.S.nb = h.nb;
  return hybrid_write<I>(c, W, H, h.a0, x, crow, uniq, val, vrow, vcol, vval);
}

// ------------------------------------------------------------- taskmapping

struct TaskArrays {
  WinSort S;
  TaskState* st;
  Header* theader;  // plan record of the transpose split
  int64_t *wnnz, *wnb, *wid, *swin, *snb, *snnz, *pnb, *pnnz, *mid, *morder, *occ, *assigned, *to_aic,
      *slot_of, *aiv_win, *aic_win, *aiv_rank, *rcnt, *aiv_off, *perm, *inv, *kept, *kscan, *scnt,
      *slot_ptr, *out_block, *eflag, *escan, *ocnt, *vrow64, *vcol64, *uniq64;
  uint64_t *dkey, *sdkey, *mkey, *smkey;
  // graph layout: transposed CSR + its hybrid split
  int64_t *rpT, *colT, *tkey_id, *sid;
  uint64_t *tkey, *stkey;
  unsigned char* valT;
  HybridArrays T;
  int64_t max_rows = 0;

  void lay(Arena& a, const Csr& c, bool layout) {
    const int64_t nnz = c.nnz;
    S.lay(a, c.rows, nnz, 16);
    const int64_t nwin = S.nwin;
    max_rows = 16 * nwin;
    st = a.take<TaskState>(1);
    theader = a.take<Header>(1);
    wnnz = a.take<int64_t>(nwin);
    wnb = a.take<int64_t>(nwin);
    wid = a.take<int64_t>(nwin);
    swin = a.take<int64_t>(nwin);
    snb = a.take<int64_t>(nwin);
    snnz = a.take<int64_t>(nwin);
    pnb = a.take<int64_t>(nwin);
    pnnz = a.take<int64_t>(nwin);
    dkey = a.take<uint64_t>(nwin);
    sdkey = a.take<uint64_t>(nwin);
    // The marginal window's blocks: at most marginal_capacity(nnz, ncols).
    const int64_t mcap = marginal_capacity(nnz, c.cols);
    mkey = a.take<uint64_t>(mcap);
    smkey = a.take<uint64_t>(mcap);
    mid = a.take<int64_t>(mcap);
    morder = a.take<int64_t>(mcap);
    occ = a.take<int64_t>(mcap + 1);
    assigned = a.take<int64_t>(mcap + 1);
    to_aic = a.take<int64_t>(nnz);  // indexed by block
    slot_of = a.take<int64_t>(nwin);
    aiv_win = a.take<int64_t>(nwin);
    aic_win = a.take<int64_t>(nwin);
    aiv_rank = a.take<int64_t>(nwin);
    rcnt = a.take<int64_t>(nwin + 1);
    aiv_off = a.take<int64_t>(nwin + 1);
    perm = a.take<int64_t>(max_rows);
    inv = a.take<int64_t>(c.rows);
    kept = a.take<int64_t>(nnz + 1);
    kscan = a.take<int64_t>(nnz + 1);
    scnt = a.take<int64_t>(nwin + 1);
    slot_ptr = a.take<int64_t>(nwin + 1);
    out_block = a.take<int64_t>(nnz);
    eflag = a.take<int64_t>(nnz + 1);
    escan = a.take<int64_t>(nnz + 1);
    ocnt = a.take<int64_t>(max_rows + 1);
    vrow64 = a.take<int64_t>(max_rows + 1);
    vcol64 = a.take<int64_t>(nnz);
    uniq64 = a.take<int64_t>(nnz);
    if (layout) {
      rpT = a.take<int64_t>(max_rows + 1);
      colT = a.take<int64_t>(nnz);
      tkey = a.take<uint64_t>(nnz);
      stkey = a.take<uint64_t>(nnz);
      tkey_id = a.take<int64_t>(nnz);
      sid = a.take<int64_t>(nnz);
      valT = a.take<unsigned char>(nnz * c.vs());
      T.lay(a, max_rows, nnz, 16);
    }
  }
};

void lay_task(Ctx& x, TaskArrays& A, const Csr& c, bool layout, void* ws) {
  x.begin(ws, c.nnz + 16 * ((c.rows + 15) / 16));
  A.lay(x.arena, c, layout);
}

Csr transposed_csr(const Csr& c, const TaskArrays& A, int64_t out_rows, int64_t n) {
  return Csr{out_rows, out_rows, n, SPMM_INDEX_I64, c.vt, A.rpT, A.colT, A.valT};
}

template <typename I>
spmm_status task_plan(const Csr& c, bool graph_layout, void* ws, size_t ws_bytes, hipStream_t s,
                      spmm_taskmap_info* info) {
  Ctx x;
  TaskArrays A;
  x.stream = s;
  x.prims.stream = s;
  const bool layout = graph_layout && c.rows == c.cols;
  lay_task(x, A, c, layout, ws);
  if (x.arena.used > ws_bytes) return fail(SPMM_ERR_CONTRACT, "preprocessing workspace too small");
  WinSort& S = A.S;
  if (spmm_status st = run_window_sort<I>(c, 16, false, S, x)) return st;
  const int64_t nwin = S.nwin, nb = S.nb, n = S.n;

  // Windows by density (descending), id ascending (custom_op.cpp:784-811).
  launch(window_stats<I>, nwin, s, static_cast<const I*>(c.rowptr), S.win_start, nwin, c.rows, A.wnnz,
         A.wnb, A.dkey, A.wid);
  if (hipError_t e = x.prims.sort_pairs(A.dkey, A.sdkey, A.wid, A.swin, nwin, 64))
    return check_hip(e, "density sort");
  launch(gather_i64, nwin, s, A.wnb, A.swin, nwin, A.snb);
  launch(gather_i64, nwin, s, A.wnnz, A.swin, nwin, A.snnz);
  if (hipError_t e = x.prims.exclusive_sum(A.snb, A.pnb, nwin)) return check_hip(e, "block prefix");
  if (hipError_t e = x.prims.exclusive_sum(A.snnz, A.pnnz, nwin)) return check_hip(e, "nnz prefix");
  // Marginal window and its block split (custom_op.cpp:813-885).
  launch(task_init, 1, s, A.st);
  launch_reduce(boundary_search, nwin, s, A.snb, A.snnz, A.pnb, A.pnnz, nwin, c.nnz, &A.st->bpos);
  launch(task_marginal, 1, s, A.st, A.swin, A.snb, A.snnz, A.pnb, A.pnnz, c.nnz);
  // The marginal window's blocks (at most mcap), keys (16 - occupancy) <<
  // pbits | first element (< n <= 2^pbits): pbits + 5 key bits.
  const int pbits = bits_for(static_cast<uint64_t>(n));
  const int64_t mcap = marginal_capacity(nb, c.cols);
  launch(marginal_keys, mcap, s, A.st, S.win_start, S.blk_first, S.blk_cnt, mcap, pbits, A.mkey, A.mid, S.err);
  if (hipError_t e = x.prims.sort_pairs(A.mkey, A.smkey, A.mid, A.morder, mcap, pbits + 5))
    return check_hip(e, "marginal sort");
  launch(marginal_occ, mcap + 1, s, A.morder, S.blk_cnt, A.st, mcap, A.occ);
  if (hipError_t e = x.prims.exclusive_sum(A.occ, A.assigned, mcap + 1)) return check_hip(e, "assigned");
  launch_reduce(marginal_min, mcap + 1, s, A.st, A.assigned, mcap);
  launch_reduce(marginal_first, mcap + 1, s, A.st, A.assigned);
  launch(marginal_finish, 1, s, A.st, A.assigned, nwin);
  launch(marginal_to_aic, mcap, s, A.st, A.morder, mcap, A.to_aic);
  // Window roles, rows and permutation (custom_op.cpp:887-940).
  launch(window_roles, nwin, s, A.st, A.swin, nwin, A.slot_of, A.aiv_win, A.aic_win);
  launch(aiv_ranks, nwin, s, A.aiv_win, A.st, nwin, A.aiv_rank);
  launch(aiv_row_counts, nwin + 1, s, A.st, A.aiv_win, nwin, c.rows, A.rcnt);
  if (hipError_t e = x.prims.exclusive_sum(A.rcnt, A.aiv_off, nwin + 1)) return check_hip(e, "row offsets");
  launch(task_rows, 1, s, A.st, A.aiv_off, nwin, c.rows, c.cols, graph_layout ? 1 : 0);
  launch(fill_kernel<int64_t>, A.max_rows, s, A.perm, A.max_rows, int64_t(-1));
  launch(task_permutation, c.rows, s, A.st, A.slot_of, A.aiv_rank, A.aiv_off, c.rows, A.perm, A.inv);
  // AIC pack (custom_op.cpp:942-979).
  launch(aic_kept, nb + 1, s, A.st, S.blk_key, A.slot_of, A.to_aic, nb, c.cols, A.kept);
  if (hipError_t e = x.prims.exclusive_sum(A.kept, A.kscan, nb + 1)) return check_hip(e, "kept scan");
  launch(slot_counts, nwin + 1, s, A.st, A.aic_win, S.win_start, A.kscan, nwin, A.scnt);
  if (hipError_t e = x.prims.exclusive_sum(A.scnt, A.slot_ptr, nwin + 1)) return check_hip(e, "slot scan");
  launch(aic_block_index, nb, s, S.blk_key, A.kept, A.kscan, S.win_start, A.slot_of, A.slot_ptr, nb, c.cols,
         A.out_block);
  // AIV pack (custom_op.cpp:981-1001).
  launch(aiv_elements, n + 1, s, A.st, S.row_of, S.elem_block, A.slot_of, A.to_aic, n, A.eflag);
  if (hipError_t e = x.prims.exclusive_sum(A.eflag, A.escan, n + 1)) return check_hip(e, "aiv scan");
  launch(aiv_out_counts, A.max_rows + 1, s, A.st, A.perm, S.row_first, A.escan, A.max_rows, A.ocnt);
  if (hipError_t e = x.prims.exclusive_sum(A.ocnt, A.vrow64, A.max_rows + 1)) return check_hip(e, "vrow scan");
  if (spmm_status st = check_launch("taskmapping")) return st;

  hipLaunchKernelGGL(collect_taskmap, dim3(1), dim3(64), 0, s, A.st, A.slot_ptr, A.vrow64, S.err, x.header,
                     Header{kMagic, S.p_begin, n, nb, 0, 0, 0, 0});
  TaskState hs;
  if (spmm_status st = read_back(&hs, A.st, 1, s)) return st;
  if (hs.err_bits & kBadOccupancy)
    return fail(SPMM_ERR_INVALID_ARGUMENT,
                "block occupancy must be in [1, window_size]; coalesce duplicate CSR entries");
  const int64_t aic_blocks = hs.n_aic_blocks, vnnz = hs.vnnz;

  spmm_taskmap_info r{};
  r.aic_windows = hs.naic;
  r.aic_blocks = aic_blocks;
  r.packed_rows = hs.out_rows;
  r.vector_nnz = vnnz;
  r.packed_layout_supported = hs.layout;
  r.marginal_window = hs.bwin;
  r.marginal_aic_blocks = hs.bwin >= 0 ? hs.baic : 0;
  r.marginal_total_blocks = hs.bwin >= 0 ? hs.bblocks : 0;
  r.shared_windows = hs.shared;
  r.estimated_aic_cost = hs.est_aic;
  r.estimated_aiv_cost = hs.est_aiv;
  r.estimated_max_cost = hs.est_max;

  if (layout) {
    // P * A^T * P^T: entry (r, c) goes to row inv[c], column inv[r], in
    // (row, position) order (packed_column_reindex.h:43-101), then the fixed
    // 295/505 split (pack_fixed_layout, custom_op.cpp:1350-1384).
    int64_t last = 0;
    if (spmm_status st = read_back(&last, S.row_first + c.rows, 1, s)) return st;
    if (S.p_begin != 0 || S.p_begin + last != c.nnz)
      return fail(SPMM_ERR_INVALID_ARGUMENT, "CSR row pointer does not end at nnz");
    // Element ids and packed rows below 2^32 travel packed in the sort value.
    const int packed = n <= 0xFFFFFFFFll && hs.out_rows <= 0xFFFFFFFFll ? 1 : 0;
    launch(transpose_keys, n, s, S.col64, S.row_of, A.inv, n, packed, A.tkey, A.tkey_id);
    if (hipError_t e = x.prims.sort_pairs(A.tkey, A.stkey, A.tkey_id, A.sid, n,
                                          bits_for(static_cast<uint64_t>(hs.out_rows))))
      return check_hip(e, "transpose sort");
    launch(transpose_rowptr, n + 1, s, A.stkey, n, hs.out_rows, A.rpT);
    spmm_status st = by_value_size(c.vs(), [&](auto u) {
      using U = decltype(u);
      launch(transpose_entries<U>, n, s, A.sid, S.row_of, A.inv, static_cast<const U*>(c.val), S.p_begin, n, packed,
             A.colT, reinterpret_cast<U*>(A.valT));
      return check_launch("transpose");
    });
    if (st) return st;
    const Csr t = transposed_csr(c, A, hs.out_rows, n);
    int64_t tk = 0, tv = 0;
    if (spmm_status st2 = hybrid_run<int64_t>(t, 295.0 / 505.0, 16, A.T, x, &tk, &tv)) return st2;
    r.t_windows = A.T.S.nwin;
    r.t_blocks = tk;
    r.t_rows = A.T.S.nwin * 16;
    r.t_vector_nnz = tv;
  }
  *info = r;
  if (!layout) return SPMM_OK;  // collect_taskmap stored the plan header
  // The transpose split's sizes beside it.
  Header ht{kMagic, A.T.S.p_begin, A.T.S.n, A.T.S.nb, r.t_blocks, r.t_vector_nnz, 0, 0};
  hipError_t e = hipMemcpyAsync(A.theader, &ht, sizeof ht, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return check_hip(e, "storing the plan");
}

template <typename I>
spmm_status task_fill(const Csr& c, bool graph_layout, void* ws, size_t ws_bytes, hipStream_t s,
                      const spmm_taskmap_out* o) {
  Ctx x;
  TaskArrays A;
  x.stream = s;
  const bool layout = graph_layout && c.rows == c.cols;
  lay_task(x, A, c, layout, ws);
  if (x.arena.used > ws_bytes) return fail(SPMM_ERR_CONTRACT, "preprocessing workspace too small");
  Header h;
  if (spmm_status st = load_header(h, x)) return st;
  WinSort& S = A.S;
  S.p_begin = h.p_begin;
  S.n = h.n;
  S.nb = h.nb;
  const int64_t aic_blocks = h.a0, vnnz = h.a1, out_rows = h.a2, naic = h.a3;
  const int64_t n = S.n, nb = S.nb, vs = c.vs();

  launch(convert_index<I>, naic + 1, s, A.slot_ptr, static_cast<I*>(o->crow_window_ptr), naic + 1);
  launch(block_columns<I>, nb, s, S.blk_key, static_cast<const int64_t*>(A.out_block), nb, c.cols,
         static_cast<I*>(o->unique_col_ids));
  launch(block_columns<int64_t>, nb, s, S.blk_key, static_cast<const int64_t*>(A.out_block), nb, c.cols,
         A.uniq64);
  launch(convert_index<I>, out_rows + 1, s, A.vrow64, static_cast<I*>(o->vrow_window_ptr), out_rows + 1);
  if (spmm_status st = zero(o->value, 16 * aic_blocks * vs, s)) return st;
  spmm_status st = by_value_size(vs, [&](auto u) {
    using U = decltype(u);
    launch(scatter_values<U>, n, s, S.selem, S.bid, S.row_of, n, int64_t(16),
           static_cast<const int64_t*>(A.out_block), int64_t(16), int64_t(0), S.win_start, S.blk_key, c.cols,
           static_cast<const U*>(c.val), S.p_begin, static_cast<U*>(o->value));
    launch(scatter_aiv<I, U>, n, s, A.eflag, A.escan, S.row_of, S.row_first, A.inv, A.vrow64, S.col64,
           static_cast<const U*>(c.val), S.p_begin, n, static_cast<I*>(o->vcol_indices),
           static_cast<U*>(o->vvalue), A.vcol64);
    return check_launch("taskmapping outputs");
  });
  if (st) return st;
  hipError_t e = hipSuccess;
  if (out_rows > 0)
    e = hipMemcpyAsync(o->permutation, A.perm, sizeof(int64_t) * out_rows, hipMemcpyDeviceToDevice, s);
  if (e == hipSuccess && c.rows > 0)
    e = hipMemcpyAsync(o->inv_permutation, A.inv, sizeof(int64_t) * c.rows, hipMemcpyDeviceToDevice, s);
  if (e != hipSuccess) return check_hip(e, "copying permutations");

  if (layout) {
    const int64_t index_max = sizeof(I) == 4 ? INT32_MAX : INT64_MAX;
    launch(fill_kernel<int>, 1, s, S.err, int64_t(1), 0);
    launch(renumber<I>, aic_blocks, s, A.uniq64, aic_blocks, A.inv, c.rows, index_max,
           static_cast<I*>(o->renumbered_unique_col_ids), S.err);
    launch(renumber<I>, vnnz, s, A.vcol64, vnnz, A.inv, c.rows, index_max,
           static_cast<I*>(o->renumbered_vcol_indices), S.err);
    int herr = 0;
    if (spmm_status st2 = read_back(&herr, S.err, 1, s)) return st2;
    if (herr & 16) return fail(SPMM_ERR_OUT_OF_RANGE, "column id cannot be mapped into the packed row layout");
    if (herr & 32) return fail(SPMM_ERR_INVALID_ARGUMENT, "inverse permutation does not map every original column");
    if (herr & 64) return fail(SPMM_ERR_OVERFLOW, "packed column id does not fit the sparse index type");
    Header ht;
    if (spmm_status st2 = read_back(&ht, A.theader, 1, s)) return st2;
    A.T.S.p_begin = ht.p_begin;
    A.T.S.n = ht.n;
    A.T.S.nb = ht.nb;
    const Csr t = transposed_csr(c, A, out_rows, n);
    return hybrid_write<I>(t, 16, A.T, ht.a0, x, o->transpose_crow_window_ptr, o->transpose_unique_col_ids,
                           o->transpose_value, o->transpose_vrow_window_ptr, o->transpose_vcol_indices,
                           o->transpose_vvalue);
  }
  return SPMM_OK;
}

spmm_status check_matrix(const spmm_csr_matrix* m, const char* op) {
  if (m == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, std::string(op) + ": null matrix");
  if (m->index_type != SPMM_INDEX_I32 && m->index_type != SPMM_INDEX_I64)
    return fail(SPMM_ERR_CONTRACT, std::string(op) + ": index arrays must be int32 or int64");
  if (m->value_type != SPMM_VALUE_F16 && m->value_type != SPMM_VALUE_F32 && m->value_type != SPMM_VALUE_F64)
    return fail(SPMM_ERR_CONTRACT, std::string(op) + ": values must be fp16, fp32 or fp64");
  if (m->rows < 0 || m->cols < 0 || m->nnz < 0)
    return fail(SPMM_ERR_INVALID_ARGUMENT, std::string(op) + ": negative extent");
  if (m->rowptr == nullptr || (m->nnz > 0 && (m->col == nullptr || m->value == nullptr)))
    return fail(SPMM_ERR_INVALID_ARGUMENT, std::string(op) + ": null device pointer");
  return SPMM_OK;
}

template <typename F>
spmm_status by_index(int32_t it, F f) {
  if (it == SPMM_INDEX_I32) return f(int32_t{});
  return f(int64_t{});
}

size_t bcsr_bytes(const spmm_csr_matrix* m, int64_t W, bool tiles) {
  Ctx x;
  WinSort S;
  CubeExtra cube;
  lay_bcsr(x, S, tiles ? &cube : nullptr, from_matrix(m), W, nullptr);
  return x.arena.used;
}

}  // namespace
}  // namespace pre
}  // namespace spmm

using namespace spmm;
using namespace spmm::pre;

extern "C" {

size_t spmm_bcsr_workspace(const spmm_csr_matrix* m, int64_t window_size) {
  if (m == nullptr || window_size < 1) return 0;
  return bcsr_bytes(m, window_size, false);
}

size_t spmm_cube_workspace(const spmm_csr_matrix* m, int64_t window_size) {
  if (m == nullptr || window_size < 1) return 0;
  return bcsr_bytes(m, window_size, true);
}

static spmm_status check_window16(int64_t W, const char* op) {
  if (W < 1 || W > 16)
    return fail(SPMM_ERR_INVALID_ARGUMENT,
                std::string(op) + ": window_size must be in [1, 16] (value blocks hold 16 rows)");
  return SPMM_OK;
}

spmm_status spmm_bcsr_plan(const spmm_csr_matrix* m, int64_t W, void* ws, size_t ws_bytes, spmm_stream s,
                           int64_t* blocks) {
  clear_error();
  if (spmm_status st = check_matrix(m, "csr_to_bcsr")) return st;
  if (spmm_status st = check_window16(W, "csr_to_bcsr")) return st;
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return bcsr_plan<decltype(i)>(c, W, ws, ws_bytes, as_stream(s), false, blocks);
  });
}

spmm_status spmm_bcsr_fill(const spmm_csr_matrix* m, int64_t W, void* ws, size_t ws_bytes, void* crow,
                           void* uniq, void* value, spmm_stream s) {
  clear_error();
  if (spmm_status st = check_matrix(m, "csr_to_bcsr")) return st;
  if (spmm_status st = check_window16(W, "csr_to_bcsr")) return st;
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return bcsr_fill<decltype(i)>(c, W, ws, ws_bytes, as_stream(s), false, crow, uniq, value);
  });
}

spmm_status spmm_cube_plan(const spmm_csr_matrix* m, int64_t W, void* ws, size_t ws_bytes, spmm_stream s,
                           int64_t* tiles) {
  clear_error();
  if (spmm_status st = check_matrix(m, "csr_to_ascend_cube")) return st;
  if (spmm_status st = check_window16(W, "csr_to_ascend_cube")) return st;
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return bcsr_plan<decltype(i)>(c, W, ws, ws_bytes, as_stream(s), true, tiles);
  });
}

spmm_status spmm_cube_fill(const spmm_csr_matrix* m, int64_t W, void* ws, size_t ws_bytes, void* crow,
                           void* uniq, void* value, spmm_stream s) {
  clear_error();
  if (spmm_status st = check_matrix(m, "csr_to_ascend_cube")) return st;
  if (spmm_status st = check_window16(W, "csr_to_ascend_cube")) return st;
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return bcsr_fill<decltype(i)>(c, W, ws, ws_bytes, as_stream(s), true, crow, uniq, value);
  });
}

size_t spmm_hybrid_workspace(const spmm_csr_matrix* m, int64_t W) {
  if (m == nullptr || W < 1) return 0;
  Ctx x;
  HybridArrays H;
  lay_hybrid(x, H, from_matrix(m), W, nullptr);
  return x.arena.used;
}

spmm_status spmm_hybrid_plan(const spmm_csr_matrix* m, double a, int64_t W, void* ws, size_t ws_bytes,
                             spmm_stream s, int64_t* kept, int64_t* vnnz) {
  clear_error();
  if (spmm_status st = check_matrix(m, "block_level_split")) return st;
  if (W < 1) return fail(SPMM_ERR_INVALID_ARGUMENT, "block_level_split: window_size must be positive");
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return hybrid_plan<decltype(i)>(c, a, W, ws, ws_bytes, as_stream(s), kept, vnnz);
  });
}

spmm_status spmm_hybrid_fill(const spmm_csr_matrix* m, double a, int64_t W, void* ws, size_t ws_bytes,
                             void* crow, void* uniq, void* value, void* vrow, void* vcol, void* vval,
                             spmm_stream s) {
  clear_error();
  (void)a;
  if (spmm_status st = check_matrix(m, "block_level_split")) return st;
  if (W < 1) return fail(SPMM_ERR_INVALID_ARGUMENT, "block_level_split: window_size must be positive");
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return hybrid_fill<decltype(i)>(c, W, ws, ws_bytes, as_stream(s), crow, uniq, value, vrow, vcol, vval);
  });
}

size_t spmm_taskmap_workspace(const spmm_csr_matrix* m, int64_t W, int graph_layout) {
  if (m == nullptr || W != 16) return 0;
  Ctx x;
  TaskArrays A;
  const Csr c = from_matrix(m);
  lay_task(x, A, c, graph_layout && c.rows == c.cols, nullptr);
  return x.arena.used;
}

spmm_status spmm_taskmap_plan(const spmm_csr_matrix* m, int64_t W, int graph_layout, void* ws,
                              size_t ws_bytes, spmm_stream s, spmm_taskmap_info* info) {
  clear_error();
  if (spmm_status st = check_matrix(m, "preprocess")) return st;
  if (W != 16) return fail(SPMM_ERR_CONTRACT, "Ascend-SpMM requires a 16-row window");
  if (info == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "preprocess: null info");
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return task_plan<decltype(i)>(c, graph_layout != 0, ws, ws_bytes, as_stream(s), info);
  });
}

spmm_status spmm_taskmap_fill(const spmm_csr_matrix* m, int64_t W, int graph_layout, void* ws,
                              size_t ws_bytes, const spmm_taskmap_out* out, spmm_stream s) {
  clear_error();
  if (spmm_status st = check_matrix(m, "preprocess")) return st;
  if (W != 16) return fail(SPMM_ERR_CONTRACT, "Ascend-SpMM requires a 16-row window");
  if (out == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "preprocess: null outputs");
  const Csr c = from_matrix(m);
  return by_index(c.it, [&](auto i) {
    return task_fill<decltype(i)>(c, graph_layout != 0, ws, ws_bytes, as_stream(s), out);
  });
}

}  // extern "C"
