// CSR gather path of the MI355X SpMM library (the vector/AIV part).
//
// Semantics follow the reference's vector engine
// (kernels/op_kernel/spmm_csr.cpp:383-423, 468-549 and the AIV branch of
// kernels/op_kernel/spmm_ascend_cube.cpp:586-673, 782-875):
//   out[i, :] = sum_{p in row i, nonzero order} value[p] * dense[col[p], :]
// accumulated in fp32 and rounded once to the output type.
//
// Work decomposition (MI355X-native, not the reference's 40-core split):
//  * Nonzero positions are cut into fixed ranges [j*R, (j+1)*R), where R is
//    a power of two chosen from nnz alone (gather_range: small matrices get
//    short ranges so that enough lane groups run at once).  A "lane group" of
//    L lanes (each lane owns 16 bytes of an output row: L = width/8 for fp16,
//    width/4 for fp32, capped at 64) processes one range.  Cut points depend
//    only on the positions and nnz, so every output element sees the same
//    fp32 operation sequence for every width N: results are deterministic and
//    bit-identical across widths.
//  * gather_tile_rows (one thread per row) records, for every tile, the row
//    holding the tile's first position.
//  * gather_tiles: a work-group takes a tile of consecutive ranges.  It reads
//    its row span from that table while it stages the tile's column ids and
//    values in LDS (one round trip), then marks, per position, the row that
//    starts there.  Each lane group then
//    streams its range flat: the dense rows of 4 consecutive nonzeros are
//    loaded together, two batches in flight (16 bytes per lane; the L lanes
//    of a group read L*16 contiguous bytes of one dense row), accumulated in
//    order, and flushed wherever the next position starts a new row.  Each
//    staged nonzero is one 16-byte LDS entry (column checked against K once,
//    value bits, row mark), so a position costs one LDS read and 32-bit
//    address arithmetic.  Empty rows are written as zeros.
//  * A short row (at most R/2 nonzeros) is summed entirely by the lane group
//    of the range where it starts (running on into the next range, staged as
//    a halo); the next range skips it.  So every such row is one
//    sequential fp32 sum, and only longer rows are split: they leave one fp32
//    partial per range in the workspace ("tail" in the range where they
//    start, "head" in every later range) and their id in the range's tail
//    entry; the post pass adds the partials in range order.
#include "common.h"
#include "lanevec.h"

namespace spmm {
namespace {

using lanes::LaneVec;
using lanes::clampi;

constexpr int kWgThreads = 256;
#ifndef SPMM_GATHER_BATCH
#define SPMM_GATHER_BATCH 4
#endif
constexpr int kBatch = SPMM_GATHER_BATCH;  // dense rows per batch
#ifndef SPMM_GATHER_INFLIGHT
#define SPMM_GATHER_INFLIGHT 2
#endif
constexpr int kInFlight = SPMM_GATHER_INFLIGHT;  // batches in flight per lane group
constexpr int kStageUnroll = 8;             // staging loads issued per thread before storing
// A row is "short" (summed by one lane group, never split) when it holds at
// most R / SPMM_GATHER_SHORT_DIV nonzeros.
#ifndef SPMM_GATHER_SPLIT_BYTES
#define SPMM_GATHER_SPLIT_BYTES 512
#endif
#ifndef SPMM_GATHER_SHORT_DIV
#define SPMM_GATHER_SHORT_DIV 2
#endif
#ifndef SPMM_GATHER_TILE_RANGES
#define SPMM_GATHER_TILE_RANGES 16
#endif
// Ranges per work-group tile (the tile stages ranges * R nonzeros in LDS).
constexpr int64_t kTileRanges = SPMM_GATHER_TILE_RANGES;

template <typename I>
struct Geometry {
  const I* rowptr;
  int64_t* tail;           // [nranges]: row that starts in range j and runs past its end, or -1
  int64_t* tile_row;       // [tiles + 1]: row holding the first position of tile t
  int64_t row_lo, row_hi;  // rows handled
  int64_t vrows;           // rowptr holds vrows + 1 entries; rows >= vrows are empty
  int64_t nnz;             // extent of col[] / value[]
  int64_t range;           // R, positions per range
  int64_t nranges;         // max(1, ceil(nnz / R))
  // Block part of the mixed operator (cwin == 0 for spmm_csr): the vector sum
  // of a row in a block window that has blocks goes to vpart in fp32 (the
  // block kernel, run afterwards, adds it to the block sum and rounds once);
  // such rows are otherwise left to the block kernel.
  const I* Crowptr;
  int64_t cwin, climit;
  float* vpart;

  __device__ inline int64_t rp(int64_t r) const {
    return clampi(static_cast<int64_t>(rowptr[r < vrows ? r : vrows]), 0, nnz);
  }
  __device__ inline int64_t lo(int64_t j) const { return j * range; }
  __device__ inline int64_t hi(int64_t j) const {
    const int64_t h = (j + 1) * range;
    return h < nnz ? h : nnz;
  }
  __device__ inline int64_t crp(int64_t s) const {
    return clampi(static_cast<int64_t>(Crowptr[s]), 0, climit);
  }
  // Row r lies in a block window that has blocks.
  __device__ inline bool in_block_window(int64_t r) const {
    const int64_t s = r / 16;
    return s < cwin && crp(s + 1) > crp(s);
  }
};

// LDS entry of one staged nonzero (16 bytes, read with one ds_read_b128):
//   x: column id, or kBadCol when it is outside [0, K)
//   y: value bits (fp16 zero-extended, or fp32)
//   z: row mark, (row + 1 - rS) << 2 | to_vpart << 1 | ends_here, where the
//      row part is set only at the position a row starts
constexpr uint32_t kBadCol = 0xFFFFFFFFu;

template <typename T>
__device__ inline uint32_t value_bits(T v) {
  if constexpr (sizeof(T) == 2)
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, v));
  else
    return __builtin_bit_cast(uint32_t, v);
}
template <typename T>
__device__ inline float bits_value(uint32_t b) {
  if constexpr (sizeof(T) == 2)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
  else
    return __builtin_bit_cast(float, b);
}

// One batch of kBatch consecutive nonzeros: raw 16-byte dense pieces, values
// and row marks.  Positions past the range end or with an invalid column
// carry value -0 and a zero dense piece, so their FMA adds exactly -0 (the
// identity of fp32 addition); positions past the range end carry mark 0.
template <typename T>
struct Batch {
  lanes::raw16_t x[kBatch];
  float v[kBatch];
  int32_t m[kBatch];
  uint32_t ok;  // bit u: position u has a dense piece to use
};

// Issues the dense loads of a batch from the LDS entries.  Positions are
// relative to the tile start.  Branch-free so the loads of a batch stay in
// flight together: skipped positions load dense row 0 (K >= 1 here).
template <typename T>
struct Stream {
  const lanes::raw16_t* s_ent;
  const T* dense_c0;  // dense + c0
  uint32_t N;
  int32_t pe;

  __device__ inline void issue(Batch<T>& b, int32_t p0) const {
    b.ok = 0;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int32_t p = p0 + u;
      const bool in = p < pe;
      const lanes::raw16_t e = s_ent[in ? p : pe - 1];
      const bool ok = in && e.x != kBadCol;
      b.ok |= ok ? 1u << u : 0u;
      b.v[u] = ok ? bits_value<T>(e.y) : -0.0f;
      b.m[u] = in ? static_cast<int32_t>(e.z) : 0;
      const uint64_t off = static_cast<uint64_t>(ok ? e.x : 0u) * N;
      b.x[u] = lanes::load_raw16(dense_c0 + off);
    }
  }
};

// Accumulates batches in position order: tracks the current row from the
// marks, routes rows of block windows to vpart, and flushes at row ends.
template <typename T>
struct Sink {
  const lanes::raw16_t* s_ent;
  int64_t rS, row_hi;
  T* out;
  int64_t N, c0;
  float* vpart;
  float* head_slot;
  float* tail_slot;
  int32_t rel;             // row in progress + 1 - rS; 0 while it is one started before the range
  bool to_vpart;           // the row in progress belongs to a block window
  float acc[lanes::LaneVec<T>::V];

  __device__ inline void flush() {
    constexpr int V = lanes::LaneVec<T>::V;
    const int64_t row = rS + rel - 1;
    // fp32 destinations: the head slot (row begun before the range) and
    // vpart (block-window rows); others are rounded into out.
    if (row < row_hi) {
      if (rel == 0 || to_vpart) {
        float* dst = rel == 0 ? head_slot : vpart + row * N + c0;
#pragma unroll
        for (int i = 0; i < V; ++i) dst[i] = acc[i];
      } else {
        lanes::LaneVec<T>::store(out + row * N + c0, acc);
      }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
  }

  __device__ inline void consume(const Batch<T>& b) {
    constexpr int V = lanes::LaneVec<T>::V;
    const lanes::raw16_t zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int32_t m = b.m[u];
      const int32_t start = m >> 2;
      rel = start ? start : rel;
      to_vpart = start ? (m & 2) != 0 : to_vpart;
      float x[V];
      lanes::LaneVec<T>::unpack((b.ok >> u & 1u) ? b.x[u] : zero, x);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = __builtin_fmaf(b.v[u], x[i], acc[i]);
      if (m & 1) flush();
    }
  }

  // The row in progress at the range end continues into the next range:
  // returns that row if it started in this range (a tail), else -1.
  __device__ inline int64_t finish(int32_t pe) {
    constexpr int V = lanes::LaneVec<T>::V;
    if (s_ent[pe - 1].z & 1u) return -1;
    float* dst = rel == 0 ? head_slot : tail_slot;
#pragma unroll
    for (int i = 0; i < V; ++i) dst[i] = acc[i];
    return rel == 0 ? -1 : rS + rel - 1;
  }
};

#ifndef SPMM_GATHER_WAVES
#define SPMM_GATHER_WAVES 5
#endif
// Waves per SIMD the register budget of gather_tiles is fitted to.
template <typename T, typename I>
__global__ __launch_bounds__(kWgThreads) __attribute__((amdgpu_waves_per_eu(SPMM_GATHER_WAVES))) void gather_tiles(
    Geometry<I> g, const I* __restrict__ col, const T* __restrict__ value,
    const T* __restrict__ dense, int64_t K, int64_t N, T* __restrict__ out, float* __restrict__ ws,
    int log2L, int64_t chunks, int64_t ranges_per_tile, int64_t slot, int wg_split) {
  constexpr int V = LaneVec<T>::V;
  extern __shared__ __align__(16) unsigned char smem[];
  // The tile's positions plus a halo of one range: a short row that starts
  // in the tile's last range is finished from the halo.
  const int64_t tile_positions = (ranges_per_tile + 1) * g.range;
  lanes::raw16_t* s_ent = reinterpret_cast<lanes::raw16_t*>(smem);
  uint32_t* s_word = reinterpret_cast<uint32_t*>(smem);  // s_word[4*i + 2] = mark of entry i
  // s_cut[k]: end (relative to P0) of the short row crossing the tile's k-th
  // range boundary P0 + k*R, or -1.
  __shared__ int32_t s_cut[kTileRanges + 1];

  // wg_split > 1: the tile's column chunks go to wg_split work-groups (chunk
  // = blockIdx % wg_split); consecutive blockIdx land on different XCDs, so
  // each XCD's L2 serves one chunk of the dense rows.
  const int64_t tile = static_cast<int64_t>(blockIdx.x) / wg_split;
  const int64_t part = static_cast<int64_t>(blockIdx.x) % wg_split;
  const int64_t j0 = tile * ranges_per_tile;
  const int64_t j1 = (j0 + ranges_per_tile < g.nranges) ? j0 + ranges_per_tile : g.nranges;
  const int64_t P0 = g.lo(j0), P1 = g.hi(j1 - 1);
  const int64_t base = g.rp(g.row_lo), end = g.rp(g.row_hi);

  // Rows overlapping the tile: [rS, rE) with rS = the row holding position P0
  // and rE = one past the row holding P1 (the next tile's first position),
  // from the tile-row table of gather_tile_rows; tiles starting outside our
  // positions [base, end) clamp to the row range.  Runs of empty rows before
  // the tile are skipped.
  const int64_t rS = P0 < base ? g.row_lo : (P0 < end ? g.tile_row[tile] : g.row_hi);
  const int64_t rE = P1 < base ? g.row_lo : (P1 < end ? g.tile_row[tile + 1] + 1 : g.row_hi);

  // Stage the tile's nonzeros as LDS entries (positions clamped to [0, nnz);
  // those outside our rows are never read), column ids checked against K
  // once here, marks cleared.  The loads do not wait for the row lookups
  // above; each thread issues its loads before the first LDS store.
  const int64_t nr = j1 - j0;
  if (threadIdx.x <= nr) s_cut[threadIdx.x] = -1;
  for (int64_t i0 = 0; i0 < tile_positions; i0 += kStageUnroll * blockDim.x) {
    I cs[kStageUnroll];
    T vs[kStageUnroll];
#pragma unroll
    for (int k = 0; k < kStageUnroll; ++k) {
      int64_t p = P0 + i0 + k * blockDim.x + threadIdx.x;
      p = p < g.nnz ? p : g.nnz - 1;
      cs[k] = col[p];
      vs[k] = value[p];
    }
#pragma unroll
    for (int k = 0; k < kStageUnroll; ++k) {
      const int64_t i = i0 + k * blockDim.x + threadIdx.x;
      if (i < tile_positions) {
        const int64_t c = static_cast<int64_t>(cs[k]);
        const uint32_t c32 = static_cast<uint64_t>(c) < static_cast<uint64_t>(K) ? static_cast<uint32_t>(c) : kBadCol;
        s_ent[i] = lanes::raw16_t{c32, value_bits<T>(vs[k]), 0u, 0u};
      }
    }
  }
  __syncthreads();
  // Mark the starts and ends of the tile's non-empty rows (ends also in the
  // halo); each position is marked only by the row that holds it.  A short
  // row (at most R / SPMM_GATHER_SHORT_DIV nonzeros) that crosses a range
  // boundary is owned by the range where it starts: s_cut tells that range
  // how far to run on and the next range where to begin.  Longer rows leave
  // one fp32 partial per range instead.  Empty rows are left to the post pass.
  for (int64_t r = rS + threadIdx.x; r < rE; r += blockDim.x) {
    const int64_t a = g.rp(r), b = g.rp(r + 1);
    if (a < b) {
      const bool start_in = a >= P0 && a < P1 && r - rS < (INT32_MAX >> 2) - 1;
      const bool end_in = b - 1 >= P0 && b - 1 < P0 + tile_positions;
      if (start_in) {
        const uint32_t vp = g.in_block_window(r) ? 2u : 0u;
        s_word[4 * (a - P0) + 2] = static_cast<uint32_t>((r - rS + 1) << 2) | vp | (end_in && b - 1 == a ? 1u : 0u);
      }
      if (end_in && !(start_in && b - 1 == a)) s_word[4 * (b - 1 - P0) + 2] = 1u;
      if (b - a <= g.range / SPMM_GATHER_SHORT_DIV) {
        const int64_t k = a < P0 ? 0 : (a - P0) / g.range + 1;  // first boundary after a
        if (k <= nr && P0 + k * g.range < b) s_cut[k] = static_cast<int32_t>(b - P0);
      }
    }
  }
  __syncthreads();

  // Lane group -> (range j, column chunk cc).
  const int L = 1 << log2L;
  const int group = threadIdx.x >> log2L;
  const int lane = threadIdx.x & (L - 1);
  const int64_t wg_chunks = chunks / wg_split;
  const int64_t j = j0 + group / wg_chunks;
  const int64_t cc = part * wg_chunks + group % wg_chunks;
  if (j >= j1) return;
  const bool reporter = lane == 0 && cc == 0;  // writes tail[j]
  const int64_t c0 = (cc * L + lane) * V;
  const int64_t lo = g.lo(j), hi = g.hi(j);
  // Skip the short row owned by the previous range; run on to the end of the
  // short row this range owns past its end.  Positions from here on are
  // relative to P0.
  const int32_t cut_in = s_cut[j - j0], cut_out = s_cut[j - j0 + 1];
  const int32_t ps = cut_in >= 0 ? cut_in : static_cast<int32_t>((lo > base ? lo : base) - P0);
  const int32_t pe = cut_out >= 0 ? cut_out : static_cast<int32_t>((hi < end ? hi : end) - P0);
  if (ps >= pe || c0 >= N) {
    if (reporter) g.tail[j] = -1;
    return;
  }

  Sink<T> sk;
  sk.s_ent = s_ent;
  sk.rS = rS;
  sk.row_hi = g.row_hi;
  sk.out = out;
  sk.N = N;
  sk.c0 = c0;
  sk.vpart = g.vpart;
  sk.to_vpart = false;
  sk.head_slot = ws + (2 * j) * slot + c0;
  sk.tail_slot = ws + (2 * j + 1) * slot + c0;
  sk.rel = 0;  // set by the first row-start mark; stays 0 for a row begun earlier
#pragma unroll
  for (int i = 0; i < V; ++i) sk.acc[i] = 0.f;

  if (K <= 0) {  // no valid column: rows still flush (as zeros)
    Batch<T> z;
    z.ok = 0;
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      z.v[u] = -0.0f;
      z.x[u] = lanes::raw16_t{0, 0, 0, 0};
    }
    for (int32_t p0 = ps; p0 < pe; p0 += kBatch) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) z.m[u] = p0 + u < pe ? static_cast<int32_t>(s_ent[p0 + u].z) : 0;
      sk.consume(z);
    }
  } else {
    // kInFlight batches of kBatch dense rows in flight: the loads of the
    // next kInFlight-1 batches are issued before a batch is accumulated.
    Stream<T> st;
    st.s_ent = s_ent;
    st.dense_c0 = dense + c0;
    st.N = static_cast<uint32_t>(N);
    st.pe = pe;
    Batch<T> bq[kInFlight];
#pragma unroll
    for (int k = 0; k + 1 < kInFlight; ++k) st.issue(bq[k], ps + k * kBatch);
    for (int32_t p0 = ps; p0 < pe; p0 += kInFlight * kBatch) {
#pragma unroll
      for (int k = 0; k < kInFlight; ++k) {
        st.issue(bq[(k + kInFlight - 1) % kInFlight], p0 + (k + kInFlight - 1) * kBatch);
        sk.consume(bq[k]);
      }
    }
  }
  const int64_t tail_row = sk.finish(pe);
  if (reporter) g.tail[j] = tail_row;
}

// Tile-row table: for every tile t whose first position P = t*T lies in a
// row of [row_lo, row_hi), tile_row[t] = that row.  One thread per row writes
// the tile starts inside its nonzero span [rp(r), rp(r+1)).
template <typename I>
__global__ __launch_bounds__(kWgThreads) void gather_tile_rows(Geometry<I> g, int64_t T, int64_t tiles) {
  const int64_t r = g.row_lo + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= g.row_hi) return;
  const int64_t a = g.rp(r), b = g.rp(r + 1);
  const int64_t t_end = (b + T - 1) / T < tiles ? (b + T - 1) / T : tiles;
  for (int64_t t = (a + T - 1) / T; t < t_end; ++t) g.tile_row[t] = r;
}

// Post pass, one launch:
//  * work-groups [0, fix_blocks): add the partials of every row that crosses
//    range ends, in range order (lane group per (range, column chunk));
//  * the rest: empty rows, 64 per wavefront, are written as zeros (rows of
//    block windows with blocks are left to the block kernel).
template <typename T, typename I>
__global__ __launch_bounds__(kWgThreads) void gather_post(Geometry<I> g, int64_t N, T* __restrict__ out,
                                                          const float* __restrict__ ws, int log2L,
                                                          int64_t chunks, int64_t slot, int64_t fix_blocks) {
  constexpr int V = LaneVec<T>::V;
  if (static_cast<int64_t>(blockIdx.x) < fix_blocks) {
    const int L = 1 << log2L;
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t item = tid >> log2L;
    const int lane = static_cast<int>(tid & (L - 1));
    if (item >= (g.nranges - 1) * chunks) return;
    const int64_t j = item / chunks;
    const int64_t cc = item - j * chunks;
    const int64_t c0 = (cc * L + lane) * V;
    if (c0 >= N) return;
    const int64_t r = g.tail[j];
    if (r < g.row_lo || r >= g.row_hi) return;  // no row starts in range j and continues
    const int64_t stop = g.rp(r + 1);

    float acc[V];
    const float* src = ws + (2 * j + 1) * slot + c0;
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = src[i];
    // Head partials of ranges j+1 .. k_end-1, read 8 at a time, added in order.
    int64_t k_end = (stop + g.range - 1) / g.range;
    if (k_end > g.nranges) k_end = g.nranges;
    constexpr int kFix = 8;
    for (int64_t k0 = j + 1; k0 < k_end; k0 += kFix) {
      lanes::raw16_t h[kFix][(V * 4 + 15) / 16];
#pragma unroll
      for (int u = 0; u < kFix; ++u) {
        const int64_t k = k0 + u < k_end ? k0 + u : k_end - 1;
        const float* hp = ws + (2 * k) * slot + c0;
#pragma unroll
        for (int w = 0; w < (V * 4 + 15) / 16; ++w) h[u][w] = lanes::load_raw16(hp + 4 * w);
      }
#pragma unroll
      for (int u = 0; u < kFix; ++u) {
        if (k0 + u < k_end) {
#pragma unroll
          for (int w = 0; w < (V * 4 + 15) / 16; ++w) {
            const lanes::float4_t f = __builtin_bit_cast(lanes::float4_t, h[u][w]);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[4 * w + i] = acc[4 * w + i] + f[i];
          }
        }
      }
    }
    if (g.in_block_window(r)) {
      float* dst = g.vpart + r * N + c0;
#pragma unroll
      for (int i = 0; i < V; ++i) dst[i] = acc[i];
    } else {
      LaneVec<T>::store(out + r * N + c0, acc);
    }
    return;
  }
  // Empty rows: wavefront w takes rows [row_lo + 64w, +64).
  const int lane = threadIdx.x & 63;
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) - fix_blocks) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t r = g.row_lo + wave * 64 + lane;
  // Rows of block windows with blocks are written by the block kernel.
  const bool zero_row = r < g.row_hi && g.rp(r) == g.rp(r + 1) && !g.in_block_window(r);
  unsigned long long pending = __ballot(zero_row);
  while (pending) {
    const int src_lane = __ffsll(static_cast<long long>(pending)) - 1;
    pending &= pending - 1;
    const int64_t rr = g.row_lo + wave * 64 + src_lane;
    for (int64_t c0 = static_cast<int64_t>(lane) * V; c0 < N; c0 += 64 * V) {
      float z[V];
#pragma unroll
      for (int i = 0; i < V; ++i) z[i] = 0.f;
      LaneVec<T>::store(out + rr * N + c0, z);
    }
  }
}

template <typename T, typename I>
spmm_status gather_typed(const void* rowptr, const void* col, const void* value, int64_t nnz,
                         int64_t vrows, int64_t row_lo, int64_t row_hi, const void* dense, int64_t K,
                         int64_t N, void* out, void* ws, size_t ws_bytes, const void* Crowptr,
                         int64_t cwin, int64_t climit, float* vpart, hipStream_t stream) {
  constexpr int V = LaneVec<T>::V;
  if (row_hi <= row_lo) return SPMM_OK;
  Geometry<I> g;
  g.rowptr = static_cast<const I*>(rowptr);
  g.row_lo = row_lo;
  g.row_hi = row_hi;
  g.vrows = vrows;
  g.nnz = nnz < 0 ? 0 : nnz;
  g.range = gather_range(g.nnz);
  g.nranges = g.nnz > 0 ? ceil_div(g.nnz, g.range) : 1;
  g.Crowptr = static_cast<const I*>(Crowptr);
  g.cwin = Crowptr ? cwin : 0;
  g.climit = climit;
  g.vpart = vpart;

  if (K > static_cast<int64_t>(kBadCol) - 1)
    return fail(SPMM_ERR_CONTRACT, "dense has too many rows for 32-bit column ids");
  const int64_t lanes_needed = N / V;
  int log2L = 0;
  while ((1 << log2L) < lanes_needed && log2L < 6) ++log2L;
  int L = 1 << log2L;
  int64_t chunks = ceil_div(lanes_needed, L);
  // Dense rows of at least SPMM_GATHER_SPLIT_BYTES: one work-group per
  // column chunk of a tile (rows of one chunk are halved first), so
  // neighbouring work-groups, which run on different XCDs, gather different
  // column pieces and each XCD's L2 holds a fraction of the dense operand.
  int wg_split = 1;
  if (SPMM_GATHER_SPLIT_BYTES > 0 && N * static_cast<int64_t>(sizeof(T)) >= SPMM_GATHER_SPLIT_BYTES) {
    if (chunks == 1 && L >= 16 && lanes_needed == L) {
      --log2L;
      L >>= 1;
      chunks = 2;
    }
    wg_split = static_cast<int>(chunks);
  }
  int64_t ranges_per_tile = (kWgThreads / L) / (chunks / wg_split);
  if (ranges_per_tile > kTileRanges) ranges_per_tile = kTileRanges;
  if (ranges_per_tile < 1) ranges_per_tile = 1;
  const int64_t groups_per_wg = ranges_per_tile * (chunks / wg_split);
  const int64_t wg_threads = groups_per_wg * L;
  const int64_t slot = gather_slot_floats(N);

  // Workspace: tail rows and the tile-row table, then the partial slots
  // (256-byte aligned).
  const size_t tail_bytes = align_up(static_cast<size_t>(2 * g.nranges + 1) * sizeof(int64_t), 256);
  const size_t need = tail_bytes + static_cast<size_t>(2 * g.nranges) * slot * sizeof(float);
  if (ws == nullptr || ws_bytes < need)
    return fail(SPMM_ERR_CONTRACT, "gather workspace too small: need " + std::to_string(need) +
                                       " bytes, got " + std::to_string(ws_bytes));
  g.tail = static_cast<int64_t*>(ws);
  g.tile_row = g.tail + g.nranges;
  float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + tail_bytes);

  if (g.nnz > 0) {
    const int64_t tiles = ceil_div(g.nranges, ranges_per_tile);
    hipLaunchKernelGGL((gather_tile_rows<I>), dim3(static_cast<unsigned>(ceil_div(row_hi - row_lo, kWgThreads))),
                       dim3(kWgThreads), 0, stream, g, ranges_per_tile * g.range, tiles);
    if (spmm_status st = check_launch("gather_tile_rows")) return st;
    const size_t lds = static_cast<size_t>((ranges_per_tile + 1) * g.range) * sizeof(lanes::raw16_t);
    hipLaunchKernelGGL((gather_tiles<T, I>), dim3(static_cast<unsigned>(tiles * wg_split)),
                       dim3(static_cast<unsigned>(wg_threads)), lds, stream, g,
                       static_cast<const I*>(col), static_cast<const T*>(value),
                       static_cast<const T*>(dense), K, N, static_cast<T*>(out), partial, log2L,
                       chunks, ranges_per_tile, slot, wg_split);
    if (spmm_status st = check_launch("gather_tiles")) return st;
  }
  const int64_t fix_items = g.nnz > 0 ? (g.nranges - 1) * chunks * L : 0;
  const int64_t fix_blocks = ceil_div(fix_items, kWgThreads);
  const int64_t row_blocks = ceil_div(ceil_div(row_hi - row_lo, 64), kWgThreads / 64);
  hipLaunchKernelGGL((gather_post<T, I>), dim3(static_cast<unsigned>(fix_blocks + row_blocks)),
                     dim3(kWgThreads), 0, stream, g, N, static_cast<T*>(out),
                     static_cast<const float*>(partial), log2L, chunks, slot, fix_blocks);
  return check_launch("gather_post");
}

}  // namespace

size_t gather_workspace_bytes(int64_t nnz, int64_t width) {
  const int64_t nr = (nnz > 0 ? ceil_div(nnz, gather_range(nnz)) : 1);
  return align_up(static_cast<size_t>(2 * nr + 1) * sizeof(int64_t), 256) +
         static_cast<size_t>(2 * nr) * gather_slot_floats(width) * sizeof(float);
}

spmm_status launch_gather(int32_t index_type, int32_t value_type, const void* rowptr,
                          const void* col, const void* value, int64_t nnz, int64_t vrows,
                          int64_t row_lo, int64_t row_hi, const void* dense, int64_t dense_rows,
                          int64_t width, void* out, void* workspace, size_t workspace_bytes,
                          const void* Crowptr, int64_t cwin, int64_t climit, float* vpart,
                          hipStream_t stream) {
#define SPMM_GATHER_CALL(T, I)                                                                 \
  return gather_typed<T, I>(rowptr, col, value, nnz, vrows, row_lo, row_hi, dense, dense_rows, \
                            width, out, workspace, workspace_bytes, Crowptr, cwin, climit, vpart, \
                            stream)
  if (value_type == SPMM_VALUE_F16) {
    if (index_type == SPMM_INDEX_I32) SPMM_GATHER_CALL(_Float16, int32_t);
    SPMM_GATHER_CALL(_Float16, int64_t);
  }
  if (index_type == SPMM_INDEX_I32) SPMM_GATHER_CALL(float, int32_t);
  SPMM_GATHER_CALL(float, int64_t);
#undef SPMM_GATHER_CALL
}

}  // namespace spmm
