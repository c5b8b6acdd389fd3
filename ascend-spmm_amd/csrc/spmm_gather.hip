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
//  * gather_tiles: a work-group takes a tile of consecutive ranges (tiles
//    are spread over the XCDs in runs of consecutive tiles, so neighbours
//    share an L2).  It stages the tile's nonzeros in LDS in one round of
//    loads: per position the byte offset of its dense row (or a sentinel
//    past the dense operand for an invalid column), the value bits, and a
//    row-end mark.  Wavefront 0 finds the row holding the tile's first
//    position by a multiway search over rowptr and marks the last position
//    of every row that ends in the tile while the others stage (when the
//    tile needs all wavefronts to stage in one round, every wavefront runs
//    the search, overlapping its staging loads, and the work-group marks the
//    rows after the staging).  Each lane group streams its range in order:
//    batches of 4 positions, two in flight, each position one raw buffer load of
//    16 bytes per lane (the buffer range check returns zeros for the
//    sentinel, so no position needs address arithmetic or a select), fp32
//    FMAs, and a flush of the accumulated row at each row-end mark.
//  * A short row (at most R/2 nonzeros, or R when R <= 32) is summed
//    entirely by the lane group of the range where it starts (running on
//    into the next range, staged as a halo); the next range skips it.  So every such row is one
//    sequential fp32 sum, and only longer rows are split: they leave one fp32
//    partial per range in the workspace ("tail" in the range where they
//    start, "head" in every later range) and their id in the range's tail
//    entry.
//  * gather_post adds those partials in range order and writes empty rows
//    as zeros.
#include "common.h"
#include "lanevec.h"

#include <atomic>
#include <type_traits>

// Raw buffer load of 16 bytes (the LLVM AMDGPU intrinsic): address = the
// resource's base + voffset + soffset, with the resource's range check
// (a load whose offset is past the extent returns zeros).
typedef int spmm_rsrc_t __attribute__((ext_vector_type(4)));
__device__ spmm::lanes::raw16_t spmm_raw_buffer_load_b128(spmm_rsrc_t rsrc, uint32_t voffset, uint32_t soffset,
                                                          int32_t aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");

namespace spmm {
namespace {

using lanes::LaneVec;
using lanes::clampi;

constexpr int kWgThreads = 256;
#ifndef SPMM_GATHER_BATCH
#define SPMM_GATHER_BATCH 4
#endif
constexpr int kBatch = SPMM_GATHER_BATCH;  // dense rows per batch
// Staging positions per thread and round: one round covers a tile of up to
// 18 * 256 positions (16 + 1 ranges of R <= 256), so its loads are all in
// flight together.
constexpr int kStageUnroll = 18;
// Dense rows of at least this many bytes are split into column chunks on
// separate work-groups (and so separate XCDs).
#ifndef SPMM_GATHER_SPLIT_BYTES
#define SPMM_GATHER_SPLIT_BYTES 512
#endif
// A row is "short" (summed by one lane group, never split) when it holds at
// most short_max(R) nonzeros: R / 2, or all of R for ranges of at most
// SPMM_GATHER_SHORT_FULL positions, where a lane group that runs on past its
// range end adds little and the partials it avoids dominate (config 4's
// vector part, R = 32).  A short row crosses at most one range end.
#ifndef SPMM_GATHER_SHORT_FULL
#define SPMM_GATHER_SHORT_FULL 32
#endif
inline int64_t short_max(int64_t range) { return range <= SPMM_GATHER_SHORT_FULL ? range : range / 2; }
#ifndef SPMM_GATHER_TILE_RANGES
#define SPMM_GATHER_TILE_RANGES 16
#endif
// Ranges per work-group tile (the tile stages ranges * R nonzeros in LDS).
constexpr int64_t kTileRanges = SPMM_GATHER_TILE_RANGES;
// Consecutive tiles one XCD (group) takes before the next group's run.
#ifndef SPMM_GATHER_XCD_RUN
#define SPMM_GATHER_XCD_RUN 16
#endif
constexpr int64_t kXcdRun = SPMM_GATHER_XCD_RUN;

template <typename I>
struct Geometry {
  const I* rowptr;
  int64_t* tail;           // [nranges]: row that starts in range j and runs past its end, or -1
  int64_t row_lo, row_hi;  // rows handled
  int64_t vrows;           // rowptr holds vrows + 1 entries; rows >= vrows are empty
  int64_t nnz;             // extent of col[] / value[]
  int64_t range;           // R, positions per range
  int64_t short_max;       // longest "short" row: short_max(R)
  int64_t nranges;         // max(1, ceil(nnz / R))
  // Block part of the mixed operator (cwin == 0 for spmm_csr): the vector sum
  // of a row in a block window that has blocks goes to vpart in fp32 (the
  // block kernel, run afterwards, adds it to the block sum and rounds once);
  // such rows are otherwise left to the block kernel.
  const I* Crowptr;
  int64_t cwin, climit;
  float* vpart;
  // Locality order of the block windows when set (order_words(cwin) int32
  // from `order`): gather_tiles' extra work-groups write one key per window
  // and one bucket histogram per share of the windows, gather_post's first
  // work-groups scatter the windows into the order.
  const I* Ccol;
  int64_t K;
  int32_t* order;   // [cwin]: the order
  int32_t* keys;    // [cwin]: bucket | rank within the share's bucket << kKeyRankShift
  int32_t* hist;    // [kXcds][kOrderBuckets]: windows per bucket of each share
  int32_t* nlocal;  // [kXcds]: local windows of each share
  // Segment work-groups (seg != nullptr): a segment of a long row crossing
  // range ends (the row's part inside one range) whose columns spread over
  // at least an eighth of [0, K) is summed by the segment work-groups at the
  // end of gather_tiles' grid, which deal such segments to the XCDs by
  // column slab; seg[2j] / seg[2j + 1] describe range j's head and tail
  // segments (written by segment_classify).
  uint32_t* seg;
  uint32_t* seg_flag;   // [chunks]: 1 when the chunk holds a segment (set by segment_classify)
  int64_t seg_chunk;    // ranges per chunk of the segment work-groups (a power of two)
  int seg_chunk_log2;
  int range_log2;       // log2(range)
  int64_t seg_chunks;   // chunks
  int64_t tile_blocks;  // work-groups before the segment work-groups in gather_tiles' grid
  int seg_split;        // segment work-groups per XCD and chunk (seg_split_for)
  float slab_scale;     // kXcds / K: column -> slab
  // [tiles]: the row holding tile t's first position t << tile_shift, which
  // segment_classify writes in place of gather_tiles' row search.
  int64_t* tile_row;
  int tile_shift;

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

// A staged tile is three LDS arrays over its positions (structure of arrays,
// 8 + sizeof(T) bytes per position; 4 aligned positions are read with one
// load of each array):
//   src:  where the position's dense row is read from (see the loaders)
//   mark: 0, or at the last position of a row (row + 1 - rS) << 1 | to_vpart
//   val:  value bits (the value type's own width); -0 for an invalid column
constexpr uint32_t kBadCol = 0xFFFFFFFFu;
static_assert(kBatch % 4 == 0 && (kBatch & (kBatch - 1)) == 0, "batches are read 4 positions at a time");

template <typename T>
using ValBits = typename std::conditional<sizeof(T) == 2, uint16_t, uint32_t>::type;
template <typename T>
constexpr ValBits<T> kNegZero = sizeof(T) == 2 ? 0x8000u : 0x80000000u;

template <typename T>
struct Staged {
  uint32_t* src;
  uint32_t* mark;
  ValBits<T>* val;
  __device__ inline Staged(unsigned char* smem, int64_t positions)
      : src(reinterpret_cast<uint32_t*>(smem)),
        mark(reinterpret_cast<uint32_t*>(smem) + positions),
        val(reinterpret_cast<ValBits<T>*>(reinterpret_cast<uint32_t*>(smem) + 2 * positions)) {}
  static constexpr size_t bytes_per_position() { return 8 + sizeof(ValBits<T>); }
  // Value bits of 4 consecutive positions from p (p % 4 == 0).
  __device__ inline void values4(int32_t p, uint32_t* vb) const {
    if constexpr (sizeof(T) == 2) {
      typedef unsigned int u2 __attribute__((ext_vector_type(2)));
      const u2 r = *reinterpret_cast<const u2*>(val + p);
      vb[0] = r[0] & 0xFFFFu;
      vb[1] = r[0] >> 16;
      vb[2] = r[1] & 0xFFFFu;
      vb[3] = r[1] >> 16;
    } else {
      const lanes::raw16_t r = *reinterpret_cast<const lanes::raw16_t*>(val + p);
#pragma unroll
      for (int u = 0; u < 4; ++u) vb[u] = r[u];
    }
  }
};

template <typename T>
__device__ inline ValBits<T> value_bits(T v) {
  return __builtin_bit_cast(ValBits<T>, v);
}
template <typename T>
__device__ inline float bits_value(uint32_t b) {
  if constexpr (sizeof(T) == 2)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
  else
    return __builtin_bit_cast(float, b);
}

// Dense-row loaders.  Each stages a 32-bit source per position and turns it
// into the lane's 16 bytes of that dense row, or zeros for an invalid column
// (whose staged value is -0, so the FMA adds exactly -0: the identity of
// fp32 addition, as an accumulator is never -0).
//
// BufferLoader (dense operands up to kBufferLimit bytes): the source is the
// row's byte offset col * row_bytes, read with a raw buffer load whose extent
// is the dense operand; an invalid column stages kBufferNone, which with any
// lane offset (< 4096) lies past the extent, so the buffer range check
// returns zeros without a memory access.  No address arithmetic per position.
constexpr uint32_t kBufferNone = 0xFFFFF000u;
constexpr int64_t kBufferLimit = kBufferNone;

using ::spmm_rsrc_t;
using ::spmm_raw_buffer_load_b128;

template <typename T>
struct BufferLoader {
  spmm_rsrc_t rsrc;
  uint32_t lane_bytes;  // c0 * sizeof(T)
  static constexpr uint32_t kNone = kBufferNone;
  __device__ inline BufferLoader(const T* dense, int64_t K, int64_t ld, int64_t N, int64_t c0) {
    const uint64_t a = reinterpret_cast<uint64_t>(dense);
    rsrc[0] = static_cast<int>(a & 0xFFFFFFFFu);
    rsrc[1] = static_cast<int>((a >> 32) & 0xFFFFu);  // stride 0: raw buffer
    rsrc[2] = static_cast<int>(static_cast<uint32_t>(buffer_extent(K, ld, N, sizeof(T))));
    rsrc[3] = 0x00020000;  // 32-bit data format; no swizzle, no thread-id offset
    lane_bytes = static_cast<uint32_t>(c0 * static_cast<int64_t>(sizeof(T)));
  }
  __device__ static inline uint32_t stage(int64_t c, int64_t K, int64_t ld) {
    return static_cast<uint64_t>(c) < static_cast<uint64_t>(K)
               ? static_cast<uint32_t>(c) * static_cast<uint32_t>(ld * static_cast<int64_t>(sizeof(T)))
               : kNone;
  }
  __device__ inline lanes::raw16_t load(uint32_t src) const {
    return spmm_raw_buffer_load_b128(rsrc, src + lane_bytes, 0u, 0);
  }
};

// GlobalLoader (larger dense operands): the source is the column id, or
// kBadCol; invalid columns load dense row 0 (K >= 1 here) and use zeros.
template <typename T>
struct GlobalLoader {
  const T* dense_c0;  // dense + c0
  uint32_t ld;        // row stride of dense (elements)
  static constexpr uint32_t kNone = kBadCol;
  __device__ inline GlobalLoader(const T* dense, int64_t, int64_t ld_, int64_t, int64_t c0)
      : dense_c0(dense + c0), ld(static_cast<uint32_t>(ld_)) {}
  __device__ static inline uint32_t stage(int64_t c, int64_t K, int64_t) {
    return static_cast<uint64_t>(c) < static_cast<uint64_t>(K) ? static_cast<uint32_t>(c) : kNone;
  }
  __device__ inline lanes::raw16_t load(uint32_t src) const {
    const bool ok = src != kNone;
    const lanes::raw16_t x = lanes::load_raw16(dense_c0 + static_cast<uint64_t>(ok ? src : 0u) * ld);
    const lanes::raw16_t zero = {0u, 0u, 0u, 0u};
    return ok ? x : zero;
  }
};

// One batch of B consecutive positions (B a multiple of 4): the lanes'
// 16-byte dense pieces, values and row-end marks.  Positions outside
// [ps, pe) carry source kNone (zero piece), value -0 and mark 0.
template <typename T, int B = kBatch>
struct Batch {
  static_assert(B % 4 == 0 && (B & (B - 1)) == 0, "batches are read 4 positions at a time");
  lanes::raw16_t x[B];
  float v[B];
  uint32_t m[B];
};

// Issues the dense loads of a batch from the staged arrays.  Positions are
// relative to the tile start; a batch starts at a multiple of 4.  The
// unmasked form is for batches wholly inside [ps, pe); the masked form (a
// range's first and last batches) gives positions outside it source kNone,
// value -0 and mark 0.
template <typename T, typename Loader>
struct Stream {
  Staged<T> s;
  Loader ld;
  int32_t ps, pe;

  template <bool kMasked, int B>
  __device__ inline void issue(Batch<T, B>& b, int32_t p0) const {
#pragma unroll
    for (int q = 0; q < B; q += 4) {
      // A masked batch reads no aligned group past the one holding pe - 1.
      const int32_t pq = !kMasked || p0 + q < pe ? p0 + q : ((pe - 1) & ~3);
      const lanes::raw16_t c4 = *reinterpret_cast<const lanes::raw16_t*>(s.src + pq);
      const lanes::raw16_t m4 = *reinterpret_cast<const lanes::raw16_t*>(s.mark + pq);
      uint32_t vb[4];
      s.values4(pq, vb);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int32_t p = p0 + q + u;
        const bool in = !kMasked || (p >= ps && p < pe);
        b.v[q + u] = bits_value<T>(in ? vb[u] : static_cast<uint32_t>(kNegZero<T>));
        b.m[q + u] = in ? m4[u] : 0u;
        b.x[q + u] = ld.load(in ? c4[u] : Loader::kNone);
      }
    }
  }
};

// Accumulates batches in position order and flushes at row ends: rows of
// block windows go to vpart, the first row of a range that began before the
// range goes to the head slot, and the rest are rounded into out.
template <typename T>
struct Sink {
  int64_t rS, row_hi;
  T* out;
  int64_t N, ld, c0;  // vpart rows hold N floats; out rows are ld elements apart
  float* vpart;
  float* head_slot;
  float* tail_slot;
  bool head;  // the row in progress began before this range
  float acc[lanes::LaneVec<T>::V];

  __device__ inline void flush(uint32_t m) {
    constexpr int V = lanes::LaneVec<T>::V;
    const int64_t row = rS + static_cast<int64_t>(m >> 1) - 1;
    if (row < row_hi) {
      if (head || (m & 1u)) {
        float* dst = head ? head_slot : vpart + row * N + c0;
#pragma unroll
        for (int i = 0; i < V; ++i) dst[i] = acc[i];
      } else {
        lanes::LaneVec<T>::store(out + row * ld + c0, acc);
      }
    }
    head = false;
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
  }

  template <int B>
  __device__ inline void consume(const Batch<T, B>& b) {
    constexpr int V = lanes::LaneVec<T>::V;
#pragma unroll
    for (int u = 0; u < B; ++u) {
      float x[V];
      lanes::LaneVec<T>::unpack(b.x[u], x);
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = __builtin_fmaf(b.v[u], x[i], acc[i]);
      if (b.m[u] != 0u) flush(b.m[u]);
    }
  }

  // The row in progress at the range end (a long row crossing it) continues
  // into the next range: its partial goes to the head slot if it began
  // before the range, else to the tail slot.
  __device__ inline void finish(bool open) {
    constexpr int V = lanes::LaneVec<T>::V;
    if (!open) return;
    float* dst = head ? head_slot : tail_slot;
#pragma unroll
    for (int i = 0; i < V; ++i) dst[i] = acc[i];
  }
};

// Row holding position P (rp(row_lo) <= P < rp(row_hi)): a multiway search
// over rowptr by one wavefront.  Each round keeps a bracket [lo, hi) with
// rp(lo) <= P < rp(hi) and probes one row per active lane, evenly spaced
// inside it (lo + step, lo + 2*step, ...); the probes at or below P form a
// prefix, whose length moves lo.  A full wavefront needs ceil(log65(rows))
// rounds; the result is uniform across the wavefront.
// spmm_csr (no block windows) over more than 65^2 rows starts from the row
// interpolated between base = rp(row_lo) and end = rp(row_hi): its first
// round probes rows kSeedStep apart around it, and when they bracket P the
// search goes on from that bracket (one more round), else from the whole
// row range.  Plain CSR rows hold positions evenly enough for that (configs
// 1-4 miss by at most 1,733 rows); the mixed op's vector part does not.
template <typename I>
__device__ inline int64_t find_row(const Geometry<I>& g, int64_t P, int64_t base, int64_t end) {
  const int lane = static_cast<int>(threadIdx.x & 63);
  const int lanes = __popcll(__ballot(true));  // a work-group's last wavefront may be partial
  int64_t lo = g.row_lo, hi = g.row_hi;
  constexpr int64_t kSeedStep = 64;
  if (g.cwin == 0 && hi - lo > 65 * 65 && end > base) {
    const double f = static_cast<double>(P - base) / static_cast<double>(end - base);
    const int64_t guess = lo + static_cast<int64_t>(f * static_cast<double>(hi - lo));
    int64_t g0 = guess - (lanes / 2) * kSeedStep;
    g0 = g0 < lo ? lo : g0;
    const int64_t r = g0 + lane * kSeedStep;
    const bool le = r < hi && g.rp(r) <= P;
    const int m = __popcll(__ballot(le));
    if (m >= 1 && m < lanes) {  // rp(g0 + (m-1) step) <= P < rp(g0 + m step), or hi
      lo = g0 + (m - 1) * kSeedStep;
      const int64_t h = g0 + m * kSeedStep;
      hi = h < hi ? h : hi;
    }
  }
  while (hi - lo > 1) {
    const int64_t step = (hi - lo + lanes) / (lanes + 1);
    const int64_t r = lo + (lane + 1) * step;
    const bool le = r < hi && g.rp(r) <= P;
    lo += __popcll(__ballot(le)) * step;
    hi = lo + step < hi ? lo + step : hi;
  }
  return lo;
}

// Locality order of the cwin block windows: a counting sort by the window's
// first block column in kOrderBuckets buckets over [0, K).  Windows that
// gather the same dense rows end up next to each other, and the block kernel
// deals runs of consecutive positions of the order to the XCDs in turn, so
// the XCDs sweep the dense operand together and each XCD's L2 holds the rows
// its next windows need.  Any permutation gives the same results (every
// window is summed by its own work-group), so ties within a bucket take the
// order of the LDS atomics.
//
// The order only pays where windows are local (their block columns span a
// small part of [0, K), as in banded or clustered matrices).  When fewer than
// half the windows span less than K / kOrderLocalDiv columns, the identity
// order is written instead.
//
// The windows are cut into kXcds shares; two steps, so that neither sits on
// the critical path of its kernel:
//  * window_keys, in gather_tiles' kXcds extra work-groups beside the
//    gathers, one per share: read each window's block range and first and
//    last block column (two dependent rounds of loads), count the share's
//    windows per bucket in LDS (the count before a window is its rank in
//    the bucket), and write key = bucket | rank << kKeyRankShift per window,
//    the share's histogram, and its number of local windows;
//  * scatter_share, in gather_post's first kXcds work-groups, one per share:
//    read the kXcds histograms, scan them into the share's start in every
//    bucket, and write each window of the share to start[bucket] + rank.
constexpr int64_t kOrderLocalDiv = 8;
constexpr int kKeyRankShift = 10;
static_assert(kOrderBuckets <= (1 << kKeyRankShift), "bucket ids fit below the rank");
static_assert((kOrderMaxWindows + kXcds - 1) / kXcds < (int64_t(1) << (31 - kKeyRankShift)),
              "ranks within a share fit the key");

// Segment words.  Range j has at most two segments of long rows that cross
// range ends: the head segment [jR, min(b, (j+1)R)) of the row crossing jR,
// and the tail segment [a, (j+1)R) of a row [a, b) starting in the range and
// crossing (j+1)R (for a row covering the whole range, only the head).  A
// word is kSegValid | slab << kSegSlabShift | offset, with offset the head
// segment's end or the tail segment's start relative to jR; 0 when the
// segment does not exist or stays with gather_tiles.  The segment's partial
// sum is the same fp32 sequence whichever work-group computes it.
constexpr uint32_t kSegValid = 0x80000000u;
constexpr int kSegSlabShift = 16;
constexpr uint32_t kSegOffsetMask = 0xFFFFu;
static_assert(kGatherRangeMax <= static_cast<int64_t>(kSegOffsetMask), "segment offsets fit the word");
// Chunks of the segment work-groups: the words of blockDim.x / 2 ranges (one
// word per thread), shared by kXcds * seg_split work-groups (seg_split per
// XCD, each taking every seg_split-th segment of its slab): a slab of a
// chunk of long rows holds about blockDim.x / 16 segments, one round of lane
// groups.  seg_split grows with the lanes a segment needs (its column
// chunks times L): 1 up to 8 lanes, 2 for one chunk of 16, 3 for two
// chunks (each best of 1-4 on config 2 at fp16 N = 64, 128 and 256).
constexpr int64_t kSegChunkRanges = kWgThreads / 2;
inline int seg_split_for(int64_t chunks, int L) { return chunks * L <= 8 ? 1 : (chunks == 1 ? 2 : 3); }
// Staging positions per lane and round in the segment work-groups (R / L
// positions per lane: 8 for R = 128 at 16 lanes).
constexpr int kSegStageUnroll = 8;
// The segment path's gather_tiles instantiation (its tiles and its segment
// work-groups) reads kSegBatch dense rows per batch, at SPMM_SEG_WAVES waves
// per SIMD (twice the rows in flight of the other instantiations, whose 4-row
// batches fit 5 waves; 8-row batches there would spill).
#ifndef SPMM_SEG_BATCH
#define SPMM_SEG_BATCH 8
#endif
#ifndef SPMM_SEG_WAVES
#define SPMM_SEG_WAVES 4
#endif
constexpr int kSegBatch = SPMM_SEG_BATCH;
// Batches of kSegBatch positions in flight per lane group in the segment
// work-groups; segments are staged in whole groups of kSegGroup positions,
// plus the kSegInflight - 1 batches the last group issues ahead.
#ifndef SPMM_SEG_INFLIGHT
#define SPMM_SEG_INFLIGHT 2
#endif
constexpr int kSegInflight = SPMM_SEG_INFLIGHT;
constexpr int kSegGroup = kSegInflight * kSegBatch;
// Staged positions per lane group for ranges of R positions.
__host__ __device__ inline int64_t seg_stage_stride(int64_t range) {
  return range + kSegGroup + (kSegInflight - 1) * kSegBatch;
}
// Segments shorter than R / kSegMinDiv positions stay with gather_tiles.
constexpr int64_t kSegMinDiv = 8;
// The segment work-groups run for matrices of at least kSegMinNnz nonzeros
// (on smaller ones the extra launch costs more than the L2 hits can save)
// whose dense operand spans at most kSegMaxDenseBytes (a column slab of 1/8
// of it is then within four times an XCD's 4 MB L2; config 2 at N = 512,
// 102 MB, gains 2%, while at 205 MB config 2 at N = 1024 loses 3%).
#ifndef SPMM_SEG_MIN_NNZ
#define SPMM_SEG_MIN_NNZ (int64_t(1) << 20)
#endif
constexpr int64_t kSegMinNnz = SPMM_SEG_MIN_NNZ;
constexpr int64_t kSegMaxDenseBytes = int64_t(128) << 20;

// Segment words of every range, one thread per row, before gather_tiles.  A
// long row (more than short_max(R) nonzeros) that crosses range ends is
// split at them; its segments go to the segment work-groups when its
// columns span at least K / kXcds (the first and last column; columns are
// sorted within a row) and the segment holds at least R / kSegMinDiv
// positions.  A segment's slab is the column slab (eighth of [0, K)) of its
// middle position, its column interpolated between the row's first and last
// columns.  Range j's head word belongs to the row holding position jR and
// its tail word to the row holding its last position, so each call writes
// every word of the ranges inside the rows; gather_tiles reads a word only
// where such a row crosses the range end.  A chunk holding any segment gets
// its flag set (cleared by the post pass).  The row holding a tile's first
// position is that tile's first row, recorded in tile_row.
template <typename I>
__global__ __launch_bounds__(kWgThreads) void segment_classify(Geometry<I> g, const I* __restrict__ col) {
  const int64_t r = g.row_lo + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int lane = static_cast<int>(threadIdx.x & 63);
  const int sh = g.range_log2, csh = g.seg_chunk_log2;
  const int64_t R = int64_t(1) << sh;
  int64_t a = 0, b = 0, ja = 0, jb = -1;
  bool split = false;
  float c_first = 0.f, c_step = 0.f;
  if (r < g.row_hi) {
    a = g.rp(r);
    b = g.rp(r + 1);
    if (a < b) {
      ja = a >> sh;
      jb = (b - 1) >> sh;
      if (b - a > g.short_max && ja != jb) {
        const int64_t cf = static_cast<int64_t>(col[a]), cl = static_cast<int64_t>(col[b - 1]);
        if (cf >= 0 && cf < g.K && cl >= 0 && cl < g.K) {
          split = (cl > cf ? cl - cf : cf - cl) * kXcds >= g.K;
          c_first = static_cast<float>(cf);
          c_step = static_cast<float>(cl - cf) / static_cast<float>(b - 1 - a);
        }
      }
    }
  }
  // Range j of row [a, b): its head word if the row holds jR, its tail
  // word if the row holds the range's last position.
  auto classify = [&](int64_t j, int64_t a, int64_t b, bool split, float c_first, float c_step) {
    auto word = [&](int64_t s0, int64_t s1, int64_t offset) -> uint32_t {
      if (!split || (s1 - s0) * kSegMinDiv < R) return 0u;
      const float c_mid = c_first + c_step * static_cast<float>(((s0 + s1) >> 1) - a);
      int slab = static_cast<int>(c_mid * g.slab_scale);
      slab = slab < 0 ? 0 : (slab >= kXcds ? kXcds - 1 : slab);
      return kSegValid | (static_cast<uint32_t>(slab) << kSegSlabShift) | static_cast<uint32_t>(offset);
    };
    const int64_t lo = j << sh, hi = lo + R < g.nnz ? lo + R : g.nnz;
    if (lo >= a) {  // the row holds lo: head segment if it crosses lo
      const int64_t e = b < hi ? b : hi;
      const uint32_t w = a < lo ? word(lo, e, e - lo) : 0u;
      g.seg[2 * j] = w;
      if (w != 0u) g.seg_flag[j >> csh] = 1u;
    }
    if (hi <= b) {  // the row holds the range's last position: tail segment if it starts here and crosses hi
      const uint32_t w = a >= lo && b > hi ? word(a, hi, a - lo) : 0u;
      g.seg[2 * j + 1] = w;
      if (w != 0u) g.seg_flag[j >> csh] = 1u;
    }
  };
  // Tiles t (first position t << tile_shift) starting in row [a, b).
  const int ts = g.tile_shift;
  auto tiles_of = [&](int64_t a, int64_t b, int64_t r, int first, int step) {
    for (int64_t t = ((a + (int64_t(1) << ts) - 1) >> ts) + first; t <= ((b - 1) >> ts); t += step) g.tile_row[t] = r;
  };
  // A row touching at most kClassifyOwn ranges is done by its thread; longer
  // rows are shared by the whole wavefront, one at a time.  A wavefront's own
  // loops run as long as its longest row's, so the bound is small: on a
  // power-law matrix of 2M nonzeros, 4 classified in 5.7 us against 8.2 us
  // for 16 and 14.8 us with every row on its own thread (2 and 8: 6.1 us).
  constexpr int64_t kClassifyOwn = 4;
  const bool own = jb - ja + 1 <= kClassifyOwn;
  if (own) {
    for (int64_t j = ja; j <= jb; ++j) classify(j, a, b, split, c_first, c_step);
    if (a < b) tiles_of(a, b, r, 0, 1);
  }
  unsigned long long shared = __ballot(!own);
  while (shared) {
    const int src = __ffsll(static_cast<long long>(shared)) - 1;
    shared &= shared - 1;
    const int64_t sa = __shfl(a, src), sb = __shfl(b, src), sr = __shfl(r, src);
    const bool ssplit = __shfl(static_cast<int>(split), src) != 0;
    const float sf = __shfl(c_first, src), ss = __shfl(c_step, src);
    const int64_t sja = sa >> sh, sjb = (sb - 1) >> sh;
    for (int64_t j = sja + lane; j <= sjb; j += 64) classify(j, sa, sb, ssplit, sf, ss);
    tiles_of(sa, sb, sr, lane, 64);
  }
}

// One work-group; hist: kOrderBuckets int32 of LDS.
template <typename I>
__device__ void window_keys(const Geometry<I>& g, int64_t part, int32_t* hist) {
  const int64_t share = (g.cwin + kXcds - 1) / kXcds;
  const int64_t s_lo = part * share;
  const int64_t s_hi = s_lo + share < g.cwin ? s_lo + share : g.cwin;
  const int64_t nt = blockDim.x;
  __shared__ int32_t s_local;
  for (int64_t i = threadIdx.x; i < kOrderBuckets; i += nt) hist[i] = 0;
  if (threadIdx.x == 0) s_local = 0;
  __syncthreads();
  int32_t local = 0;
  constexpr int kU = 4;  // windows per thread per round, their loads issued together
  for (int64_t s0 = s_lo; s0 < s_hi; s0 += nt * kU) {
    int64_t b0[kU], b1[kU], c[kU], e[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t s = s0 + int64_t(u) * nt + threadIdx.x;
      b0[u] = s < s_hi ? g.crp(s) : 0;
      b1[u] = s < s_hi ? g.crp(s + 1) : 0;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      c[u] = b1[u] > b0[u] ? static_cast<int64_t>(g.Ccol[b0[u]]) : 0;
      e[u] = b1[u] > b0[u] ? static_cast<int64_t>(g.Ccol[b1[u] - 1]) : 0;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t s = s0 + int64_t(u) * nt + threadIdx.x;
      if (s >= s_hi) continue;
      // Column ids are clamped to [0, K) (an invalid id only adds zeros in
      // the block kernel), so the span arithmetic cannot overflow.
      const int64_t first = g.K > 0 ? clampi(c[u], 0, g.K - 1) : 0, last = g.K > 0 ? clampi(e[u], 0, g.K - 1) : 0;
      const int32_t bucket = b1[u] > b0[u] && g.K > 0 ? static_cast<int32_t>(first * kOrderBuckets / g.K) : 0;
      const int64_t span = last > first ? last - first : first - last;
      local += span * kOrderLocalDiv < g.K ? 1 : 0;
      g.keys[s] = bucket | (atomicAdd(&hist[bucket], 1) << kKeyRankShift);
    }
  }
  atomicAdd(&s_local, local);
  __syncthreads();
  for (int64_t i = threadIdx.x; i < kOrderBuckets; i += nt) g.hist[part * kOrderBuckets + i] = hist[i];
  if (threadIdx.x == 0) g.nlocal[part] = s_local;
}

// One work-group of kWgThreads threads; start: kOrderBuckets int32 of LDS,
// run: kWgThreads int32 of LDS.
template <typename I>
__device__ void scatter_share(const Geometry<I>& g, int64_t part, int32_t* start, int32_t* run) {
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t share = (g.cwin + kXcds - 1) / kXcds;
  const int64_t s_lo = part * share;
  const int64_t s_hi = s_lo + share < g.cwin ? s_lo + share : g.cwin;
  int64_t local = 0;
#pragma unroll
  for (int b = 0; b < kXcds; ++b) local += g.nlocal[b];
  if (2 * local < g.cwin) {  // not local: identity order
    for (int64_t s = s_lo + tid; s < s_hi; s += nt) g.order[s] = static_cast<int32_t>(s);
    return;
  }
  // Thread tid takes buckets [tid * kPer, (tid + 1) * kPer): their totals
  // over the shares, and the windows of the shares before this one, which
  // is this share's offset inside each bucket.
  constexpr int kPer = (kOrderBuckets + kWgThreads - 1) / kWgThreads;
  int32_t tot[kPer];
  int32_t sum = 0;
  {
    int32_t h[kXcds][kPer];
#pragma unroll
    for (int b = 0; b < kXcds; ++b)
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int k = tid * kPer + q;
        h[b][q] = k < kOrderBuckets ? g.hist[b * kOrderBuckets + k] : 0;
      }
#pragma unroll
    for (int q = 0; q < kPer; ++q) {
      int32_t pre = 0;
      tot[q] = 0;
#pragma unroll
      for (int b = 0; b < kXcds; ++b) {
        tot[q] += h[b][q];
        pre += b < part ? h[b][q] : 0;
      }
      const int k = tid * kPer + q;
      if (k < kOrderBuckets) start[k] = pre;
      sum += tot[q];
    }
  }
  // Exclusive scan of the per-thread bucket totals (inclusive Hillis-Steele
  // scan, minus the own sum), then each bucket's start.
  run[tid] = sum;
  __syncthreads();
  for (int off = 1; off < nt; off *= 2) {
    const int32_t t = tid >= off ? run[tid - off] : 0;
    __syncthreads();
    run[tid] += t;
    __syncthreads();
  }
  int32_t at = run[tid] - sum;
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int k = tid * kPer + q;
    if (k < kOrderBuckets) {
      start[k] += at;
      at += tot[q];
    }
  }
  __syncthreads();
  constexpr int kU = 8;  // keys per thread per round, their loads issued together
  for (int64_t s0 = s_lo; s0 < s_hi; s0 += int64_t(nt) * kU) {
    int32_t key[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t s = s0 + int64_t(u) * nt + tid;
      key[u] = s < s_hi ? g.keys[s] : -1;
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (key[u] < 0) continue;
      const int64_t s = s0 + int64_t(u) * nt + tid;
      g.order[start[key[u] & ((1 << kKeyRankShift) - 1)] + (key[u] >> kKeyRankShift)] = static_cast<int32_t>(s);
    }
  }
}

// Segment work-groups, the last work-groups of gather_tiles' grid (wid counts
// them from 0; wid % kXcds is the XCD they run on).  Work-group wid runs on
// XCD x = wid % kXcds, is part h = (wid / kXcds) % seg_split of its XCD's
// share, and reads the segment words of the ranges
// [c * blockDim.x / 2, (c + 1) * blockDim.x / 2), c = wid / (kXcds * seg_split),
// which segment_classify wrote before this launch.
// It sums every seg_split-th segment (from h) of column slab x, so each
// XCD's L2 serves one eighth of the dense rows these segments gather.  When
// one slab holds more segments than its work-groups take in two rounds (a
// row far longer than the chunk keeps its chunk inside one slab), the
// chunk's segments are dealt in kXcds * seg_split equal parts of their word
// order instead (part x * seg_split + h).  A lane group stages its segment's sources and
// values in LDS (padded to whole batches with empty positions: value -0,
// zero piece) and streams them as gather_tiles does, so the partial is the
// same fp32 sequence, written to the range's head or tail slot.
template <typename T, typename I>
__device__ void segment_worker(const Geometry<I>& g, int64_t wid, const I* __restrict__ col,
                               const T* __restrict__ value, const T* __restrict__ dense, int64_t K, int64_t N,
                               int64_t ld, float* __restrict__ ws, int64_t slot, int log2L, int64_t chunks,
                               unsigned char* smem) {
  constexpr int V = LaneVec<T>::V;
  constexpr int kWaves = kWgThreads / 64;
  static_assert(2 * kSegChunkRanges == kWgThreads, "one segment word per thread");
  // The work-group has gather_tiles' block size (at most kWgThreads, a
  // multiple of 64): its chunk is blockDim.x / 2 ranges, one word per thread.
  const int nthreads = static_cast<int>(blockDim.x);
  const int64_t chunk_ranges = nthreads / 2;
  const int waves = nthreads / 64;
  __shared__ uint32_t s_word[2 * kSegChunkRanges];
  __shared__ int32_t s_item[2 * kSegChunkRanges];
  __shared__ int32_t s_hist[kXcds];
  __shared__ int32_t s_wave[kWaves];
  const int64_t range = g.range, nranges = g.nranges, nnz = g.nnz;
  const int tid = static_cast<int>(threadIdx.x);
  const int lane64 = tid & 63, wave = tid >> 6;
  const int x = static_cast<int>(wid % kXcds);
  const int split = g.seg_split;
  const int h = static_cast<int>((wid / kXcds) % split);
  const int64_t c = wid / (kXcds * split);
  const int64_t w0 = c * (2 * chunk_ranges);
  // Chunks without segments (flag clear) have nothing to do.
  if (g.seg_flag[c] == 0u) return;  // uniform
  const int64_t left = 2 * nranges - w0;
  const int nw = left < 2 * chunk_ranges ? static_cast<int>(left) : nthreads;
  const uint32_t w = tid < nw ? g.seg[w0 + tid] : 0u;
  const bool valid = (w & kSegValid) != 0u;
  const int slab = static_cast<int>((w >> kSegSlabShift) & (kXcds - 1));
  s_word[tid] = w;
  if (tid < kXcds) s_hist[tid] = 0;
  __syncthreads();
  if (valid) atomicAdd(&s_hist[slab], 1);
  __syncthreads();
  int most = 0;
#pragma unroll
  for (int i = 0; i < kXcds; ++i) most = s_hist[i] > most ? s_hist[i] : most;
  const int L = 1 << log2L;
  const int groups = nthreads >> log2L;
  const int per_round = static_cast<int>(groups / chunks);
  // Candidates in word order: the segments of slab x, or (parts mode) all.
  const bool by_slab = most <= 2 * split * per_round;
  const bool cand = valid && (!by_slab || slab == x);
  const unsigned long long below = (1ull << lane64) - 1ull;
  const unsigned long long mb = __ballot(cand);
  if (lane64 == 0) s_wave[wave] = __popcll(mb);
  __syncthreads();
  int m = 0, mbefore = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    mbefore += i < wave ? s_wave[i] : 0;
    m += i < waves ? s_wave[i] : 0;
  }
  if (cand) s_item[mbefore + __popcll(mb & below)] = tid;
  // This work-group's segments: candidates first, first + step, ...
  const int parts = kXcds * split;
  const int q = x * split + h;
  const int first = by_slab ? h : static_cast<int>(int64_t(q) * m / parts);
  const int step = by_slab ? split : 1;
  const int n = by_slab ? (m > h ? (m - h + split - 1) / split : 0)
                        : static_cast<int>(int64_t(q + 1) * m / parts) - first;

  __syncthreads();  // s_item complete

  // Lane group g takes pairs (segment, column chunk) g, g + groups, ...; its
  // staging area is its own and the lane group lies inside one wavefront, so
  // staging needs only wavefront-scope ordering, and a wavefront without a
  // pair exits at once.
  const int group = tid >> log2L, lane = tid & (L - 1);
  const int64_t stride = seg_stage_stride(range);
  uint32_t* st_src = reinterpret_cast<uint32_t*>(smem) + group * stride;
  float* st_val = reinterpret_cast<float*>(smem) + (groups + group) * stride;
  const int64_t pairs = int64_t(n) * chunks;
  for (int64_t p = group; p < pairs; p += groups) {
    const int wi = s_item[first + static_cast<int>(p / chunks) * step];
    const uint32_t word = s_word[wi];
    const int64_t j = (w0 + wi) >> 1;
    const int64_t lo = j * range;
    const int64_t hi = lo + range < nnz ? lo + range : nnz;
    const int64_t off = static_cast<int64_t>(word & kSegOffsetMask);
    int64_t s0 = (wi & 1) ? lo + off : lo;
    int64_t s1 = (wi & 1) ? hi : lo + off;
    s1 = s1 < hi ? s1 : hi;
    s0 = s0 < s1 ? s0 : s1;
    const int64_t c0 = ((p % chunks) * L + lane) * V;
    float* dst = ws + (2 * j + (wi & 1)) * slot + c0;
    const int32_t n_pos = static_cast<int32_t>(s1 - s0);
    // segment_classify writes only non-empty segments; an empty one can come
    // only from a word this call did not write (row pointers that do not
    // cover [0, nnz)), and is skipped before any index is formed from it.
    if (n_pos <= 0) continue;
    const int32_t n_pad = (n_pos + kSegGroup - 1) / kSegGroup * kSegGroup;
    const int32_t n_stage = n_pad + (kSegInflight - 1) * kSegBatch;
    // The previous pair's staging reads are done before it is overwritten.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    // kSegStageUnroll positions per lane per round, their loads in flight together.
    for (int32_t i0 = 0; i0 < n_stage; i0 += kSegStageUnroll * L) {
      I cs[kSegStageUnroll];
      T vs[kSegStageUnroll];
#pragma unroll
      for (int u = 0; u < kSegStageUnroll; ++u) {
        // Unconditional loads (clamped into the segment; n_pos >= 1), so no
        // branch separates them.
        const int32_t i = i0 + u * L + lane;
        const int64_t q = s0 + (i < n_pos ? i : n_pos - 1);
        cs[u] = col[q];
        vs[u] = value[q];
      }
#pragma unroll
      for (int u = 0; u < kSegStageUnroll; ++u) {
        const int32_t i = i0 + u * L + lane;
        if (i < n_stage) {
          const uint32_t src =
              i < n_pos ? BufferLoader<T>::stage(static_cast<int64_t>(cs[u]), K, ld) : BufferLoader<T>::kNone;
          st_src[i] = src;
          st_val[i] = src != BufferLoader<T>::kNone ? static_cast<float>(vs[u]) : -0.f;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (n_pos > 0 && c0 < N) {
      const BufferLoader<T> ldr(dense, K, ld, N, c0);
      float acc[V];
#pragma unroll
      for (int i = 0; i < V; ++i) acc[i] = 0.f;
      lanes::raw16_t xb[kSegInflight][kSegBatch];
      float vb[kSegInflight][kSegBatch];
      auto issue = [&](lanes::raw16_t* xs, float* vs, int32_t q) {
#pragma unroll
        for (int u = 0; u < kSegBatch; u += 4) {
          const lanes::raw16_t s4 = *reinterpret_cast<const lanes::raw16_t*>(st_src + q + u);
          const lanes::float4_t v4 = *reinterpret_cast<const lanes::float4_t*>(st_val + q + u);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            xs[u + k] = ldr.load(s4[k]);
            vs[u + k] = v4[k];
          }
        }
      };
      auto consume = [&](const lanes::raw16_t* xs, const float* vs) {
#pragma unroll
        for (int u = 0; u < kSegBatch; ++u) {
          float xf[V];
          LaneVec<T>::unpack(xs[u], xf);
#pragma unroll
          for (int i = 0; i < V; ++i) acc[i] = __builtin_fmaf(vs[u], xf[i], acc[i]);
        }
      };
      // kSegInflight batches in flight: the loads of batch k + kSegInflight - 1
      // are issued before batch k is accumulated.  Batches past n_pad read
      // the empty positions staged after it (no memory access) and are never
      // accumulated.
#pragma unroll
      for (int b = 0; b + 1 < kSegInflight; ++b) issue(xb[b], vb[b], b * kSegBatch);
      for (int32_t q = 0; q < n_pad; q += kSegGroup) {
#pragma unroll
        for (int b = 0; b < kSegInflight; ++b) {
          constexpr int kAhead = kSegInflight - 1;
          issue(xb[(b + kAhead) % kSegInflight], vb[(b + kAhead) % kSegInflight], q + (b + kAhead) * kSegBatch);
          consume(xb[b], vb[b]);
        }
      }
#pragma unroll
      for (int i = 0; i < V; ++i) dst[i] = acc[i];
    }
  }
}

#ifndef SPMM_GATHER_WAVES
#define SPMM_GATHER_WAVES 5
#endif
// Waves per SIMD the register budget of gather_tiles is fitted to:
// SPMM_GATHER_WAVES, or SPMM_SEG_WAVES for the instantiation with segment
// work-groups (buffer loads, no window order, kSegBatch-row batches).
template <typename T, typename I, typename Loader, bool kOrder, bool kSeg>
__global__ __launch_bounds__(kWgThreads) __attribute__((amdgpu_waves_per_eu(kSeg ? SPMM_SEG_WAVES : SPMM_GATHER_WAVES))) void gather_tiles(
    Geometry<I> g, const I* __restrict__ col, const T* __restrict__ value,
    const T* __restrict__ dense, int64_t K, int64_t N, int64_t ld, T* __restrict__ out, float* __restrict__ ws,
    int log2L, int64_t chunks, int64_t ranges_per_tile, int64_t slot, int wg_split, int64_t tiles,
    int64_t tiles_per_group) {
  constexpr int V = LaneVec<T>::V;
  extern __shared__ __align__(16) unsigned char smem[];
  // The tile's positions plus a halo of one range: a short row that starts
  // in the tile's last range is finished from the halo.
  const int64_t tile_positions = (ranges_per_tile + 1) * g.range;
  const Staged<T> sa(smem, tile_positions);
  // Per range boundary k of the tile (position P0 + k*R, k = 0..ranges):
  //  s_cut[k]:  end (relative to P0) of the short row crossing it, or -1;
  //  s_long[k]: the long row crossing it, or -1.
  //  s_long_a[k]: that long row's first position.
  __shared__ int32_t s_cut[kTileRanges + 1];
  __shared__ int64_t s_long[kTileRanges + 1];
  __shared__ int64_t s_long_a[kTileRanges + 1];

  // XCD-aware tile order: the XCD of work-group g (g % kXcds) takes column
  // part g % kXcds % wg_split of a contiguous run of tiles, so neighbouring
  // tiles, whose rows tend to share dense rows, share an L2, and with
  // wg_split > 1 each XCD's L2 serves one column chunk of the dense rows.
  // With a window order to write (kOrder: a separate instantiation, so the
  // plain gather keeps its register budget), work-groups [0, kXcds) come
  // first and write the windows' sort keys while the gathers run.
  // With segment words (dense operands within the buffer limit only), the
  // segment work-groups follow the tiles in the grid.
  int64_t bid = static_cast<int64_t>(blockIdx.x);
  static_assert(!kSeg || (std::is_same<Loader, BufferLoader<T>>::value && !kOrder), "segments: buffer loads only");
  if constexpr (kSeg) {
    if (bid >= g.tile_blocks) {
      segment_worker<T, I>(g, bid - g.tile_blocks, col, value, dense, K, N, ld, ws, slot, log2L, chunks, smem);
      return;
    }
  }
  if constexpr (kOrder) {
    if (bid < kXcds) {
      window_keys(g, bid, reinterpret_cast<int32_t*>(smem));
      return;
    }
    bid -= kXcds;
  }
  const int64_t xcd = bid % kXcds;
  const int64_t part = xcd % wg_split;
  const int64_t idx = bid / kXcds;
  const int64_t tile = ((idx / kXcdRun) * (kXcds / wg_split) + xcd / wg_split) * kXcdRun + idx % kXcdRun;
  if (tile >= tiles) return;  // uniform over the work-group, before any barrier
  const int64_t j0 = tile * ranges_per_tile;
  const int64_t j1 = (j0 + ranges_per_tile < g.nranges) ? j0 + ranges_per_tile : g.nranges;
  const int64_t P0 = g.lo(j0), P1 = g.hi(j1 - 1);
  const int64_t base = g.rp(g.row_lo), end = g.rp(g.row_hi);

  // Stage the tile's nonzeros (positions clamped to [0, nnz); those outside
  // our rows are never read): loader source per column (checked against K
  // once here), value bits (-0 for an invalid column) and cleared marks
  // (cleared by the search wavefront instead when it marks the rows), while
  // the row search below runs.
  const int64_t nr = j1 - j0;
  if (threadIdx.x <= nr) {
    s_cut[threadIdx.x] = -1;
    s_long[threadIdx.x] = -1;
  }
  // rS: the row holding position P0 (tiles starting outside our positions
  // [base, end) clamp to the row range); runs of empty rows before the tile
  // are skipped.  It comes from a row search (or, kSeg, from tile_row,
  // clamped to the row range: row pointers that decrease leave entries
  // unwritten).  The search runs in wavefront 0 alone while the other
  // wavefronts stage, when they can stage the tile in one round: its probes
  // then do not wait behind staging loads of its own (loads return in order).
  // Otherwise every wavefront runs it, overlapping its own staging loads.
  int64_t rS = g.row_hi;
  if constexpr (kSeg)
    rS = P0 < base ? g.row_lo : (P0 < end ? clampi(g.tile_row[tile], g.row_lo, g.row_hi - 1) : g.row_hi);
  // Mark the last position of every non-empty row that ends in the tile (or
  // its halo); each position is marked only by the row that holds it.  The
  // tile's rows run from rS while they start at or before P1 (the row holding
  // P1 included; later rows start in the next tile), below row_hi.  A short
  // row (at most short_max(R) nonzeros) that crosses a range
  // boundary is owned by the range where it starts: s_cut tells that range
  // how far to run on and the next range where to begin.  A longer row leaves
  // one fp32 partial per range instead (s_long).  Empty rows are left to the
  // post pass.  mark_row handles row r and returns its first position (P1 + 1
  // past the rows).
  auto mark_row = [&](int64_t r) {
    const int64_t a = r < g.row_hi ? g.rp(r) : P1 + 1;
    if (a <= P1) {
      const int64_t b = g.rp(r + 1);
      if (a < b) {
        if (b - 1 >= P0 && b - 1 < P0 + tile_positions && r - rS < (INT32_MAX >> 1) - 1) {
          const uint32_t vp = g.in_block_window(r) ? 1u : 0u;
          sa.mark[b - 1 - P0] = static_cast<uint32_t>((r - rS + 1) << 1) | vp;
        }
        int64_t k = a < P0 ? 0 : (a - P0) / g.range + 1;  // first boundary after a
        if (b - a <= g.short_max) {
          if (k <= nr && P0 + k * g.range < b) s_cut[k] = static_cast<int32_t>(b - P0);
        } else {
          for (; k <= nr && P0 + k * g.range < b; ++k) {
            s_long[k] = r;
            s_long_a[k] = a;
          }
        }
      }
    }
    return a;
  };
  const bool search_wave = !kSeg && blockDim.x >= 128 &&
                           tile_positions <= kStageUnroll * static_cast<int64_t>(blockDim.x - 64);
  __shared__ int64_t s_rS;
  if (search_wave && threadIdx.x < 64) {
    rS = P0 < base ? g.row_lo : (P0 < end ? find_row(g, P0, base, end) : g.row_hi);
    if (threadIdx.x == 0) s_rS = rS;
    // Then the marks, by this wavefront alone while the others stage: it
    // clears every mark of the tile first (the staging leaves them), in
    // program order before its own row marks.
    for (int64_t i = threadIdx.x; i < tile_positions; i += 64) sa.mark[i] = 0u;
    for (int64_t r0 = rS;; r0 += 64) {
      const int64_t a = mark_row(r0 + threadIdx.x);
      if (__ballot(threadIdx.x == 63 && a <= P1) == 0) break;
    }
  } else {
    // The tile's positions from a work-group-uniform base (P0 < nnz), 32-bit
    // offsets clamped to the last position.
    const I* __restrict__ col_t = col + P0;
    const T* __restrict__ value_t = value + P0;
    const uint32_t last = static_cast<uint32_t>(g.nnz - 1 - P0);
    const uint32_t tid = search_wave ? threadIdx.x - 64 : threadIdx.x;
    const uint32_t stagers = search_wave ? blockDim.x - 64 : blockDim.x;
    for (int64_t i0 = 0; i0 < tile_positions; i0 += kStageUnroll * stagers) {
      I cs[kStageUnroll];
      T vs[kStageUnroll];
      // The stager count through an empty asm: offsets recomputed per round
      // rather than hoisted out of the loop (where they would hold
      // kStageUnroll address registers each and spill).
      uint32_t bd = stagers;
      __asm__ volatile("" : "+s"(bd));
#pragma unroll
      for (int k = 0; k < kStageUnroll; ++k) {
        if (i0 + k * bd < tile_positions) {  // uniform over the stagers
          uint32_t o = static_cast<uint32_t>(i0 + k * bd + tid);
          o = o < last ? o : last;
          cs[k] = col_t[o];
          vs[k] = value_t[o];
        }
      }
      if constexpr (!kSeg)
        if (i0 == 0 && !search_wave) rS = P0 < base ? g.row_lo : (P0 < end ? find_row(g, P0, base, end) : g.row_hi);
#pragma unroll
      for (int k = 0; k < kStageUnroll; ++k) {
        const int64_t i = i0 + k * bd + tid;
        if (i < tile_positions) {
          const uint32_t src = Loader::stage(static_cast<int64_t>(cs[k]), K, ld);
          sa.src[i] = src;
          if (!search_wave) sa.mark[i] = 0u;
          sa.val[i] = src != Loader::kNone ? value_bits<T>(vs[k]) : kNegZero<T>;
        }
      }
    }
  }
  __syncthreads();
  if (search_wave) {
    rS = s_rS;
  } else {
    for (int64_t r0 = rS;; r0 += blockDim.x) {
      const int64_t a = mark_row(r0 + threadIdx.x);
      // Another chunk of rows when the chunk's last row still belongs to the tile.
      if (!__syncthreads_or(threadIdx.x == blockDim.x - 1 && a <= P1)) break;
    }
  }

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
  int32_t ps = cut_in >= 0 ? cut_in : static_cast<int32_t>((lo > base ? lo : base) - P0);
  int32_t pe = cut_out >= 0 ? cut_out : static_cast<int32_t>((hi < end ? hi : end) - P0);
  // Long rows crossing the range's ends: hrow crosses lo (the range starts
  // inside it), trow crosses hi; the tail row is trow when it starts here.
  // Segments left to the segment work-groups are skipped here: the range
  // then starts after the head segment and ends before the tail segment.
  const int64_t hrow = s_long[j - j0], trow = s_long[j - j0 + 1];
  const bool t_here = trow >= 0 && s_long_a[j - j0 + 1] >= lo;
  const uint32_t h_word = kSeg && hrow >= 0 ? g.seg[2 * j] : 0u;
  const uint32_t t_word = kSeg && t_here ? g.seg[2 * j + 1] : 0u;
  if (h_word != 0u) ps = static_cast<int32_t>(lo + (h_word & kSegOffsetMask) - P0);
  if (t_word != 0u) pe = static_cast<int32_t>(lo + (t_word & kSegOffsetMask) - P0);
  // A word's offset lies inside its range; one that does not (a workspace
  // another call overwrote) must still not run past the staged positions.
  if (kSeg && pe > tile_positions) pe = static_cast<int32_t>(tile_positions);
  if (reporter) g.tail[j] = t_here ? trow : -1;
  if (ps >= pe || c0 >= N) return;

  Sink<T> sk;
  sk.rS = rS;
  sk.row_hi = g.row_hi;
  sk.out = out;
  sk.N = N;
  sk.ld = ld;
  sk.c0 = c0;
  sk.vpart = g.vpart;
  sk.head_slot = ws + (2 * j) * slot + c0;
  sk.tail_slot = ws + (2 * j + 1) * slot + c0;
  // The first row began before the range when a long row crosses its start
  // (and its head segment stays here).
  sk.head = cut_in < 0 && lo > base && hrow >= 0 && h_word == 0u;
#pragma unroll
  for (int i = 0; i < V; ++i) sk.acc[i] = 0.f;

  // Two batches of kB dense rows in flight: the loads of the next batch
  // are issued before a batch is accumulated.  The first batch (kB-aligned
  // start, positions before ps masked) and the last two are issued masked;
  // the steady-state loop only issues batches wholly inside [ps, pe).
  constexpr int kB = kSeg ? kSegBatch : kBatch;
  const Stream<T, Loader> st{sa, Loader(dense, K, ld, N, c0), ps, pe};
  int32_t p = ps & ~(kB - 1);
  Batch<T, kB> A, B;
  st.template issue<true>(A, p);
  for (; p + 3 * kB <= pe; p += 2 * kB) {
    st.template issue<false>(B, p + kB);
    sk.consume(A);
    st.template issue<false>(A, p + 2 * kB);
    sk.consume(B);
  }
  // A holds batch p; at most two more batches start before pe.
  if (p + kB < pe) {
    st.template issue<true>(B, p + kB);
    sk.consume(A);
    if (p + 2 * kB < pe) {
      st.template issue<true>(A, p + 2 * kB);
      sk.consume(B);
      sk.consume(A);
    } else {
      sk.consume(B);
    }
  } else {
    sk.consume(A);
  }
  sk.finish(sa.mark[pe - 1] == 0u);
}

// Post pass, one launch:
//  * with a window order to write (g.order), work-groups [0, kXcds) scatter
//    one share of the windows each into the order (scatter_share; LDS:
//    kOrderBuckets + kWgThreads int32), and the classes below follow;
//  * work-groups [0, fix_blocks): add the partials of every row that crosses
//    range ends, in range order (lane group per (range, column chunk));
//  * the next zero_blocks: zero the block kernel's window counters (mixed
//    operator), which that kernel expects at zero, and clear the chunk
//    flags of the segment work-groups for the next call;
//  * the rest: empty rows, 64 per wavefront, are written as zeros (rows of
//    block windows with blocks are left to the block kernel).
template <typename T, typename I>
__global__ __launch_bounds__(kWgThreads) void gather_post(Geometry<I> g, int64_t N, int64_t ld, T* __restrict__ out,
                                                          const float* __restrict__ ws, int log2L,
                                                          int64_t chunks, int64_t slot, int64_t fix_blocks,
                                                          uint32_t* zero_counts, int64_t count, int64_t zero_blocks) {
  constexpr int V = LaneVec<T>::V;
  int64_t bid = static_cast<int64_t>(blockIdx.x);
  if (g.order != nullptr) {
    if (bid < kXcds) {
      extern __shared__ __align__(16) unsigned char smem[];
      int32_t* start = reinterpret_cast<int32_t*>(smem);
      scatter_share(g, bid, start, start + kOrderBuckets);
      return;
    }
    bid -= kXcds;
  }
  if (bid >= fix_blocks && bid < fix_blocks + zero_blocks) {
    const int64_t i = (bid - fix_blocks) * blockDim.x + threadIdx.x;
    if (i < count) zero_counts[i] = 0u;
    if (g.seg != nullptr && i < g.seg_chunks) g.seg_flag[i] = 0u;
    return;
  }
  if (bid < fix_blocks) {
    const int L = 1 << log2L;
    const int64_t tid = bid * blockDim.x + threadIdx.x;
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
      LaneVec<T>::store(out + r * ld + c0, acc);
    }
    return;
  }
  // Empty rows: wavefront w takes rows [row_lo + 64w, +64).
  const int lane = threadIdx.x & 63;
  const int64_t wave =
      (bid - fix_blocks - zero_blocks) * (blockDim.x >> 6) + (threadIdx.x >> 6);
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
      LaneVec<T>::store(out + rr * ld + c0, z);
    }
  }
}

// Gather-rate probe (measurement only, never part of an SpMM): the dense-row
// gathers of gather_tiles over the same nonzeros and ranges -- staged column
// ids and values, one raw buffer load of 16 bytes per lane per nonzero, two
// batches of 4 in flight, fp32 FMAs -- without the row search, marks,
// partial sums or output rows.  Each thread writes its sum to sink (so the
// loads stay live).  Its time bounds what the gather path can reach on the
// input: the ceiling bench.py reports beside the SpMM's rate.
template <typename T>
__global__ __launch_bounds__(kWgThreads) void gather_probe(const int32_t* __restrict__ col,
                                                           const T* __restrict__ value, int64_t nnz,
                                                           const T* __restrict__ dense, int64_t K, int64_t N,
                                                           int log2L, int64_t range, float* __restrict__ sink) {
  constexpr int V = LaneVec<T>::V;
  extern __shared__ __align__(16) unsigned char smem[];
  const int64_t groups = static_cast<int64_t>(blockDim.x) >> log2L;
  const int64_t tile_positions = groups * range;
  const Staged<T> sa(smem, tile_positions);
  const int64_t P0 = static_cast<int64_t>(blockIdx.x) * tile_positions;
  for (int64_t i0 = 0; i0 < tile_positions; i0 += kStageUnroll * blockDim.x) {
    int32_t cs[kStageUnroll];
    T vs[kStageUnroll];
#pragma unroll
    for (int k = 0; k < kStageUnroll; ++k) {
      const int64_t p = P0 + i0 + k * blockDim.x + threadIdx.x;
      cs[k] = p < nnz ? col[p] : -1;
      vs[k] = p < nnz ? value[p] : static_cast<T>(0);
    }
#pragma unroll
    for (int k = 0; k < kStageUnroll; ++k) {
      const int64_t i = i0 + k * blockDim.x + threadIdx.x;
      if (i < tile_positions) {
        const uint32_t src = BufferLoader<T>::stage(static_cast<int64_t>(cs[k]), K, N);
        sa.src[i] = src;
        sa.mark[i] = 0u;
        sa.val[i] = src != BufferLoader<T>::kNone ? value_bits<T>(vs[k]) : kNegZero<T>;
      }
    }
  }
  __syncthreads();
  const int group = threadIdx.x >> log2L;
  const int lane = threadIdx.x & ((1 << log2L) - 1);
  const int32_t ps = static_cast<int32_t>(group * range);
  const int64_t left = nnz - P0 - ps;
  const int32_t pe = ps + static_cast<int32_t>(left < range ? left : range);
  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;
  if (left > 0 && static_cast<int64_t>(lane) * V < N) {
    const Stream<T, BufferLoader<T>> st{sa, BufferLoader<T>(dense, K, N, N, static_cast<int64_t>(lane) * V), ps, pe};
    auto consume = [&](const Batch<T>& b) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        float x[V];
        LaneVec<T>::unpack(b.x[u], x);
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = __builtin_fmaf(b.v[u], x[i], acc[i]);
      }
    };
    int32_t p = ps;
    Batch<T> A, B;
    st.template issue<true>(A, p);
    for (; p + 3 * kBatch <= pe; p += 2 * kBatch) {
      st.template issue<false>(B, p + kBatch);
      consume(A);
      st.template issue<false>(A, p + 2 * kBatch);
      consume(B);
    }
    if (p + kBatch < pe) {
      st.template issue<true>(B, p + kBatch);
      consume(A);
      if (p + 2 * kBatch < pe) {
        st.template issue<true>(A, p + 2 * kBatch);
        consume(B);
        consume(A);
      } else {
        consume(B);
      }
    } else {
      consume(A);
    }
  }
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) sum += acc[i];
  sink[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = sum;
}

// Geometry of the probe launch: lane-group width, ranges per work-group
// (the gather path's R), work-groups and sink floats.
struct ProbeGeometry {
  int log2L = 0;
  int64_t range = 0, groups = 0, blocks = 0;
  ProbeGeometry(int64_t nnz, int64_t N, int64_t elem_bytes) {
    const int64_t lanes_needed = N / (16 / elem_bytes);
    while ((int64_t(1) << log2L) < lanes_needed && log2L < 6) ++log2L;
    range = gather_range(nnz);
    groups = kWgThreads >> log2L;
    blocks = nnz > 0 ? ceil_div(ceil_div(nnz, range), groups) : 0;
  }
  int64_t sink_floats() const { return blocks * kWgThreads; }
};

template <typename T>
spmm_status probe_typed(const void* col, const void* value, int64_t nnz, const void* dense, int64_t K, int64_t N,
                        float* sink, hipStream_t stream) {
  const ProbeGeometry pg(nnz, N, sizeof(T));
  if (pg.blocks == 0) return SPMM_OK;
  if (N > (int64_t(16) << 6) / static_cast<int64_t>(sizeof(T)))
    return fail(SPMM_ERR_CONTRACT, "spmm_gather_probe: rows wider than 64 lanes");
  if (buffer_extent(K, N, N, sizeof(T)) > kBufferLimit)
    return fail(SPMM_ERR_CONTRACT, "spmm_gather_probe: dense operand beyond 4 GB");
  const size_t lds = static_cast<size_t>(pg.groups * pg.range) * Staged<T>::bytes_per_position();
  hipLaunchKernelGGL((gather_probe<T>), dim3(static_cast<unsigned>(pg.blocks)), dim3(kWgThreads), lds, stream,
                     static_cast<const int32_t*>(col), static_cast<const T*>(value), nnz,
                     static_cast<const T*>(dense), K, N, pg.log2L, pg.range, sink);
  return check_launch("gather_probe");
}

// Compute units of the current device (read once per device; 256 on MI355X,
// used when the query fails).
int64_t device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  if (dev >= 0 && dev < kMaxDevices) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (dev < 0 || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev >= 0 && dev < kMaxDevices) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

template <typename T, typename I>
spmm_status gather_typed(const void* rowptr, const void* col, const void* value, int64_t nnz,
                         int64_t vrows, int64_t row_lo, int64_t row_hi, const void* dense, int64_t K,
                         int64_t N, int64_t ld, void* out, void* ws, size_t ws_bytes, const void* Crowptr,
                         int64_t cwin, int64_t climit, float* vpart, const void* Ccol, int32_t* order,
                         uint32_t* zero_counts, int64_t count, hipStream_t stream) {
  constexpr int V = LaneVec<T>::V;
  if (row_hi <= row_lo) return SPMM_OK;
  Geometry<I> g;
  g.rowptr = static_cast<const I*>(rowptr);
  g.row_lo = row_lo;
  g.row_hi = row_hi;
  g.vrows = vrows;
  g.nnz = nnz < 0 ? 0 : nnz;
  g.range = gather_range(g.nnz);
  g.short_max = short_max(g.range);
  g.nranges = g.nnz > 0 ? ceil_div(g.nnz, g.range) : 1;
  g.Crowptr = static_cast<const I*>(Crowptr);
  g.cwin = Crowptr ? cwin : 0;
  g.climit = climit;
  g.vpart = vpart;
  g.Ccol = static_cast<const I*>(Ccol);
  g.K = K;
  // `order` holds order_words(cwin) int32: the order, the windows' keys, the
  // shares' histograms and local-window counts.
  g.order = Crowptr && cwin > 0 && cwin <= kOrderMaxWindows && nnz > 0 ? order : nullptr;
  g.keys = g.order != nullptr ? g.order + cwin : nullptr;
  g.hist = g.order != nullptr ? g.keys + cwin : nullptr;
  g.nlocal = g.order != nullptr ? g.hist + kXcds * kOrderBuckets : nullptr;

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
    wg_split = static_cast<int>(chunks);  // 2: lanes_needed <= 128 and L = 64 for the widest rows
  }
  int64_t ranges_per_tile = (kWgThreads / L) / (chunks / wg_split);
  if (ranges_per_tile > kTileRanges) ranges_per_tile = kTileRanges;
  if (ranges_per_tile < 1) ranges_per_tile = 1;
  // The mixed operator's vector part often runs as one round of tiles, all
  // resident at once, and each CU's gathers are bound by the CU itself: the
  // CUs holding one tile more than the rest finish last (config 3 at N=128:
  // 933 tiles on 256 CUs, 4 on 165 of them, ending 6 us after those with 3).
  // Fewer ranges per tile are taken when that cuts the busiest CU's ranges
  // (tiles per CU, rounded up, times ranges per tile) by at least 5%; not
  // with column-split tiles (two work-groups per tile: config 3 at N=256
  // measured slower).  Results do not depend on the tiling.
  if (g.cwin > 0 && wg_split == 1 && ranges_per_tile >= 8 && g.nnz > 0) {
    const int64_t cus = device_cus();
    auto units = [&](int64_t r) { return ceil_div(ceil_div(g.nranges, r), cus) * r; };
    const int64_t full = units(ranges_per_tile);
    int64_t best = ranges_per_tile, best_units = full;
    for (int64_t r = ranges_per_tile - 1; r >= ranges_per_tile / 2; --r)
      if (units(r) < best_units) {
        best_units = units(r);
        best = r;
      }
    if (best_units * 20 <= full * 19) ranges_per_tile = best;
  }
  const int64_t groups_per_wg = ranges_per_tile * (chunks / wg_split);
  const int64_t wg_threads = groups_per_wg * L;
  const int64_t slot = gather_slot_floats(N);

  // Workspace: tail rows, the partial slots, the segment words, the chunk
  // flags of the segment work-groups, then the tiles' first rows (256-byte
  // aligned pieces).
  const size_t tail_bytes = align_up(static_cast<size_t>(g.nranges) * sizeof(int64_t), 256);
  const size_t partial_bytes = static_cast<size_t>(2 * g.nranges) * slot * sizeof(float);
  const size_t seg_bytes = align_up(static_cast<size_t>(2 * g.nranges) * sizeof(uint32_t), 256);
  const size_t flag_bytes = align_up(static_cast<size_t>(g.nranges) * sizeof(uint32_t), 256);
  const size_t need = tail_bytes + partial_bytes + seg_bytes + flag_bytes + static_cast<size_t>(g.nranges) * sizeof(int64_t);
  if (ws == nullptr || ws_bytes < need)
    return fail(SPMM_ERR_CONTRACT, "gather workspace too small: need " + std::to_string(need) +
                                       " bytes, got " + std::to_string(ws_bytes));
  g.tail = static_cast<int64_t*>(ws);
  float* partial = reinterpret_cast<float*>(static_cast<char*>(ws) + tail_bytes);

  // Dense operands within a 32-bit byte extent use buffer loads.
  const int64_t extent = buffer_extent(K, ld, N, sizeof(T));
  const bool buffer = extent <= kBufferLimit;
  // Segment work-groups for spmm_csr on large matrices whose dense operand
  // is at most kSegMaxDenseBytes (an XCD's column slab of it then stays near
  // its L2).  The vector part of the mixed operator holds the rows the cost
  // model left to the vector engine, and its calls are not worth the extra
  // classification launch (config 3's mixed op +5 us, no wide rows).
  // Their work-groups have gather_tiles' block size, which must hold whole
  // wavefronts (narrow rows give smaller tiles); chunks, ranges and tiles
  // span powers of two (segment_classify works with shifts).
  auto log2_of = [](int64_t v) {
    int l = 0;
    while ((int64_t(1) << l) < v) ++l;
    return l;
  };
  g.seg_chunk = wg_threads / 2;
  g.seg_chunk_log2 = log2_of(g.seg_chunk);
  g.range_log2 = log2_of(g.range);
  g.tile_shift = log2_of(ranges_per_tile * g.range);
  const bool pow2 = (int64_t(1) << g.seg_chunk_log2) == g.seg_chunk && (int64_t(1) << g.range_log2) == g.range &&
                    (int64_t(1) << g.tile_shift) == ranges_per_tile * g.range;
  const bool seg_on = g.cwin == 0 && g.nnz >= kSegMinNnz && K > 0 && buffer && extent <= kSegMaxDenseBytes &&
                      wg_threads % 64 == 0 && pow2;
  g.seg = seg_on ? reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + tail_bytes + partial_bytes) : nullptr;
  g.seg_flag = seg_on ? reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + tail_bytes + partial_bytes + seg_bytes)
                      : nullptr;
  g.tile_row = seg_on ? reinterpret_cast<int64_t*>(static_cast<char*>(ws) + tail_bytes + partial_bytes + seg_bytes +
                                                    flag_bytes)
                      : nullptr;
  g.seg_chunks = seg_on ? ceil_div(g.nranges, g.seg_chunk) : 0;
  g.seg_split = seg_split_for(chunks, L);
  g.slab_scale = K > 0 ? static_cast<float>(static_cast<double>(kXcds) / static_cast<double>(K)) : 0.f;
  g.tile_blocks = 0;

  if (g.nnz > 0) {
    const int64_t tiles = ceil_div(g.nranges, ranges_per_tile);
    size_t lds = static_cast<size_t>((ranges_per_tile + 1) * g.range) * Staged<T>::bytes_per_position();
    if (g.order && lds < kOrderBuckets * sizeof(int32_t)) lds = kOrderBuckets * sizeof(int32_t);  // window_keys' histogram
    auto kernel = seg_on ? gather_tiles<T, I, BufferLoader<T>, false, true>
                  : g.order ? (buffer ? gather_tiles<T, I, BufferLoader<T>, true, false>
                                      : gather_tiles<T, I, GlobalLoader<T>, true, false>)
                            : (buffer ? gather_tiles<T, I, BufferLoader<T>, false, false>
                                      : gather_tiles<T, I, GlobalLoader<T>, false, false>);
    // kXcds / wg_split groups of XCDs take runs of kXcdRun tiles in turn.
    if (kXcds % wg_split != 0) return fail(SPMM_ERR_CONTRACT, "gather: column split does not divide the XCDs");
    const int64_t groups = kXcds / wg_split;
    const int64_t tiles_per_group = ceil_div(tiles, groups * kXcdRun) * kXcdRun;
    g.tile_blocks = kXcds * tiles_per_group + (g.order ? kXcds : 0);
    int64_t blocks = g.tile_blocks;
    if (seg_on) {
      // Segment words and tile rows first, then the tiles with the segment
      // work-groups after them in the same grid (a multiple of kXcds
      // work-groups precedes them, so work-group b of them runs on XCD
      // b % kXcds).
      hipLaunchKernelGGL((segment_classify<I>), dim3(static_cast<unsigned>(ceil_div(row_hi - row_lo, kWgThreads))),
                         dim3(kWgThreads), 0, stream, g, static_cast<const I*>(col));
      if (spmm_status st = check_launch("segment_classify")) return st;
      blocks += kXcds * g.seg_split * g.seg_chunks;
      const size_t seg_lds =
          static_cast<size_t>(wg_threads >> log2L) * seg_stage_stride(g.range) * 2 * sizeof(uint32_t);
      if (lds < seg_lds) lds = seg_lds;
    }
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(static_cast<unsigned>(wg_threads)), lds, stream, g,
                       static_cast<const I*>(col), static_cast<const T*>(value),
                       static_cast<const T*>(dense), K, N, ld, static_cast<T*>(out), partial, log2L,
                       chunks, ranges_per_tile, slot, wg_split, tiles, tiles_per_group);
    if (spmm_status st = check_launch("gather_tiles")) return st;
  }
  const int64_t fix_items = g.nnz > 0 ? (g.nranges - 1) * chunks * L : 0;
  const int64_t fix_blocks = ceil_div(fix_items, kWgThreads);
  const int64_t row_blocks = ceil_div(ceil_div(row_hi - row_lo, 64), kWgThreads / 64);
  const int64_t zero_items = (zero_counts != nullptr ? count : 0) > g.seg_chunks ? count : g.seg_chunks;
  const int64_t zero_blocks = ceil_div(zero_items, kWgThreads);
  const int64_t order_blocks = g.order != nullptr ? kXcds : 0;
  const size_t post_lds = g.order != nullptr ? (kOrderBuckets + kWgThreads) * sizeof(int32_t) : 0;
  hipLaunchKernelGGL((gather_post<T, I>),
                     dim3(static_cast<unsigned>(order_blocks + fix_blocks + zero_blocks + row_blocks)),
                     dim3(kWgThreads), post_lds, stream, g, N, ld, static_cast<T*>(out),
                     static_cast<const float*>(partial), log2L, chunks, slot, fix_blocks, zero_counts, count,
                     zero_blocks);
  return check_launch("gather_post");
}

}  // namespace

size_t gather_workspace_bytes(int64_t nnz, int64_t width) {
  const int64_t nr = (nnz > 0 ? ceil_div(nnz, gather_range(nnz)) : 1);
  return align_up(static_cast<size_t>(nr) * sizeof(int64_t), 256) +
         static_cast<size_t>(2 * nr) * gather_slot_floats(width) * sizeof(float) +
         align_up(static_cast<size_t>(2 * nr) * sizeof(uint32_t), 256) + align_up(static_cast<size_t>(nr) * sizeof(uint32_t), 256) +
         static_cast<size_t>(nr) * sizeof(int64_t);
}

size_t gather_probe_sink_floats(int64_t nnz, int64_t width, int32_t value_type) {
  return static_cast<size_t>(ProbeGeometry(nnz, width, value_type == SPMM_VALUE_F16 ? 2 : 4).sink_floats());
}

spmm_status launch_gather_probe(int32_t value_type, const void* col, const void* value, int64_t nnz,
                                const void* dense, int64_t dense_rows, int64_t width, float* sink,
                                hipStream_t stream) {
  if (value_type == SPMM_VALUE_F16)
    return probe_typed<_Float16>(col, value, nnz, dense, dense_rows, width, sink, stream);
  return probe_typed<float>(col, value, nnz, dense, dense_rows, width, sink, stream);
}

spmm_status launch_gather(int32_t index_type, int32_t value_type, const void* rowptr,
                          const void* col, const void* value, int64_t nnz, int64_t vrows,
                          int64_t row_lo, int64_t row_hi, const void* dense, int64_t dense_rows,
                          int64_t width, int64_t ld, void* out, void* workspace, size_t workspace_bytes,
                          const void* Crowptr, int64_t cwin, int64_t climit, float* vpart,
                          const void* Ccol, int32_t* order, uint32_t* zero_counts, int64_t count,
                          hipStream_t stream) {
#define SPMM_GATHER_CALL(T, I)                                                                 \
  return gather_typed<T, I>(rowptr, col, value, nnz, vrows, row_lo, row_hi, dense, dense_rows, \
                            width, ld, out, workspace, workspace_bytes, Crowptr, cwin, climit, vpart, \
                            Ccol, order, zero_counts, count, stream)
  if (value_type == SPMM_VALUE_F16) {
    if (index_type == SPMM_INDEX_I32) SPMM_GATHER_CALL(_Float16, int32_t);
    SPMM_GATHER_CALL(_Float16, int64_t);
  }
  if (index_type == SPMM_INDEX_I32) SPMM_GATHER_CALL(float, int32_t);
  SPMM_GATHER_CALL(float, int64_t);
#undef SPMM_GATHER_CALL
}

}  // namespace spmm
