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
//    loads, for each of its K-step blocks, C consecutive columns
//    n0 + C*q .. n0 + C*q + C-1 of the block's dense row in one load (fp16:
//    C = 4, 8 bytes, or C = 8, 16 bytes, for outputs of 256 columns or more
//    and of 128 columns on grids of many windows, lane_cols_for; fp32: C = 4,
//    16 bytes).  MFMA j (j < C) takes element j of each load, so
//    its B column q is the dense column n0 + C*q + j.  C MFMAs therefore
//    cover a column group of 16*C columns and the accumulator lane holds C
//    consecutive output columns.  An output element's MFMA sequence is the
//    same for either C.
//  * A work-group first stages its chunk's block sources (each block's dense
//    row offset) in LDS.  The block values stream from memory one K-step at
//    a time beside the dense pieces, and pass through a per-wave LDS ring
//    from which the A fragment A[r][k] = Cvalue[16*(b0+k) + r] is read in
//    the [block][row] layout the reference's converters produce.  Dense
//    pieces are raw buffer loads whose range check turns an invalid or
//    padding block into zeros (no branches; dense operands past 4 GB use
//    64-bit global loads with selects).  With C = 4 the next K-step's loads
//    are issued before the current step's MFMAs, and the accumulators are
//    finished (plus the vector sums, rounded once) straight from registers.
//  * Waves of the work-group take column groups round-robin; each group
//    runs the whole K loop, so every output element sees the same MFMA
//    sequence for every width N.
//  * Windows longer than a chunk (block_chunk_for: 2048 blocks fp16, 1024
//    fp32, growing with the total block count) are cut at fixed block
//    positions: the window's own work-group takes its first chunk, and
//    "overflow" work-groups take the rest in fixed global block ranges (only
//    one window can overflow into a range).  Each
//    piece's work-group stores its fp32 sum and counts itself on the
//    window's counter; the one that completes the count adds the pieces in
//    order (first chunk, then the overflow ranges), so the split is
//    deterministic and needs no combine launch.  The counters start at zero
//    when the gather kernels of the same call ran first (their post pass
//    zeroes them); otherwise (a call with no vector part) the window's own
//    work-group computes the same pieces one after another and adds them in
//    the same order, so no counter and no zeroing launch are needed and the
//    results are the same bit for bit.
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

#include <type_traits>

// Raw buffer loads of 8 and 16 bytes (the LLVM AMDGPU intrinsics): address =
// the resource's base + voffset + soffset, with the resource's range check (a
// load whose offset is past the extent returns zeros).
typedef int spmm_block_rsrc_t __attribute__((ext_vector_type(4)));
typedef int spmm_block_i2_t __attribute__((ext_vector_type(2)));
typedef int spmm_block_i4_t __attribute__((ext_vector_type(4)));
__device__ spmm_block_i2_t spmm_block_buffer_load_b64(spmm_block_rsrc_t rsrc, uint32_t voffset, uint32_t soffset,
                                                      int32_t aux) __asm("llvm.amdgcn.raw.buffer.load.v2i32");
__device__ spmm_block_i4_t spmm_block_buffer_load_b128(spmm_block_rsrc_t rsrc, uint32_t voffset, uint32_t soffset,
                                                       int32_t aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");

namespace spmm {
namespace {

using lanes::LaneVec;
using lanes::clampi;

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// Waves per window work-group: one per column group, up to this many (the
// rest loop), so wide outputs do not lengthen each wave's chain of K-steps.
#ifndef SPMM_BLOCK_MAX_WAVES
#define SPMM_BLOCK_MAX_WAVES 4
#endif
constexpr int kMaxWaves = SPMM_BLOCK_MAX_WAVES;


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
  int64_t K, N, ld;        // N columns computed; dense and out rows are ld elements apart
  T* out;
  const float* vpart;      // [16*windows][N] fp32 vector sums of block-window rows (gather pass)
  float* slots;            // [noverflow][2][16][N] fp32 partials of windows longer than kbig
  uint32_t* cnt;           // [noverflow]: pieces stored so far of the window whose second chunk starts in range k
  int64_t kbig, noverflow, per_xcd;
  int64_t stage;           // blocks staged in LDS at a time (multiple of the K-step)
  int zero_empty;          // no vector part: windows without blocks write their rows as zeros
  int serial;              // counters not zeroed: a long window's own work-group computes every piece
  const int32_t* order;    // locality order of the windows (from the gather post pass), or null

  __device__ inline int64_t crp(int64_t s) const { return clampi(static_cast<int64_t>(Crowptr[s]), 0, limit); }
  __device__ inline int64_t vrp(int64_t r) const {
    return clampi(static_cast<int64_t>(Vrowptr[r < vrows ? r : vrows]), 0, vnnz);
  }
  // Row r has vector-part nonzeros (then the gather pass left their sum in vpart).
  __device__ inline bool row_has_vector(int64_t r) const { return r < vrows && vrp(r) != vrp(r + 1); }
};

// K-step of the MFMA loop: blocks per step (fp16 16x16x32 takes 8 blocks per
// lane group of 16 lanes, fp32 16x16x4 takes 4).
template <typename T>
constexpr int64_t k_step() { return sizeof(T) == 2 ? 32 : 16; }

// Columns a lane holds, C: 4 (an 8-byte fp16 piece or a 16-byte fp32 piece
// of a dense row) or 8 (a 16-byte fp16 piece).  Sixteen lanes cover a column
// group of 16 * C columns, and a K-step runs C MFMAs, one per column of the
// piece.  fp16 takes C = 8 for outputs of at least 256 columns (two or more
// waves per window), and at 128 columns when there are at least
// kWideMinWindows windows: one wave then sums a window's 128 columns, and
// half the waves of C = 4 let every window of a large grid be resident at
// once (config 3, N=128: 35 -> 25 us).  Fewer windows keep C = 4 at 128
// columns, whose two waves per window fill more of the chip (config 2's
// preprocess layout, 687 windows: 110 us with C = 4, 132 us with C = 8).
// The MFMA sequence of an output element does not depend on C.
template <int C>
using half_c = _Float16 __attribute__((ext_vector_type(C)));
constexpr int64_t kWideMinWindows = 2048;
template <typename T>
constexpr int lane_cols_for(int64_t N, int64_t windows) {
  return sizeof(T) == 2 && (N >= 256 || (N >= 128 && windows >= kWideMinWindows)) ? 8 : 4;
}

// The piece of a dense row one lane loads per block.
template <typename T, int C>
using Piece = typename std::conditional<sizeof(T) == 2, half_c<C>, float4_t>::type;

// Dense-piece loaders.  Each stages a 32-bit source per block (in LDS, once
// per chunk) and turns it into the lane's piece of that dense row, or zeros
// for an invalid block column or a padding block.  A lane whose columns lie
// past N reads columns 0 .. C-1 of the same rows instead: MFMA output column
// q depends on B column q only, and those output columns are never stored.
//
// BlockBufferLoader (dense operands up to kBlockBufferLimit bytes): the
// source is the row's byte offset col * N * sizeof(T), read with a raw buffer
// load whose extent is the dense operand; an invalid block stages
// kBlockBufferNone, which with any lane offset (< 4096) lies past the extent,
// so the buffer range check returns zeros without a memory access.  No
// branches and no per-block address arithmetic.
constexpr uint32_t kBlockBufferNone = 0xFFFFF000u;
constexpr int64_t kBlockBufferLimit = kBlockBufferNone;

template <typename T, int C>
struct BlockBufferLoader {
  spmm_block_rsrc_t rsrc;
  uint32_t lane_bytes;
  static constexpr uint32_t kNone = kBlockBufferNone;
  __device__ inline BlockBufferLoader(const T* dense, int64_t K, int64_t ld, int64_t N, int64_t col0) {
    const uint64_t p = reinterpret_cast<uint64_t>(dense);
    rsrc[0] = static_cast<int>(p & 0xFFFFFFFFu);
    rsrc[1] = static_cast<int>((p >> 32) & 0xFFFFu);  // stride 0: raw buffer
    rsrc[2] = static_cast<int>(static_cast<uint32_t>(buffer_extent(K, ld, N, sizeof(T))));
    rsrc[3] = 0x00020000;  // 32-bit data format; no swizzle, no thread-id offset
    lane_bytes = static_cast<uint32_t>(col0 * static_cast<int64_t>(sizeof(T)));
  }
  __device__ static inline uint32_t stage(int64_t c, int64_t K, int64_t ld) {
    return static_cast<uint64_t>(c) < static_cast<uint64_t>(K)
               ? static_cast<uint32_t>(c) * static_cast<uint32_t>(ld * static_cast<int64_t>(sizeof(T)))
               : kNone;
  }
  __device__ inline Piece<T, C> load(uint32_t src) const {
    if constexpr (sizeof(Piece<T, C>) == 8)
      return __builtin_bit_cast(Piece<T, C>, spmm_block_buffer_load_b64(rsrc, src + lane_bytes, 0u, 0));
    else
      return __builtin_bit_cast(Piece<T, C>, spmm_block_buffer_load_b128(rsrc, src + lane_bytes, 0u, 0));
  }
};

// BlockGlobalLoader (larger dense operands): the source is the column id, or
// kBadCol; an invalid block loads dense row 0 (K >= 1 here) and uses zeros.
constexpr uint32_t kBadCol = 0xFFFFFFFFu;

template <typename T, int C>
struct BlockGlobalLoader {
  const T* dense_c;  // dense + the lane's first column
  uint32_t ld;  // row stride of dense (elements)
  static constexpr uint32_t kNone = kBadCol;
  __device__ inline BlockGlobalLoader(const T* dense, int64_t, int64_t ld_, int64_t, int64_t col0)
      : dense_c(dense + col0), ld(static_cast<uint32_t>(ld_)) {}
  __device__ static inline uint32_t stage(int64_t c, int64_t K, int64_t) {
    return static_cast<uint64_t>(c) < static_cast<uint64_t>(K) ? static_cast<uint32_t>(c) : kNone;
  }
  __device__ inline Piece<T, C> load(uint32_t src) const {
    const bool ok = src != kNone;
    const Piece<T, C> x = *reinterpret_cast<const Piece<T, C>*>(dense_c + static_cast<uint64_t>(ok ? src : 0u) * ld);
    return ok ? x : Piece<T, C>(static_cast<T>(0));
  }
};

// LDS staging of one chunk of blocks [b0, b1) (b1 - b0 <= stage): the
// loader's source per block column, checked against K here once, and the 16
// values of every block, loaded with coalesced 16-byte pieces (Cvalue is
// 16-byte aligned by contract).  The chunk is padded to a whole K-step with
// invalid sources and zero values, so the MFMA loop reads LDS without bounds
// checks.  With `finish` set it also returns the window's vector-row bits
// (bit r: row 16*s + r has vector-part nonzeros, whose fp32 sum is in vpart),
// read in the same round trip.
// Row stride of dense and out: a.ld for a column pass of a wider operand
// (kS), else the width itself.  A compile-time choice: the one-pass kernels
// keep the offsets (and registers) of a stride equal to the width.
template <bool kS, typename T, typename I>
__device__ inline int64_t row_stride(const BlockArgs<T, I>& a) {
  return kS ? a.ld : a.N;
}

// LDS staging of one chunk of blocks [b0, b1) (b1 - b0 <= stage): the
// loader's source per block column, checked against K here once.  Loads are
// issued kStageUnroll per thread before any LDS write, so a chunk costs one
// round trip per kStageUnroll * blockDim.x blocks.  The chunk is padded to a
// whole K-step with invalid sources, so the MFMA loop reads LDS without
// bounds checks.  The blocks' values are not staged: each wave streams them
// one K-step at a time (group_sum).  With `finish` set it also returns the
// window's vector-row bits (bit r: row 16*s + r has vector-part nonzeros,
// whose fp32 sum is in vpart), read in the same round trip.
constexpr int kStageUnroll = 2;

template <typename T, typename I, typename Loader, bool kS>
__device__ inline unsigned stage_chunk(const BlockArgs<T, I>& a, int64_t s, bool finish, int64_t b0,
                                       int64_t b1, uint32_t* s_src) {
  __shared__ unsigned s_vec;
  const int64_t n = b1 - b0;
  const int64_t n_pad = (n + k_step<T>() - 1) / k_step<T>() * k_step<T>();
  if (threadIdx.x == 0) s_vec = 0;
  const bool vec = finish && threadIdx.x < 16 && a.row_has_vector(16 * s + threadIdx.x);
  const int64_t nt = blockDim.x;
  for (int64_t i0 = 0; i0 < n_pad; i0 += kStageUnroll * nt) {
    I c[kStageUnroll];
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      const int64_t i = i0 + u * nt + threadIdx.x;
      c[u] = i < n ? a.Ccol[b0 + i] : static_cast<I>(-1);
    }
#pragma unroll
    for (int u = 0; u < kStageUnroll; ++u) {
      const int64_t i = i0 + u * nt + threadIdx.x;
      if (i < n_pad) s_src[i] = i < n ? Loader::stage(static_cast<int64_t>(c[u]), a.K, row_stride<kS>(a)) : Loader::kNone;
    }
  }
  __syncthreads();
  if (vec) atomicOr(&s_vec, 1u << threadIdx.x);
  __syncthreads();
  return s_vec;
}

template <typename T, int C>
__device__ inline void store_cols(T* p, const float* v) {
  if constexpr (sizeof(T) == 2) {
    half_c<C> h;
#pragma unroll
    for (int i = 0; i < C; ++i) h[i] = static_cast<_Float16>(v[i]);
    __builtin_nontemporal_store(h, reinterpret_cast<half_c<C>*>(p));
  } else {
    __builtin_nontemporal_store(float4_t{v[0], v[1], v[2], v[3]}, reinterpret_cast<float4_t*>(p));
  }
}

// One K-step of one lane: its dense pieces (kPieces blocks) and its 16-byte
// piece of the step's block values (a K-step's values are 1 KB for either
// type: 32 fp16 blocks or 16 fp32 blocks of 16 rows; lane l holds bytes
// [16 l, 16 l + 16)).
template <typename T, int C>
struct StepOperands {
  static constexpr int kPieces = sizeof(T) == 2 ? 8 : 4;
  Piece<T, C> x[kPieces];
  lanes::raw16_t v;
};

// Bytes of a wave's ring for the A fragments in LDS: two K-steps of 1 KB.
constexpr size_t kRingBytes = 2 * 1024;

// MFMA sum of staged blocks [0, n) for the column group at n0.  Lane
// (q = lane % 16, kg = lane / 16) loads columns n0 + C*q .. n0 + C*q + C-1
// of its blocks' dense rows with one load per block (16 lanes read
// 16 * C * sizeof(T) contiguous bytes); MFMA j takes element j of each load,
// so its B column q is the dense column n0 + C*q + j and the accumulator lane
// holds C consecutive output columns of rows 4kg .. 4kg+3.  The A fragment
// comes from the blocks' values, `vals` (the chunk's first block), which the
// wave streams one K-step at a time: each lane loads one 16-byte piece of
// the step's 1 KB of values with the step's dense pieces, and at multiply
// time the wave writes the step to its LDS ring and reads the fragment
// A[r][k] = value[16 k + r] back (LDS operations of one wave complete in
// order; the wavefront fence keeps the compiler from moving the reads above
// the write).  The loads of the next K-step are issued before the current
// step's MFMAs (two steps of operands in registers).  Adds to `acc`.
template <typename T, typename I, int C, typename Loader, bool kS>
__device__ inline void group_sum(const BlockArgs<T, I>& a, const uint32_t* s_src, const T* vals,
                                 unsigned char* ring, int64_t n, int64_t n0, int lane, float4_t (&acc)[C]) {
  static_assert(C == 4 || (C == 8 && sizeof(T) == 2), "lane columns: 4, or 8 for fp16");
  const int q = lane & 15, kg = lane >> 4;
  const int64_t col0 = n0 + C * q < a.N ? n0 + C * q : 0;  // N % C == 0
  const Loader ld(a.dense, a.K, row_stride<kS>(a), a.N, col0);
  if (a.K <= 0 || n <= 0) return;  // uniform: no valid dense row
  const int32_t steps = static_cast<int32_t>((n + k_step<T>() - 1) / k_step<T>());
  // 16-byte pieces of the chunk's values; pieces past them (the padding of
  // the last K-step) are zeros.
  const lanes::raw16_t* vpieces = reinterpret_cast<const lanes::raw16_t*>(vals);
  const int64_t vlimit = n * static_cast<int64_t>(sizeof(T));  // 16 values per block: 16 * n * sizeof(T) / 16 pieces

  // fp16: the lane's 8 blocks of a 32-block step are consecutive (8kg ..);
  // fp32: its 4 blocks of a 16-block step are kg, kg+4, kg+8, kg+12.
  auto fetch = [&](StepOperands<T, C>& o, int32_t st) {
    const int64_t piece = static_cast<int64_t>(st) * 64 + lane;
    o.v = piece < vlimit ? vpieces[piece] : lanes::raw16_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int e = 0; e < StepOperands<T, C>::kPieces; ++e) {
      const int32_t blk = sizeof(T) == 2 ? st * 32 + 8 * kg + e : st * 16 + 4 * e + kg;
      o.x[e] = ld.load(s_src[blk]);
    }
  };
  auto multiply = [&](const StepOperands<T, C>& o, int32_t st) {
    lanes::raw16_t* slot = reinterpret_cast<lanes::raw16_t*>(ring + (st & 1) * 1024);
    slot[lane] = o.v;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    const T* sv = reinterpret_cast<const T*>(slot);
    if constexpr (sizeof(T) == 2) {
      half8_t av;
#pragma unroll
      for (int e = 0; e < 8; ++e) av[e] = sv[(8 * kg + e) * 16 + q];
#pragma unroll
      for (int j = 0; j < C; ++j) {
        half8_t b;
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = o.x[e][j];
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, acc[j], 0, 0, 0);
      }
    } else {
      float4_t av;
#pragma unroll
      for (int e = 0; e < 4; ++e) av[e] = sv[(4 * e + kg) * 16 + q];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u], o.x[u][j], acc[j], 0, 0, 0);
      }
    }
  };
  if constexpr (C == 8) {
    // Twice the operands per step: one step in registers (a second would
    // not fit the register budget of 4 waves per SIMD).
    for (int32_t st = 0; st < steps; ++st) {
      StepOperands<T, C> A;
      fetch(A, st);
      multiply(A, st);
    }
    return;
  }
  StepOperands<T, C> A, B;
  fetch(A, 0);
  int32_t st = 0;
  for (; st + 3 <= steps; st += 2) {
    fetch(B, st + 1);
    multiply(A, st);
    fetch(A, st + 2);
    multiply(B, st + 1);
  }
  // A holds step st; one or two steps remain.
  if (st + 2 == steps) {
    fetch(B, st + 1);
    multiply(A, st);
    multiply(B, st + 1);
  } else {
    multiply(A, st);
  }
}

// Bit r set: row 16*s + r has vector-part nonzeros (their fp32 sum is in
// vpart).  All threads of the work-group must call it.
template <typename T, typename I>
__device__ inline unsigned window_vector_rows(const BlockArgs<T, I>& a, int64_t s) {
  __shared__ unsigned s_vec;
  if (threadIdx.x == 0) s_vec = 0;
  __syncthreads();
  if (threadIdx.x < 16 && a.row_has_vector(16 * s + threadIdx.x)) atomicOr(&s_vec, 1u << threadIdx.x);
  __syncthreads();
  return s_vec;
}

// Sums blocks [b0, b1) of window s and, with `slot` null, finishes rows
// 16*s .. 16*s+15 straight from the accumulators: block sum, plus the row's
// vector sum if it has one, rounded once.  With `slot` set, the fp32 block
// sum goes to that [16][N] workspace slot instead.  Blocks are staged in LDS
// `a.stage` at a time (a multiple of the K-step, so the MFMA sequence does
// not depend on it); a window that fits is staged once for all column groups.
template <typename T, typename I, int C, typename Loader, bool kS>
__device__ inline void window_chunk(const BlockArgs<T, I>& a, int64_t s, int64_t b0, int64_t b1,
                                    float* slot, uint32_t* s_col, unsigned char* ring) {
  const int64_t n = b1 - b0;
  const bool once = n <= a.stage;
  unsigned vec = 0;
  if (once)
    vec = stage_chunk<T, I, Loader, kS>(a, s, slot == nullptr, b0, b1, s_col);
  else if (slot == nullptr)
    vec = window_vector_rows(a, s);
  constexpr int64_t kGroupCols = 16 * C;
  T* const out_w = a.out + 16 * s * row_stride<kS>(a);
  const float* const vpart_w = a.vpart + 16 * s * a.N;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int q = lane & 15, kg = lane >> 4;
  const int64_t groups = (a.N + kGroupCols - 1) / kGroupCols;
  // Uniform trip count over the work-group (staging synchronises it).
  for (int64_t gbase = 0; gbase < groups; gbase += waves) {
    const int64_t g = gbase + wave;
    const bool active = g < groups;
    const int64_t n0 = kGroupCols * g;
    float4_t acc[C];
#pragma unroll
    for (int j = 0; j < C; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};
    if (once) {
      if (active) group_sum<T, I, C, Loader, kS>(a, s_col, a.Cvalue + 16 * b0, ring, n, n0, lane, acc);
    } else {
      for (int64_t sb = 0; sb < n; sb += a.stage) {
        const int64_t m = n - sb < a.stage ? n - sb : a.stage;
        __syncthreads();  // the previous piece is no longer read
        stage_chunk<T, I, Loader, kS>(a, s, false, b0 + sb, b0 + sb + m, s_col);
        if (active) group_sum<T, I, C, Loader, kS>(a, s_col, a.Cvalue + 16 * (b0 + sb), ring, m, n0, lane, acc);
      }
    }
    const int64_t c0 = n0 + C * q;
    if (!active || c0 >= a.N) continue;
    // Element offsets inside the window's 16 x N tile (< 2^14) from the
    // window's base pointers, which are uniform: no 64-bit row address per
    // lane stays live across the column-group loop.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * kg + e;
      const uint32_t o = static_cast<uint32_t>(r * a.N + c0);  // in the [16][N] vpart / slot tile
      const uint32_t oo = kS ? static_cast<uint32_t>(r * a.ld + c0) : o;  // in the output window
      float v[C];
#pragma unroll
      for (int j = 0; j < C; ++j) v[j] = acc[j][e];
      if (slot) {
        // Read by another work-group, possibly on another XCD: agent-scope
        // atomic stores, performed coherently across the XCDs' L2s.
#pragma unroll
        for (int w = 0; w < C; w += 2) {
          const uint64_t bits = static_cast<uint64_t>(__float_as_uint(v[w])) |
                                (static_cast<uint64_t>(__float_as_uint(v[w + 1])) << 32);
          __hip_atomic_store(reinterpret_cast<uint64_t*>(slot + o + w), bits, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        }
        continue;
      }
      if (vec >> r & 1u) {
#pragma unroll
        for (int w = 0; w < C; w += 4) {
          const float4_t p = *reinterpret_cast<const float4_t*>(vpart_w + o + w);
#pragma unroll
          for (int i = 0; i < 4; ++i) v[w + i] = v[w + i] + p[i];
        }
      }
      store_cols<T, C>(out_w + oo, v);
    }
  }
}

// Adds the pieces of window s (first chunk in slot (k0, 1), then the
// segments of overflow ranges k0 .. k_end in slot (k, 0)) in that order,
// plus the rows' vector sums, rounds once and writes the window's 16 rows.
// Every piece is stored and performed before any thread of the work-group
// calls it.
template <bool kS, typename T, typename I>
__device__ inline void combine_window(const BlockArgs<T, I>& a, int64_t s, int64_t k0, int64_t k_end) {
  const int64_t n = 16 * a.N;
  auto load4 = [](const float* p) {
    lanes::float4_t f;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint64_t bits = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p) + h, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      f[2 * h] = __uint_as_float(static_cast<uint32_t>(bits));
      f[2 * h + 1] = __uint_as_float(static_cast<uint32_t>(bits >> 32));
    }
    return f;
  };
  // Each thread keeps kIt groups of 4 elements and walks the pieces in order,
  // the next piece's loads in flight while the current one is added: about
  // one round trip per piece.
  constexpr int kIt = 4;
  const int64_t stride = 4 * static_cast<int64_t>(blockDim.x);
  for (int64_t base = 4 * static_cast<int64_t>(threadIdx.x); base < n; base += kIt * stride) {
    lanes::float4_t acc[kIt], nxt[kIt];
#pragma unroll
    for (int t = 0; t < kIt; ++t) {
      const int64_t i = base + t * stride < n ? base + t * stride : base;
      acc[t] = load4(a.slots + (2 * k0 + 1) * n + i);
      nxt[t] = load4(a.slots + (2 * k0) * n + i);
    }
    for (int64_t q = k0; q <= k_end; ++q) {
      lanes::float4_t cur[kIt];
#pragma unroll
      for (int t = 0; t < kIt; ++t) cur[t] = nxt[t];
      if (q < k_end) {
#pragma unroll
        for (int t = 0; t < kIt; ++t) {
          const int64_t i = base + t * stride < n ? base + t * stride : base;
          nxt[t] = load4(a.slots + (2 * (q + 1)) * n + i);
        }
      }
#pragma unroll
      for (int t = 0; t < kIt; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[t][e] = acc[t][e] + cur[t][e];
    }
#pragma unroll
    for (int t = 0; t < kIt; ++t) {
      const int64_t i = base + t * stride;
      if (i >= n) break;
      const int64_t r = i / a.N, c = i - r * a.N;  // 4 elements of one row (N % 4 == 0)
      const int64_t row = 16 * s + r;
      lanes::float4_t v = acc[t];
      if (a.row_has_vector(row)) {
        const lanes::float4_t vp = *reinterpret_cast<const lanes::float4_t*>(a.vpart + row * a.N + c);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = v[e] + vp[e];
      }
      T* dst = a.out + row * row_stride<kS>(a) + c;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = static_cast<T>(v[e]);
    }
  }
}

// A window of blocks [b0, b1), longer than kbig, is summed in pieces: its own
// work-group's first chunk (slot (k0, 1), k0 = (b0 + kbig) / kbig) and one
// segment per overflow range k0 .. k_end (slot (k, 0)).  After storing its
// piece, a work-group counts itself on cnt[k0]; the one that completes the
// count adds first chunk + segments k0, k0+1, ... in order, adds the rows'
// vector sums, rounds once and writes the window's 16 rows, then resets the
// counter to zero for the next call.  With a.serial the window's own
// work-group has stored every piece and adds them without a counter.  All
// threads of the work-group call it.
template <bool kS, typename T, typename I>
__device__ inline void settle_window(const BlockArgs<T, I>& a, int64_t s, int64_t b0, int64_t b1) {
  __shared__ uint32_t s_last;
  const int64_t k0 = (b0 + a.kbig) / a.kbig;
  const int64_t k_end = (b1 - 1) / a.kbig;
  // The pieces are stored and read with agent-scope atomic accesses, which
  // on gfx950 are performed at the device coherence point (write-through
  // stores, loads that bypass non-coherent cache lines).  A wave's vector
  // memory counter reaches zero only when its stores are performed, so
  // after every wave's wait and the barrier, all of this work-group's
  // pieces are visible to any work-group that reads the count.  Agent-scope
  // release/acquire fences would say the same in the HIP memory model, but
  // they write back and invalidate the whole L2 of the XCD per piece: with
  // them config 5's graph path (thousands of pieces) took 18.9 instead of
  // 12.2 ms.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (!a.serial) {
    if (threadIdx.x == 0) {
      const uint32_t old = __hip_atomic_fetch_add(a.cnt + k0, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = static_cast<int64_t>(old) + 1 == k_end - k0 + 2 ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
  }
  combine_window<kS>(a, s, k0, k_end);
  if (!a.serial && threadIdx.x == 0) __hip_atomic_store(a.cnt + k0, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Work-groups [0, 8*per_xcd): window s (XCD-aware runs) computes its first
// kbig blocks; a window with at most kbig blocks is finished here.  A longer
// window leaves its first-chunk sum in slot (k0, 1), k0 = (b0 + kbig) / kbig.
// Work-groups 8*per_xcd + k: overflow range k = blocks [k*kbig, (k+1)*kbig).
// Only the window holding block k*kbig can have blocks past its first chunk
// in that range; that segment's sum goes to slot (k, 0).
#ifndef SPMM_BLOCK_WAVES
#define SPMM_BLOCK_WAVES 4
#endif
#ifndef SPMM_BLOCK_WAVES_WIDE
#define SPMM_BLOCK_WAVES_WIDE 4
#endif
// Waves per SIMD the register budget of block_windows is fitted to (C = 8
// holds twice the accumulators and dense pieces).
// A window that fits one staging piece (the common case) takes the lean
// path with C-column pieces; longer windows and the overflow ranges take
// 4-column pieces (their MFMA sequence per output element is the same, so
// results do not depend on the path), which keeps their chunk loops and
// partial stores out of the lean path's register budget.
template <typename T, typename I, int C, template <typename, int> class LoaderT, bool kS>
__global__ __launch_bounds__(64 * kMaxWaves) __attribute__((amdgpu_waves_per_eu(C == 8 ? SPMM_BLOCK_WAVES_WIDE : SPMM_BLOCK_WAVES))) void block_windows(BlockArgs<T, I> a) {
  extern __shared__ __align__(16) unsigned char smem[];
  // The wave's ring of A fragments (kRingBytes per wave), then the staged
  // column sources ([stage] uint32).
  unsigned char* ring = smem + (threadIdx.x >> 6) * kRingBytes;
  uint32_t* s_col = reinterpret_cast<uint32_t*>(smem + (blockDim.x >> 6) * kRingBytes);
  const int64_t lead = a.per_xcd * kXcds;
  const int64_t g = blockIdx.x;
  const int64_t n16 = 16 * a.N;
  if (g < lead) {
    const int64_t idx = g / kXcds;
    int64_t s = ((idx / kBlockXcdRun) * kXcds + g % kXcds) * kBlockXcdRun + idx % kBlockXcdRun;
    if (s >= a.windows) return;  // uniform over the work-group
    if (a.order != nullptr) {
      // The order is written earlier in the same call; an entry outside
      // [0, windows) (a workspace shared by overlapping calls) is skipped
      // rather than used as an index.
      s = a.order[s];
      if (s < 0 || s >= a.windows) return;  // uniform over the work-group
    }
    const int64_t b0 = a.crp(s);
    int64_t b1 = a.crp(s + 1);
    if (b1 <= b0) {  // empty window: its rows are the vector pass's, or zeros
      if (a.zero_empty) {
        const int64_t per_row = a.N * static_cast<int64_t>(sizeof(T)) / 16;  // 16-byte pieces of a row
        for (int64_t i = threadIdx.x; i < 16 * per_row; i += blockDim.x) {
          const int64_t r = i / per_row;
          reinterpret_cast<lanes::raw16_t*>(a.out + (16 * s + r) * row_stride<kS>(a))[i - r * per_row] =
              lanes::raw16_t{0u, 0u, 0u, 0u};
        }
      }
      return;
    }
    if (b1 - b0 <= a.stage) {
      window_chunk<T, I, C, LoaderT<T, C>, kS>(a, s, b0, b1, nullptr, s_col, ring);
      return;
    }
    const bool single = b1 - b0 <= a.kbig;
    const int64_t k0 = (b0 + a.kbig) / a.kbig;
    // Piece k0 - 1 is the first chunk.  With a.serial, the same work-group
    // then sums the segment of every overflow range k = k0 .. (b1 - 1) / kbig
    // into slot (k, 0): the blocks an overflow work-group would take.
    const int64_t k_last = single || !a.serial ? k0 - 1 : (b1 - 1) / a.kbig;
    for (int64_t k = k0 - 1; k <= k_last; ++k) {
      if (k >= k0) __syncthreads();  // the previous piece's staged columns are no longer read
      const int64_t bk = k * a.kbig;
      const int64_t lo = k < k0 ? b0 : (b0 + a.kbig > bk ? b0 + a.kbig : bk);
      const int64_t hi = k < k0 ? (single ? b1 : b0 + a.kbig) : (b1 < bk + a.kbig ? b1 : bk + a.kbig);
      float* const slot = single ? nullptr : a.slots + (k < k0 ? 2 * k0 + 1 : 2 * k) * n16;
      window_chunk<T, I, 4, LoaderT<T, 4>, kS>(a, s, lo, hi, slot, s_col, ring);
    }
    if (!single) settle_window<kS>(a, s, b0, b1);
    return;
  }
  const int64_t k = g - lead;
  if (k >= a.noverflow) return;
  const int64_t bk = k * a.kbig;
  // s = window holding block bk: last s with crp(s) <= bk.
  int64_t first_above, unused;
  wg_lower_bound2([&](int64_t i) { return a.crp(i); }, 0, a.windows, bk + 1, bk + 1, first_above, unused);
  const int64_t s = first_above - 1;
  const bool valid = s >= 0 && s < a.windows;
  const int64_t b0 = valid ? a.crp(s) : 0, b1 = valid ? a.crp(s + 1) : 0;
  const bool owns = valid && b0 < bk && b1 > b0 + a.kbig;
  if (!owns) return;
  // Every overflow range from the window's second chunk, k0 = (b0 + kbig) /
  // kbig, to (b1 - 1) / kbig holds a non-empty segment of it.
  const int64_t lo = b0 + a.kbig > bk ? b0 + a.kbig : bk;
  const int64_t hi = b1 < bk + a.kbig ? b1 : bk + a.kbig;
  if (lo >= hi) return;
  window_chunk<T, I, 4, LoaderT<T, 4>, kS>(a, s, lo, hi, a.slots + (2 * k) * n16, s_col, ring);
  settle_window<kS>(a, s, b0, b1);
}

template <typename T, typename I>
spmm_status block_typed(const void* Crowptr, const void* Ccol, const void* Cvalue, int64_t windows,
                        int64_t block_count, int64_t block_values, const void* Vrowptr,
                        int64_t vector_rows, int64_t vector_nnz, const void* dense, int64_t K,
                        int64_t N, int64_t ldd, void* out, const float* vpart, float* slots, const int32_t* order,
                        bool counters_zeroed, hipStream_t stream) {
  if (windows <= 0) return SPMM_OK;
  if (K > static_cast<int64_t>(kBadCol) - 1)
    return fail(SPMM_ERR_CONTRACT, "dense has too many rows for 32-bit column ids");
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
  a.ld = ldd;
  a.out = static_cast<T*>(out);
  a.vpart = vpart;
  a.slots = slots;
  a.zero_empty = vector_nnz == 0 ? 1 : 0;
  a.order = order;
  a.serial = counters_zeroed ? 0 : 1;
  a.kbig = block_chunk_for(sizeof(T) == 2 ? SPMM_VALUE_F16 : SPMM_VALUE_F32, a.limit);
  a.noverflow = block_overflow_ranges(a.limit, a.kbig);
  a.cnt = reinterpret_cast<uint32_t*>(slots + a.noverflow * 2 * 16 * N);
  a.per_xcd = ceil_div(windows, kXcds * kBlockXcdRun) * kBlockXcdRun;
  const int C = lane_cols_for<T>(N, windows);
  const int64_t groups = ceil_div(N, 16 * C);
  const int waves = groups < kMaxWaves ? static_cast<int>(groups) : kMaxWaves;
  // Staging piece (4 bytes of LDS per block): about twice the mean window,
  // from 64 blocks up to the chunk, so most windows stage once and LDS per
  // work-group stays small enough for 16 work-groups per CU.
  const int64_t mean = a.limit / windows;
  a.stage = 64;
  while (a.stage < 2 * mean && a.stage < a.kbig) a.stage *= 2;
  const size_t stage_lds = static_cast<size_t>(waves) * kRingBytes + static_cast<size_t>(a.stage) * sizeof(uint32_t);
  // Overflow work-groups only where the counters were zeroed (else each long
  // window's own work-group takes its overflow segments).
  const int64_t grid = a.per_xcd * kXcds + (a.serial ? 0 : a.noverflow);
  constexpr int kWide = sizeof(T) == 2 ? 8 : 4;  // fp32 only has C = 4
  // Dense operands within a 32-bit byte extent use buffer loads.
  const bool buffer = buffer_extent(K, ldd, N, sizeof(T)) <= kBlockBufferLimit;
  // Column passes (ldd > N) take the strided instantiations.
  auto kernel = ldd == N ? (buffer ? (C == 8 ? block_windows<T, I, kWide, BlockBufferLoader, false>
                                            : block_windows<T, I, 4, BlockBufferLoader, false>)
                                   : (C == 8 ? block_windows<T, I, kWide, BlockGlobalLoader, false>
                                             : block_windows<T, I, 4, BlockGlobalLoader, false>))
                         : (buffer ? (C == 8 ? block_windows<T, I, kWide, BlockBufferLoader, true>
                                            : block_windows<T, I, 4, BlockBufferLoader, true>)
                                   : (C == 8 ? block_windows<T, I, kWide, BlockGlobalLoader, true>
                                             : block_windows<T, I, 4, BlockGlobalLoader, true>));
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(64 * waves), stage_lds, stream, a);
  return check_launch("block_windows");
}

}  // namespace

int64_t block_overflow_ranges(int64_t blocks, int64_t kbig) {
  return blocks > kbig ? ceil_div(blocks, kbig) : 0;
}

spmm_status launch_block(int32_t index_type, int32_t value_type, const void* Crowptr,
                         const void* Ccol, const void* Cvalue, int64_t windows,
                         int64_t block_count, int64_t block_values, const void* Vrowptr,
                         int64_t vector_rows, int64_t vector_nnz, const void* dense,
                         int64_t dense_rows, int64_t width, int64_t ld, void* out, const float* vpart,
                         float* slots, const int32_t* order, bool counters_zeroed, hipStream_t stream) {
#define SPMM_BLOCK_CALL(T, I)                                                                   \
  return block_typed<T, I>(Crowptr, Ccol, Cvalue, windows, block_count, block_values, Vrowptr, \
                           vector_rows, vector_nnz, dense, dense_rows, width, ld, out, vpart, slots, \
                           order, counters_zeroed, stream)
  if (value_type == SPMM_VALUE_F16) {
    if (index_type == SPMM_INDEX_I32) SPMM_BLOCK_CALL(_Float16, int32_t);
    SPMM_BLOCK_CALL(_Float16, int64_t);
  }
  if (index_type == SPMM_INDEX_I32) SPMM_BLOCK_CALL(float, int32_t);
  SPMM_BLOCK_CALL(float, int64_t);
#undef SPMM_BLOCK_CALL
}

}  // namespace spmm
