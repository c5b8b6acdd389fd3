// Internal helpers shared by the HIP translation units of libspmm_mi355x.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/spmm_mi355x.h"

namespace spmm {

// Per-thread message of the last failure (spmm_last_error()).
void set_error(const std::string& msg);
void clear_error();

// Records `msg` and returns `code`.
spmm_status fail(spmm_status code, const std::string& msg);

// Converts a HIP error of a launch or runtime call to SPMM_ERR_DEVICE.
spmm_status check_hip(hipError_t err, const char* what);

// Launch-time check: returns the pending launch error (if any) as a status.
spmm_status check_launch(const char* what);

inline hipStream_t as_stream(spmm_stream s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// XCDs of an MI355X.  Work-groups are dispatched round-robin over them, so
// work-group g runs on XCD g % kXcds and shares that XCD's L2 with g +- kXcds.
constexpr int kXcds = 8;

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Bytes a raw buffer resource must span to read `width` columns of each of K
// rows that lie ld elements apart: the last row's slab ends there.
__host__ __device__ inline int64_t buffer_extent(int64_t K, int64_t ld, int64_t width, int64_t elem_bytes) {
  return K > 0 ? ((K - 1) * ld + width) * elem_bytes : 0;
}

// Column passes.  A dense operand much larger than the 256 MB Infinity Cache
// is swept in slabs of `pass_width` columns (rows ld = N apart), one SpMM
// pass per slab: the gathers of a pass then hit a 512 MiB slab instead of the
// whole operand.  Every output element is computed by the same operation
// sequence as in one full-width pass (the kernels' results do not depend on
// the width), so the passes change only the speed: config 5 (1M x 512 fp32,
// 2 GiB) takes 10.4 ms in four passes of 128 columns against 12.3 ms in one.
// Slabs keep at least 512-byte rows (narrower ones were slower there).
constexpr int64_t kPassSlabBytes = int64_t(512) << 20;
constexpr int64_t kPassMinRowBytes = 512;
inline int64_t pass_width(int64_t K, int64_t N, int64_t elem_bytes) {
  int64_t w = N;
  while (w % 32 == 0 && (w / 2) * elem_bytes >= kPassMinRowBytes && K * w * elem_bytes > kPassSlabBytes) w /= 2;
  return w;
}

// Split length R of the CSR gather path: nonzero positions are cut into
// ranges [j*R, (j+1)*R), one lane group per range.  R is the largest power of
// two in [kGatherRangeMin, kGatherRangeMax] with about nnz / R >=
// kGatherSplit ranges, so small matrices still run enough lane groups at once
// to cover memory latency.  It depends on nnz only (not on width or dtype),
// which is what makes the gather results identical for every feature width.
#ifndef SPMM_GATHER_SPLIT
#define SPMM_GATHER_SPLIT 12288
#endif
constexpr int64_t kGatherSplit = SPMM_GATHER_SPLIT;
constexpr int64_t kGatherRangeMin = 16;
constexpr int64_t kGatherRangeMax = 256;
inline int64_t gather_range(int64_t nnz) {
  int64_t r = kGatherRangeMin;
  while (r < kGatherRangeMax && 2 * r * kGatherSplit <= nnz) r *= 2;
  return r;
}

// fp32 storage of one partial row in the gather workspace, padded so every
// slot starts 256-byte aligned.
inline int64_t gather_slot_floats(int64_t width) { return (width + 63) / 64 * 64; }

// ---- internal launchers (defined in the .hip files) ----------------------

// Vector (CSR gather) part over rows [row_lo, row_hi) of the CSR given by
// (rowptr, col, value): rowptr holds vrows + 1 entries (rows >= vrows are
// empty) and col/value hold `nnz`.  Writes every row of [row_lo, row_hi).
// With a block part (Crowptr != nullptr, cwin windows, climit usable blocks),
// the vector sums of rows in block windows with blocks go to `vpart` (fp32)
// instead of `out`, and their empty rows are left to the block kernel.
// `dense` and `out` hold `width` columns per row, rows `ld` elements apart
// (ld >= width: a column slab of wider matrices); vpart rows hold `width`
// floats.  `zero_counts` (count entries, may be null) is zeroed by the post
// pass, for the block kernel that runs next.
spmm_status launch_gather(int32_t index_type, int32_t value_type,
                          const void* rowptr, const void* col, const void* value,
                          int64_t nnz, int64_t vrows, int64_t row_lo, int64_t row_hi,
                          const void* dense, int64_t dense_rows, int64_t width, int64_t ld,
                          void* out, void* workspace, size_t workspace_bytes,
                          const void* Crowptr, int64_t cwin, int64_t climit, float* vpart,
                          const void* Ccol, int32_t* order, uint32_t* zero_counts, int64_t count,
                          hipStream_t stream);

// Locality order of the block windows: with `order` set (order_words(cwin)
// int32), extra work-groups of the gather kernel, running beside the
// gathers, bucket the windows by first block column (kOrderBuckets buckets)
// in kXcds shares, the post pass's first work-groups scatter each share into
// the order, and the block kernel follows that order.  Used for at most kOrderMaxWindows windows,
// dense rows of at least kOrderMinRowBytes (fp16 N >= 128, fp32 N >= 64),
// and a vector part (the gather kernel runs).
constexpr int64_t kOrderMaxWindows = 16384;
constexpr int kOrderBuckets = 1024;
#ifndef SPMM_ORDER_MIN_ROW_BYTES
#define SPMM_ORDER_MIN_ROW_BYTES 256
#endif
constexpr int64_t kOrderMinRowBytes = SPMM_ORDER_MIN_ROW_BYTES;

// Window positions -> XCDs in the block kernel: XCDs take runs of this many
// consecutive positions in turn (work-group g runs on XCD g % kXcds).  Runs
// of 64 against 32: config 3's bcsr op 23.5 -> 22.6 us at N=128, 38.6 -> 38.0
// us at N=256, the mixed ops flat; 8 or 16 are slower, 128 slows the mixed
// ops.
#ifndef SPMM_BLOCK_XCD_RUN
#define SPMM_BLOCK_XCD_RUN 64
#endif
constexpr int64_t kBlockXcdRun = SPMM_BLOCK_XCD_RUN;

// int32 words of the order workspace for `windows` windows: the order, one
// key per window, a histogram per XCD share and a local-window count per share.
inline int64_t order_words(int64_t windows) { return 2 * windows + kXcds * (kOrderBuckets + 1); }

inline bool block_order_wanted(int64_t windows, int64_t vector_nnz, int64_t width, int32_t value_type) {
  const int64_t row_bytes = width * (value_type == SPMM_VALUE_F16 ? 2 : 4);
  return windows > 0 && windows <= kOrderMaxWindows && vector_nnz > 0 && row_bytes >= kOrderMinRowBytes;
}

// Gather-rate probe (measurement): the gather path's dense-row loads over
// the same nonzeros, without rows or output; int32 column ids.
size_t gather_probe_sink_floats(int64_t nnz, int64_t width, int32_t value_type);
spmm_status launch_gather_probe(int32_t value_type, const void* col, const void* value, int64_t nnz,
                                const void* dense, int64_t dense_rows, int64_t width, float* sink,
                                hipStream_t stream);

// Thread-per-row scalar CSR baseline over rows [0, rows) (no workspace).
spmm_status launch_rowscalar(int32_t index_type, int32_t value_type, const void* rowptr, const void* col,
                             const void* value, int64_t rows, int64_t nnz, const void* dense, int64_t K,
                             int64_t N, void* out, hipStream_t stream);

// Workspace bytes launch_gather may use for at most `nnz` vector nonzeros.
size_t gather_workspace_bytes(int64_t nnz, int64_t width);

// Blocks of a window handled by one work-group before the window is split
// into chunks that separate work-groups sum and the last of them adds in
// order.  Large enough that ordinary windows are never split (each overflow
// range costs a work-group and a window search), and growing with the total
// block count (at most about 16384 chunks, 4096 blocks per chunk at most),
// so large inputs keep the partial sums (and their workspace) small; it
// depends on the value type and the block count only, never on the width,
// so results do not depend on the width.  fp32 keeps 1024: the split also
// bounds the fp32 accumulation chain of hub rows (config 5's rows of 8192
// nonzeros miss the 1e-4 tolerance in 44 of 35M sampled elements with 4096).
inline int64_t block_chunk_for(int32_t value_type, int64_t blocks) {
  int64_t k = value_type == SPMM_VALUE_F16 ? 2048 : 1024;
  while (k < 4096 && blocks / k > 16384) k *= 2;
  return k;
}

// Number of fixed overflow ranges for `blocks` usable blocks.
int64_t block_overflow_ranges(int64_t blocks, int64_t kbig);

// Block (BCSR 16x1) part.  `dense` and `out` rows are `ld` elements apart,
// `width` columns computed (vpart and slots rows hold `width` floats).  Runs
// after the gather pass: every window with
// blocks is written to `out` as block sum + the fp32 vector sums the gather
// pass left in `vpart` ([16*windows][width]) for its rows with vector
// nonzeros, rounded once.  `slots` holds the pieces of windows longer than
// block_chunk ([ranges][2][16][width] fp32) followed by one uint32 counter per
// range (block_counter_offset).  `counters_zeroed`: the gather's post pass of
// the same call zeroed the counters (launch_gather's zero_counts), and
// overflow work-groups take the long windows' segments, counted on them;
// otherwise each long window's own work-group sums its segments one after
// another (the same pieces added in the same order: the same results) and
// the counters are not used.
spmm_status launch_block(int32_t index_type, int32_t value_type,
                         const void* Crowptr, const void* Ccol, const void* Cvalue,
                         int64_t windows, int64_t block_count, int64_t block_values,
                         const void* Vrowptr, int64_t vector_rows, int64_t vector_nnz,
                         const void* dense, int64_t dense_rows, int64_t width, int64_t ld,
                         void* out, const float* vpart, float* slots, const int32_t* order,
                         bool counters_zeroed, hipStream_t stream);

}  // namespace spmm
