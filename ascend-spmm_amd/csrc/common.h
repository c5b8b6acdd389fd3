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

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Split length of the CSR gather path: nonzero positions are cut into ranges
// [j*R, (j+1)*R).  It is a constant of the build, independent of width and
// dtype, which is what makes the gather results identical for every feature
// width.
#ifndef SPMM_GATHER_RANGE
#define SPMM_GATHER_RANGE 256
#endif
constexpr int64_t kGatherRange = SPMM_GATHER_RANGE;

// fp32 storage of one partial row in the gather workspace, padded so every
// slot starts 256-byte aligned.
inline int64_t gather_slot_floats(int64_t width) { return (width + 63) / 64 * 64; }

// ---- internal launchers (defined in the .hip files) ----------------------

// Vector (CSR gather) part over rows [row_lo, row_hi) of the CSR given by
// (rowptr, col, value) with `nnz` valid entries.  Writes rows to `out`.
spmm_status launch_gather(int32_t index_type, int32_t value_type,
                          const void* rowptr, const void* col, const void* value,
                          int64_t nnz, int64_t row_lo, int64_t row_hi,
                          const void* dense, int64_t dense_rows, int64_t width,
                          void* out, void* workspace, size_t workspace_bytes,
                          hipStream_t stream);

// Workspace bytes launch_gather may use for at most `nnz` vector nonzeros.
size_t gather_workspace_bytes(int64_t nnz, int64_t width);

// Block (BCSR 16x1) part: every window s < windows computes its block sum on
// MFMA, adds the vector-part nonzeros of rows 16*s .. 16*s+15 that exist
// (row < vector_rows), and writes rows 16*s .. 16*s+15 of `out`.
spmm_status launch_block(int32_t index_type, int32_t value_type,
                         const void* Crowptr, const void* Ccol, const void* Cvalue,
                         int64_t windows, int64_t block_count, int64_t block_values,
                         const void* Vrowptr, const void* Vcol, const void* Vvalue,
                         int64_t vector_rows, int64_t vector_nnz,
                         const void* dense, int64_t dense_rows, int64_t width,
                         void* out, hipStream_t stream);

}  // namespace spmm
