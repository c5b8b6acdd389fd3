/*
 * spmm_mi355x.h — C ABI of the MI355X (gfx950) SpMM library `libspmm_mi355x.so`.
 *
 * This is the drop-in boundary for the SpMM hot path of Ascend-SpMM.  Every
 * entry point below replaces one call site of the reference's CANN/aclnn
 * layer or one of its host-side preprocessing routines; the citation next to
 * each declaration names the reference code it stands in for (paths are
 * relative to the Ascend-SpMM repository root).
 *
 * Conventions
 *  - Plain pointers and sizes only; no C++ or torch types cross this boundary.
 *  - All device pointers are HIP device memory owned by the caller.  The
 *    library never allocates device memory for its outputs; scratch space is
 *    the caller-provided workspace, sized by the matching *_workspace call.
 *  - Launches are asynchronous on the given stream unless the comment says
 *    the call synchronises (the *_plan calls read a few sizes back).
 *  - Index arrays of one call share one index type (int32 or int64); value
 *    arrays and the dense operand share one value type (fp16 or fp32).
 *  - Kernels never read outside the extents passed in: row pointers are
 *    clamped to the index arrays and out-of-range column ids contribute zero.
 *  - On failure a call returns a non-zero spmm_status and records a message
 *    retrievable (per thread) with spmm_last_error().
 *  - Reentrant: calls on different streams may run concurrently.
 */
#ifndef SPMM_MI355X_H_
#define SPMM_MI355X_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Each maps to one Python exception type in the extension,
 * matching what the reference raises for the same condition:
 * INVALID_ARGUMENT -> ValueError   (std::invalid_argument in the reference)
 * OUT_OF_RANGE     -> IndexError   (std::out_of_range)
 * OVERFLOW         -> OverflowError(std::overflow_error)
 * CONTRACT         -> RuntimeError (TORCH_CHECK failures)
 * DEVICE           -> RuntimeError (a HIP runtime error) */
typedef enum spmm_status {
  SPMM_OK = 0,
  SPMM_ERR_INVALID_ARGUMENT = 1,
  SPMM_ERR_OUT_OF_RANGE = 2,
  SPMM_ERR_OVERFLOW = 3,
  SPMM_ERR_CONTRACT = 4,
  SPMM_ERR_DEVICE = 5
} spmm_status;

typedef enum spmm_index_type { SPMM_INDEX_I32 = 0, SPMM_INDEX_I64 = 1 } spmm_index_type;
typedef enum spmm_value_type { SPMM_VALUE_F16 = 0, SPMM_VALUE_F32 = 1, SPMM_VALUE_F64 = 2 } spmm_value_type;

/* Opaque HIP stream (hipStream_t); NULL is the default stream. */
typedef void* spmm_stream;

/* Message of the last failed call on this thread ("" if none). */
const char* spmm_last_error(void);

/* Library version string, e.g. "spmm_mi355x 0.1 gfx950". */
const char* spmm_version(void);

/* ------------------------------------------------------------------------
 * spmm_csr — C[M,N] = A[M,K] (CSR) x dense[K,N]
 *
 * Replaces EXEC_NPU_CMD(aclnnSpmmCsr, ...) in spmm_csr_impl_npu
 * (extension/custom_op.cpp:67-88) and the tiling + kernel behind it
 * (kernels/op_host/spmm_csr.cpp:8-35, kernels/op_kernel/spmm_csr.cpp:226-569).
 * The reference's per-core `start` array is a tiling aid; the MI355X kernel
 * partitions on the device, so `start` is not an argument here.
 *
 * Every output row is written (rows without nonzeros become zero), so `out`
 * need not be cleared.  Each row is accumulated in fp32 in nonzero order and
 * rounded once to the value type (round-to-nearest-even).  Rows longer than
 * the library's fixed split length are cut at split points that depend only
 * on the row pointer, and their fp32 pieces are added in order, so results are
 * deterministic and identical for every feature width N.
 * ---------------------------------------------------------------------- */
typedef struct spmm_csr_desc {
  int64_t rows;        /* M: rowptr holds rows + 1 entries                 */
  int64_t nnz;         /* extent of col[] and value[]                      */
  int64_t dense_rows;  /* K: rows of dense                                 */
  int64_t width;       /* N: columns of dense and out (row-major, contiguous) */
  int32_t index_type;  /* spmm_index_type                                  */
  int32_t value_type;  /* spmm_value_type (F16 or F32)                     */
} spmm_csr_desc;

spmm_status spmm_csr_workspace(const spmm_csr_desc* desc, size_t* bytes);

spmm_status spmm_csr_run(const spmm_csr_desc* desc,
                         const void* rowptr, const void* col, const void* value,
                         const void* dense, void* out,
                         void* workspace, size_t workspace_bytes,
                         spmm_stream stream);

/* Allocation-free spmm_csr: same arguments (minus the workspace), same
 * kernels and bit-identical results as spmm_csr_run.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Its scratch is a fixed device array inside the library, of
 * spmm_csr_noalloc_max_scratch() bytes (64 MiB) per GPU, held from the
 * library's load until the process ends; the call allocates nothing.  A call
 * whose scratch (spmm_csr_workspace's figure) exceeds it fails with
 * SPMM_ERR_CONTRACT before touching the device.  Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (different streams, or
 * host threads, without ordering between them) race and must not be made.
 * The first call on each device looks up the array's device address
 * (hipGetSymbolAddress) and keeps it; make that first call outside stream
 * capture (one eager call before capturing), so that no capture sees the
 * lookup.  Later calls only launch kernels and may be captured. */
size_t spmm_csr_noalloc_max_scratch(void);

spmm_status spmm_csr_run_noalloc(const spmm_csr_desc* desc,
                                 const void* rowptr, const void* col, const void* value,
                                 const void* dense, void* out, spmm_stream stream);

/* Gather-rate probe.  No counterpart in the reference: a measurement for
 * callers judging spmm_csr_run against what the GPU can gather.  It runs the
 * dense-row gathers of spmm_csr_run over the same nonzeros (column ids and
 * values staged per tile, one 16-byte piece of every nonzero's dense row per
 * lane, fp32 FMAs) without the row bookkeeping, partial sums or output rows,
 * and writes one float per thread to `sink` (spmm_gather_probe_sink(desc)
 * floats, 16-byte aligned).  int32 column ids; dense operand up to 4 GB;
 * rowptr is not read. */
size_t spmm_gather_probe_sink(const spmm_csr_desc* desc);

spmm_status spmm_gather_probe(const spmm_csr_desc* desc, const void* col, const void* value,
                              const void* dense, float* sink, spmm_stream stream);

/* Thread-per-row scalar CSR SpMM, same arguments and result contract as
 * spmm_csr_run (same sums in the same order within a row; no workspace).
 * No counterpart in the reference: it is the baseline that the block path's
 * speed-up is stated against (one thread per output row, nonzeros in order,
 * 16-byte pieces of the dense row), for callers comparing kernels. */
spmm_status spmm_csr_rowscalar_run(const spmm_csr_desc* desc,
                                   const void* rowptr, const void* col, const void* value,
                                   const void* dense, void* out, spmm_stream stream);

/* ------------------------------------------------------------------------
 * spmm_mixed — the spmm_ascend_cube operator:
 *   out[16*s + r, :]  = sum_{b in [Crowptr[s], Crowptr[s+1])} Cvalue[16*b + r] * dense[Ccol[b], :]
 *   out[i, :]        += sum_{p in [Vrowptr[i], Vrowptr[i+1])} Vvalue[p] * dense[Vcol[p], :]
 * with out rows = max(16 * block_windows, vector_rows).
 *
 * Replaces EXEC_NPU_CMD(aclnnSpmmAscendCube, ...) in spmm_ascend_cube_impl_npu
 * (extension/custom_op.cpp:115-152), its tiling
 * (kernels/op_host/spmm_ascend_cube.cpp:8-51) and the mixed AIC/AIV kernel
 * (kernels/op_kernel/spmm_ascend_cube.cpp:16-311, 543-907).  The per-core
 * Cstart/Vstart arrays of the reference are not needed.
 *
 * The block part (16x1 BCSR windows) runs on fp16/fp32 MFMA.  The vector
 * part runs the CSR gather path of spmm_csr first; for rows of block windows
 * that have blocks it leaves the fp32 vector sum in the workspace, and the
 * block kernel adds it after the block sum and rounds once.  With
 * block_windows == 0 the result is bit-identical to spmm_csr on the same CSR.
 * Every output row is written.  dense, out and Cvalue must be 16-byte
 * aligned (SPMM_ERR_CONTRACT otherwise).
 * ---------------------------------------------------------------------- */
typedef struct spmm_mixed_desc {
  int64_t block_windows;  /* Crowptr.numel - 1                              */
  int64_t block_count;    /* Ccol_ids.numel                                 */
  int64_t block_values;   /* Cvalue.numel (>= 16 * blocks referenced)       */
  int64_t vector_rows;    /* Vrowptr.numel - 1                              */
  int64_t vector_nnz;     /* min(Vcol_ids.numel, Vvalue.numel)              */
  int64_t dense_rows;     /* K                                              */
  int64_t width;          /* N                                              */
  int32_t index_type;
  int32_t value_type;
} spmm_mixed_desc;

spmm_status spmm_mixed_workspace(const spmm_mixed_desc* desc, size_t* bytes);

spmm_status spmm_mixed_run(const spmm_mixed_desc* desc,
                           const void* Crowptr, const void* Ccol, const void* Cvalue,
                           const void* Vrowptr, const void* Vcol, const void* Vvalue,
                           const void* dense, void* out,
                           void* workspace, size_t workspace_bytes,
                           spmm_stream stream);

/* Number of output rows spmm_mixed_run writes: max(16*block_windows, vector_rows). */
int64_t spmm_mixed_out_rows(const spmm_mixed_desc* desc);

/* ------------------------------------------------------------------------
 * spmm_cube_op — the legacy spmm_cube operator.  Window w (16 output rows)
 * owns nonzeros [rowptr[w], rowptr[w+1]); each carries col = (c << 4) | r,
 * c the dense row and r the row inside the window.  Maximal runs of
 * consecutive nonzeros with equal c form one 16x1 block whose row r is the
 * value of the run's last nonzero with row r:
 *   out[16*w + r, :] = sum over window w's runs of block[r] * dense[c, :]
 * with out rows = 16 * windows, every row written.  Replaces
 * EXEC_NPU_CMD(aclnnSpmmCube, ...) in spmm_cube_impl_npu
 * (extension/custom_op.cpp:91-113) and its kernel
 * (kernels/op_kernel/spmm_cube.cpp:53-146).  Decoded on the device into the
 * block layout of spmm_mixed_run and run on its MFMA block kernel.  c outside
 * [0, dense_rows) contributes zero.  Width contract: 0 < N <= 1024 (fp16) or
 * 512 (fp32), N % 16 == 0; dense and out 16-byte aligned; nnz < 2^31 - 1.
 * The workspace holds the decoded blocks (16 values per nonzero at most).
 * ---------------------------------------------------------------------- */
typedef struct spmm_cube_op_desc {
  int64_t windows;     /* rowptr.numel - 1                                */
  int64_t nnz;         /* col.numel (== value.numel)                      */
  int64_t dense_rows;  /* K                                               */
  int64_t width;       /* N                                               */
  int32_t index_type;
  int32_t value_type;
} spmm_cube_op_desc;

spmm_status spmm_cube_op_workspace(const spmm_cube_op_desc* desc, size_t* bytes);

spmm_status spmm_cube_op_run(const spmm_cube_op_desc* desc,
                             const void* rowptr, const void* col, const void* value,
                             const void* dense, void* out,
                             void* workspace, size_t workspace_bytes,
                             spmm_stream stream);

/* ------------------------------------------------------------------------
 * Row permutation of a node tensor (P and P^T of the graph layout).
 *
 * spmm_pack_rows:    packed[inv[i], :] = src[i, :] for i < rows; every other
 *                    packed row is zero (if inv repeats a packed row, the
 *                    largest i wins).  Replaces pack_node_tensor's
 *                    new_zeros + index_copy_ (spmm_npu.py:23-47).  Needs a
 *                    workspace of spmm_pack_workspace(packed_rows) bytes.
 * spmm_restore_rows: dst[i, :] = packed[inv[i], :].  Replaces
 *                    restore_node_tensor's index_select (spmm_npu.py:50-62).
 * `row_bytes` is the byte size of one row (any element type).  `inv` is int64.
 * Entries of inv outside [0, packed_rows) are skipped by pack and give a zero
 * row in restore (the Python layer rejects them before the call, as the
 * reference does).
 * ---------------------------------------------------------------------- */
size_t spmm_pack_workspace(int64_t packed_rows);

spmm_status spmm_pack_rows(const void* src, int64_t rows, int64_t row_bytes,
                           const int64_t* inv, void* packed, int64_t packed_rows,
                           void* workspace, size_t workspace_bytes,
                           spmm_stream stream);

spmm_status spmm_restore_rows(const void* packed, int64_t packed_rows, int64_t row_bytes,
                              const int64_t* inv, int64_t rows, void* dst,
                              spmm_stream stream);

/* ------------------------------------------------------------------------
 * Preprocessing on the GPU (layout conversion and work partitioning).
 *
 * The reference runs these on the host with ATen accessors; here they are
 * device pipelines whose outputs are bit-identical to the reference's
 * (integer arrays, and values copied bit for bit).  Index outputs use the
 * input's index type; permutations are int64.
 *
 * Each conversion is two calls on the same workspace:
 *   *_workspace(...)  bytes of workspace (depends only on the sizes)
 *   *_plan(...)       runs the pipeline into the workspace and returns the
 *                     output sizes (synchronises the stream)
 *   *_fill(...)       writes the outputs into caller buffers of those sizes
 * Input requirements (checked on the device, reported by *_plan):
 *   row pointer monotone within [0, nnz]  -> SPMM_ERR_INVALID_ARGUMENT
 *   column ids in [0, cols)               -> SPMM_ERR_CONTRACT
 *   (bcsr / cube) ascending columns per row, as the reference's docs
 *   require (extension/custom_op.cpp:1430,1440) -> SPMM_ERR_INVALID_ARGUMENT
 * ---------------------------------------------------------------------- */
typedef struct spmm_csr_matrix {
  int64_t rows;        /* rowptr holds rows + 1 entries                    */
  int64_t cols;
  int64_t nnz;         /* extent of col[] and value[]                      */
  int32_t index_type;  /* spmm_index_type                                  */
  int32_t value_type;  /* spmm_value_type: F16, F32 or F64 (copied only)   */
  const void* rowptr;  /* device pointers                                  */
  const void* col;
  const void* value;
} spmm_csr_matrix;

/* csr_to_bcsr: BCSR(16x1).  Replaces ToBCSR / csr_to_bcsr
 * (extension/custom_op.cpp:594-746).  Outputs: crow_window_ptr[nwin+1],
 * unique_col_ids[blocks], value[16*blocks], nwin = ceil(rows/window_size),
 * 1 <= window_size <= 16. */
size_t spmm_bcsr_workspace(const spmm_csr_matrix* m, int64_t window_size);
spmm_status spmm_bcsr_plan(const spmm_csr_matrix* m, int64_t window_size, void* workspace,
                           size_t workspace_bytes, spmm_stream stream, int64_t* blocks);
spmm_status spmm_bcsr_fill(const spmm_csr_matrix* m, int64_t window_size, void* workspace,
                           size_t workspace_bytes, void* crow_window_ptr, void* unique_col_ids,
                           void* value, spmm_stream stream);

/* csr_to_ascend_cube: 16x16 cube tiles.  Replaces your_logic_kernel /
 * csr_to_ascend_cube (extension/custom_op.cpp:429-592).  Outputs:
 * crow_window_ptr[nwin+1] (tile offsets), unique_col_ids[16*tiles] (zero
 * padded per window), value[256*tiles]. */
size_t spmm_cube_workspace(const spmm_csr_matrix* m, int64_t window_size);
spmm_status spmm_cube_plan(const spmm_csr_matrix* m, int64_t window_size, void* workspace,
                           size_t workspace_bytes, spmm_stream stream, int64_t* tiles);
spmm_status spmm_cube_fill(const spmm_csr_matrix* m, int64_t window_size, void* workspace,
                           size_t workspace_bytes, void* crow_window_ptr, void* unique_col_ids,
                           void* value, spmm_stream stream);

/* block_level_split: density-threshold BCSR(window_size x 1) + CSR split.
 * Replaces hybrid_split_impl / block_level_split
 * (extension/custom_op.cpp:1139-1348, 1390-1412).  Outputs:
 * crow_window_ptr[nwin+1], unique_col_ids[kept_blocks],
 * value[window_size*kept_blocks], vrow_window_ptr[window_size*nwin+1],
 * vcol_indices[vector_nnz], vvalue[vector_nnz]. */
size_t spmm_hybrid_workspace(const spmm_csr_matrix* m, int64_t window_size);
spmm_status spmm_hybrid_plan(const spmm_csr_matrix* m, double a, int64_t window_size,
                             void* workspace, size_t workspace_bytes, spmm_stream stream,
                             int64_t* kept_blocks, int64_t* vector_nnz);
spmm_status spmm_hybrid_fill(const spmm_csr_matrix* m, double a, int64_t window_size,
                             void* workspace, size_t workspace_bytes, void* crow_window_ptr,
                             void* unique_col_ids, void* value, void* vrow_window_ptr,
                             void* vcol_indices, void* vvalue, spmm_stream stream);

/* preprocess: the 295/505 cost-model AIC/AIV task mapping with the marginal
 * window split, row permutation and (graph_layout on a square matrix) the
 * renumbered columns and the fixed-layout transpose P*A^T*P^T.  Replaces
 * taskmapping / preprocess (extension/custom_op.cpp:749-1137, with
 * boundary_bucket_sort.h and packed_column_reindex.h).  window_size must be
 * 16 (SPMM_ERR_CONTRACT otherwise, as the reference's TORCH_CHECK). */
typedef struct spmm_taskmap_info {
  int64_t aic_windows;            /* crow_window_ptr: aic_windows + 1       */
  int64_t aic_blocks;             /* unique_col_ids; value: 16*aic_blocks   */
  int64_t packed_rows;            /* vrow_window_ptr: packed_rows + 1; permutation */
  int64_t vector_nnz;             /* vcol_indices, vvalue                   */
  int64_t packed_layout_supported;
  int64_t marginal_window;        /* -1 if none                             */
  int64_t marginal_aic_blocks;
  int64_t marginal_total_blocks;
  int64_t shared_windows;
  double estimated_aic_cost;
  double estimated_aiv_cost;
  double estimated_max_cost;
  /* transpose_* (graph layout only; all 0 otherwise)                     */
  int64_t t_windows;              /* transpose_crow_window_ptr: t_windows+1 */
  int64_t t_blocks;               /* transpose_unique_col_ids; value 16*t_blocks */
  int64_t t_rows;                 /* transpose_vrow_window_ptr: t_rows + 1  */
  int64_t t_vector_nnz;
} spmm_taskmap_info;

typedef struct spmm_taskmap_out {
  void* crow_window_ptr;
  void* unique_col_ids;
  void* value;
  void* vrow_window_ptr;
  void* vcol_indices;
  void* vvalue;
  void* renumbered_unique_col_ids;  /* graph layout: aic_blocks entries   */
  void* renumbered_vcol_indices;    /* graph layout: vector_nnz entries   */
  void* transpose_crow_window_ptr;
  void* transpose_unique_col_ids;
  void* transpose_value;
  void* transpose_vrow_window_ptr;
  void* transpose_vcol_indices;
  void* transpose_vvalue;
  int64_t* permutation;             /* packed_rows entries (-1 = padding)  */
  int64_t* inv_permutation;         /* rows entries                        */
} spmm_taskmap_out;

size_t spmm_taskmap_workspace(const spmm_csr_matrix* m, int64_t window_size, int graph_layout);
spmm_status spmm_taskmap_plan(const spmm_csr_matrix* m, int64_t window_size, int graph_layout,
                              void* workspace, size_t workspace_bytes, spmm_stream stream,
                              spmm_taskmap_info* info);
spmm_status spmm_taskmap_fill(const spmm_csr_matrix* m, int64_t window_size, int graph_layout,
                              void* workspace, size_t workspace_bytes,
                              const spmm_taskmap_out* out, spmm_stream stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* SPMM_MI355X_H_ */
