/*
 * spmm_oracle.c — CPU restatement of Ascend-SpMM's hot-path algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only as the checker.
 * The product (ascend-spmm_amd/) never links, imports or calls it.
 *
 * Each function restates one reference routine (paths relative to the
 * Ascend-SpMM repository root) in plain single-threaded C:
 *   or_spmm_f64         C = A*B in fp64 — the mathematics the kernels
 *                       (kernels/op_kernel/spmm_csr.cpp:383-423,
 *                       spmm_ascend_cube.cpp:16-311) approximate.
 *   or_spmm_cube_f64    the window-encoded spmm_cube operator in fp64
 *                       (kernels/op_kernel/spmm_cube.cpp:53-146)
 *   or_make_start       make_start (tests/task_mapping/common.py:119-127)
 *   or_csr_to_bcsr      ToBCSR (extension/custom_op.cpp:594-713)
 *   or_csr_to_cube      your_logic_kernel (extension/custom_op.cpp:429-560)
 *   or_hybrid_split     hybrid_split_impl (extension/custom_op.cpp:1146-1348)
 *   or_bucket_sort      stable_bucket_sort_by_occupancy_desc
 *                       (extension/boundary_bucket_sort.h:13-56)
 *   or_renumber         renumber_columns_for_packed_layout
 *                       (extension/packed_column_reindex.h:14-41)
 *   or_transpose        transpose_into_packed_layout
 *                       (extension/packed_column_reindex.h:43-101)
 *   or_preprocess       taskmapping (extension/custom_op.cpp:765-1110) incl.
 *                       pack_fixed_layout (:1350-1384)
 *
 * Values are copied, never computed on, by the preprocessing routines, so they
 * are handled as opaque elements of `vs` bytes (bit-exact copies).
 * Indices are int64 here; callers convert.
 *
 * Status codes: 0 ok, 1 invalid_argument, 2 out_of_range, 3 overflow_error,
 * 4 runtime (TORCH_CHECK).  or_last_error() returns the message.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { OR_OK = 0, OR_INVALID = 1, OR_RANGE = 2, OR_OVERFLOW = 3, OR_RUNTIME = 4 };

static char g_err[256];
const char* or_last_error(void) { return g_err; }
static int fail(int code, const char* msg) {
  snprintf(g_err, sizeof g_err, "%s", msg);
  return code;
}

#define ALLOC(type, n) ((type*)calloc((size_t)((n) > 0 ? (n) : 1), sizeof(type)))

/* ------------------------------------------------------------------ SpMM */

/* C[r, :] = sum_{p in [rowptr[r], rowptr[r+1])} val[p] * B[col[p], :] in fp64. */
void or_spmm_f64(int64_t rows, const int64_t* rowptr, const int64_t* col, const double* val,
                 int64_t K, int64_t N, const double* B, double* C) {
  for (int64_t r = 0; r < rows; ++r) {
    double* out = C + r * N;
    for (int64_t n = 0; n < N; ++n) out[n] = 0.0;
    for (int64_t p = rowptr[r]; p < rowptr[r + 1]; ++p) {
      const int64_t c = col[p];
      if (c < 0 || c >= K) continue;
      const double v = val[p];
      const double* b = B + c * N;
      for (int64_t n = 0; n < N; ++n) out[n] += v * b[n];
    }
  }
}

/* Window-encoded SpMM of the legacy spmm_cube operator
 * (kernels/op_kernel/spmm_cube.cpp:53-146): window w owns nonzeros
 * [rowptr[w], rowptr[w+1]); col = (c << 4) | r.  A maximal run of
 * consecutive nonzeros with equal c is one 16x1 block whose row r holds the
 * value of the run's last nonzero with row r (the kernel stores each value
 * into its block slot, so a later one overwrites); the block adds
 * block[r] * B[c, :] to output row 16*w + r.  c outside [0, K) adds nothing.
 * Output: 16 * windows rows, in fp64. */
void or_spmm_cube_f64(int64_t windows, const int64_t* rowptr, const int64_t* col, const double* val,
                      int64_t nnz, int64_t K, int64_t N, const double* B, double* C) {
  for (int64_t i = 0; i < 16 * windows * N; ++i) C[i] = 0.0;
  for (int64_t w = 0; w < windows; ++w) {
    int64_t a = rowptr[w], b = rowptr[w + 1];
    a = a < 0 ? 0 : (a > nnz ? nnz : a);
    b = b < a ? a : (b > nnz ? nnz : b);
    int64_t p = a;
    while (p < b) {
      const int64_t c = col[p] >> 4;
      double blk[16];
      int have[16];
      for (int r = 0; r < 16; ++r) { blk[r] = 0.0; have[r] = 0; }
      int64_t q = p;
      while (q < b && (col[q] >> 4) == c) {
        const int r = (int)(col[q] & 15);
        blk[r] = val[q];
        have[r] = 1;
        ++q;
      }
      if (c >= 0 && c < K)
        for (int r = 0; r < 16; ++r)
          if (have[r]) {
            double* out = C + (16 * w + r) * N;
            const double* row = B + c * N;
            for (int64_t n = 0; n < N; ++n) out[n] += blk[r] * row[n];
          }
      p = q;
    }
  }
}

/* -------------------------------------------------------------- make_start */

/* start[k] = searchsorted(pointer, k*ceil(total/cores), right) - 1, clamped at
 * 0; all zeros when total <= 0 (tests/task_mapping/common.py:119-127). */
void or_make_start(const int64_t* pointer, int64_t n, int64_t cores, int32_t* start) {
  const int64_t total = n > 0 ? pointer[n - 1] : 0;
  if (total <= 0) {
    for (int64_t k = 0; k < cores; ++k) start[k] = 0;
    return;
  }
  const int64_t chunk = (total + cores - 1) / cores;
  for (int64_t k = 0; k < cores; ++k) {
    const int64_t target = k * chunk;
    int64_t lo = 0, hi = n; /* first index with pointer[i] > target */
    while (lo < hi) {
      const int64_t mid = lo + (hi - lo) / 2;
      if (pointer[mid] <= target) lo = mid + 1; else hi = mid;
    }
    int64_t s = lo - 1;
    start[k] = (int32_t)(s < 0 ? 0 : s);
  }
}

/* ------------------------------------------------- 16-way window merge core */

/* Shared by ToBCSR and your_logic_kernel: walk one window's rows as a k-way
 * merge.  Each step takes the row head with the smallest column (ties -> the
 * lowest row, as std::min_element), calls `emit`, and advances that row.
 * Exhausted and padding rows carry the sentinel `ncols`. */
typedef struct {
  const int64_t* crow;
  const int64_t* col;
  int64_t nrows, ncols, nwindows, window_size;
} merge_in;

typedef void (*emit_fn)(void* ctx, int64_t col_id, int64_t row_id, int64_t pos);

static void merge_window(const merge_in* in, int64_t w, void* ctx, emit_fn emit) {
  const int64_t W = in->window_size, offset = w * W;
  int64_t* head = ALLOC(int64_t, W);
  int64_t* start = ALLOC(int64_t, W);
  int64_t tag = W;
  for (int64_t i = 0; i < W; ++i) {
    if (i + offset < in->nrows) {
      start[i] = in->crow[i + offset];
      if (start[i] == in->crow[i + offset + 1]) {
        --tag;
        head[i] = in->ncols;
      } else {
        head[i] = in->col[start[i]];
      }
    } else {
      --tag;
      head[i] = in->ncols;
    }
  }
  while (tag) {
    int64_t row = 0;
    for (int64_t i = 1; i < W; ++i)
      if (head[i] < head[row]) row = i;
    emit(ctx, head[row], row, start[row]);
    start[row] += 1;
    if (start[row] == in->crow[row + offset + 1]) {
      --tag;
      head[row] = in->ncols;
    } else {
      head[row] = in->col[start[row]];
    }
  }
  free(head);
  free(start);
}

/* ---------------------------------------------------------------- ToBCSR */

typedef struct {
  const unsigned char* val;
  int64_t vs;
  int64_t* unique_col_ids;
  unsigned char* value;
  int64_t col_ptr, last_col_id;
} bcsr_ctx;

static void bcsr_emit(void* p, int64_t col_id, int64_t row_id, int64_t pos) {
  bcsr_ctx* c = (bcsr_ctx*)p;
  if (c->last_col_id != col_id) {
    c->unique_col_ids[c->col_ptr++] = col_id;
    c->last_col_id = col_id;
  }
  /* value[16*col_ptr - 16 + row_id] = v (custom_op.cpp:661) */
  memcpy(c->value + (16 * c->col_ptr - 16 + row_id) * c->vs, c->val + pos * c->vs, (size_t)c->vs);
}

/* Outputs: crow_window_ptr[nwindows+1], unique_col_ids[<= nnz], value[16 * n]
 * (caller-zeroed, element size vs).  Returns the block count in *nblocks. */
int or_csr_to_bcsr(const int64_t* crow, const int64_t* col, const unsigned char* val, int64_t vs,
                   int64_t nrows, int64_t ncols, int64_t window_size, int64_t* crow_window_ptr,
                   int64_t* unique_col_ids, unsigned char* value, int64_t* nblocks) {
  if (window_size < 1 || window_size > 16)
    return fail(OR_INVALID, "window_size must be in [1, 16] (value blocks hold 16 rows)");
  const int64_t nwindows = (nrows + window_size - 1) / window_size;
  merge_in in = {crow, col, nrows, ncols, nwindows, window_size};
  bcsr_ctx ctx = {val, vs, unique_col_ids, value, 0, -1};
  for (int64_t w = 0; w < nwindows; ++w) {
    crow_window_ptr[w] = ctx.col_ptr;
    ctx.last_col_id = -1;
    merge_window(&in, w, &ctx, bcsr_emit);
  }
  crow_window_ptr[nwindows] = ctx.col_ptr;
  *nblocks = ctx.col_ptr;
  return OR_OK;
}

/* ------------------------------------------------------- your_logic_kernel */

typedef struct {
  const unsigned char* val;
  int64_t vs;
  int64_t* unique_col_ids;
  unsigned char* value;
  int64_t col_ptr, blk_ptr, cnt, last_col_id;
} cube_ctx;

static void cube_emit(void* p, int64_t col_id, int64_t row_id, int64_t pos) {
  cube_ctx* c = (cube_ctx*)p;
  if (c->last_col_id != col_id) {
    c->unique_col_ids[c->col_ptr++] = col_id;
    c->cnt++;
    if (c->cnt == 16) {
      c->cnt = 0;
      c->blk_ptr++;
    }
    c->last_col_id = col_id;
  }
  /* value[256*blk_ptr + 16*row_id + cnt] = v (custom_op.cpp:501) */
  memcpy(c->value + (256 * c->blk_ptr + 16 * row_id + c->cnt) * c->vs, c->val + pos * c->vs,
         (size_t)c->vs);
}

/* Outputs: crow_window_ptr[nwindows+1] (tile offsets), unique_col_ids[16*ntiles]
 * (zero-padded per window), value[256*ntiles] (caller-zeroed). */
int or_csr_to_cube(const int64_t* crow, const int64_t* col, const unsigned char* val, int64_t vs,
                   int64_t nrows, int64_t ncols, int64_t window_size, int64_t* crow_window_ptr,
                   int64_t* unique_col_ids, unsigned char* value, int64_t* ntiles) {
  if (window_size < 1 || window_size > 16)
    return fail(OR_INVALID, "window_size must be in [1, 16] (value tiles hold 16 rows)");
  const int64_t nwindows = (nrows + window_size - 1) / window_size;
  merge_in in = {crow, col, nrows, ncols, nwindows, window_size};
  cube_ctx ctx = {val, vs, unique_col_ids, value, 0, 0, -1, -1};
  for (int64_t w = 0; w < nwindows; ++w) {
    crow_window_ptr[w] = ctx.blk_ptr;
    ctx.cnt = -1;
    ctx.last_col_id = -1;
    merge_window(&in, w, &ctx, cube_emit);
    if (ctx.cnt != -1) {
      for (; ctx.cnt < 15; ctx.cnt++) unique_col_ids[ctx.col_ptr++] = 0;
      ctx.blk_ptr++;
    }
  }
  crow_window_ptr[nwindows] = ctx.blk_ptr;
  *ntiles = ctx.blk_ptr;
  if (ctx.col_ptr != ctx.blk_ptr * 16) return fail(OR_RUNTIME, "Error: tile column count");
  return OR_OK;
}

/* ------------------------------------------------------------ bucket sort */

/* Stable sort of `columns` by occupancy[column] descending; equal counts keep
 * their order.  Errors as boundary_bucket_sort.h:19-36. */
int or_bucket_sort(int64_t* columns, int64_t n, const int64_t* occupancy, int64_t nocc,
                   int64_t max_occupancy) {
  if (max_occupancy <= 0) {
    if (n == 0) return OR_OK;
    return fail(OR_INVALID, "max occupancy must be positive");
  }
  for (int64_t i = 0; i < n; ++i) {
    const int64_t c = columns[i];
    if (c < 0 || c >= nocc) return fail(OR_RANGE, "column id is outside the occupancy array");
    const int64_t cnt = occupancy[c];
    if (cnt <= 0 || cnt > max_occupancy)
      return fail(OR_INVALID,
                  "block occupancy must be in [1, window_size]; coalesce duplicate CSR entries");
  }
  int64_t* sorted = ALLOC(int64_t, n);
  int64_t k = 0;
  for (int64_t cnt = max_occupancy; cnt >= 1; --cnt)
    for (int64_t i = 0; i < n; ++i)
      if (occupancy[columns[i]] == cnt) sorted[k++] = columns[i];
  memcpy(columns, sorted, (size_t)n * sizeof(int64_t));
  free(sorted);
  return OR_OK;
}

/* ---------------------------------------------------------- renumbering */

/* out[i] = inv[cols[i]] with the checks of packed_column_reindex.h:22-37;
 * index_max is the largest value of the sparse index type. */
int or_renumber(const int64_t* cols, int64_t n, const int64_t* inv, int64_t ninv,
                int64_t index_max, int64_t* out) {
  for (int64_t i = 0; i < n; ++i) {
    const int64_t c = cols[i];
    if (c < 0 || c >= ninv)
      return fail(OR_RANGE, "column id cannot be mapped into the packed row layout");
    const int64_t pc = inv[c];
    if (pc < 0) return fail(OR_INVALID, "inverse permutation does not map every original column");
    if ((uint64_t)pc > (uint64_t)index_max)
      return fail(OR_OVERFLOW, "packed column id does not fit the sparse index type");
    out[i] = pc;
  }
  return OR_OK;
}

/* ------------------------------------------------------ packed transpose */

/* CSR of P*A^T*P^T: entry (r, c, v) of A goes to row inv[c] with column inv[r];
 * entries are placed in (original row, position) order.  `rows` = length of
 * inv.  Errors as packed_column_reindex.h:55-91. */
int or_transpose(const int64_t* rowptr, const int64_t* cols, const unsigned char* vals, int64_t vs,
                 int64_t nnz, const int64_t* inv, int64_t rows, int64_t packed_rows,
                 int64_t* rowptrT, int64_t* colsT, unsigned char* valsT) {
  if (rowptr[rows] != nnz) return fail(OR_INVALID, "CSR row pointer does not end at nnz");
  for (int64_t r = 0; r <= packed_rows; ++r) rowptrT[r] = 0;
  for (int64_t p = 0; p < nnz; ++p) {
    const int64_t c = cols[p];
    if (c < 0 || c >= rows) return fail(OR_RANGE, "transpose column is outside the graph");
    const int64_t pr = inv[c];
    if (pr < 0 || pr >= packed_rows) return fail(OR_INVALID, "invalid packed row in inverse permutation");
    rowptrT[pr + 1]++;
  }
  for (int64_t r = 0; r < packed_rows; ++r) rowptrT[r + 1] += rowptrT[r];
  int64_t* next = ALLOC(int64_t, packed_rows + 1);
  memcpy(next, rowptrT, (size_t)(packed_rows + 1) * sizeof(int64_t));
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t pc = inv[r];
    if (pc < 0 || pc >= packed_rows) {
      free(next);
      return fail(OR_INVALID, "invalid packed column in inverse permutation");
    }
    const int64_t b = rowptr[r], e = rowptr[r + 1];
    if (b > e || e > nnz || b < 0) {
      free(next);
      return fail(OR_INVALID, "non-monotonic CSR row pointer");
    }
    for (int64_t p = b; p < e; ++p) {
      const int64_t d = next[inv[cols[p]]]++;
      colsT[d] = pc;
      memcpy(valsT + d * vs, vals + p * vs, (size_t)vs);
    }
  }
  free(next);
  return OR_OK;
}

/* --------------------------------------------------------- hybrid split */

typedef struct {
  int64_t* crow_window_ptr; int64_t n_crow;
  int64_t* unique_col_ids;  int64_t n_unique;
  unsigned char* value;     int64_t n_value;  /* elements */
  int64_t* vrow_window_ptr; int64_t n_vrow;
  int64_t* vcol_indices;    int64_t n_vnnz;
  unsigned char* vvalue;
} or_split_out;

typedef struct { int64_t win, col, cnt, idx; } block_info;

static int cmp_i64(const void* a, const void* b) {
  const int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return (x > y) - (x < y);
}

/* Stable ascending order of blocks by cnt: sort by (cnt, original index). */
static int cmp_block_cnt(const void* a, const void* b) {
  const block_info* x = (const block_info*)a;
  const block_info* y = (const block_info*)b;
  if (x->cnt != y->cnt) return (x->cnt > y->cnt) - (x->cnt < y->cnt);
  return (x->idx > y->idx) - (x->idx < y->idx);
}

/* Output buffers of `out` are caller-allocated at upper bounds:
 * crow nwin+1, unique nnz, value 16*nnz elements (zeroed), vrow m_pad+1,
 * vcol nnz, vvalue nnz elements. */
int or_hybrid_split(const int64_t* crow, const int64_t* col, const unsigned char* val, int64_t vs,
                    int64_t nrows, int64_t ncols, double a, int64_t window_size,
                    or_split_out* out) {
  if (window_size < 1) return fail(OR_INVALID, "window_size must be positive");
  const int64_t W = window_size;
  const int64_t num_windows = (nrows + W - 1) / W;
  const int64_t m_pad = num_windows * W;
  const int64_t nnz_all = nrows > 0 ? crow[nrows] : 0;

  /* Phase 1 (custom_op.cpp:1160-1190): blocks in window-major first-seen order. */
  block_info* blocks = ALLOC(block_info, nnz_all);
  int64_t* win_start = ALLOC(int64_t, num_windows + 1);
  int64_t* epoch = ALLOC(int64_t, ncols);
  int64_t* cnt = ALLOC(int64_t, ncols);
  for (int64_t c = 0; c < ncols; ++c) epoch[c] = -1;
  int64_t nb = 0;
  for (int64_t w = 0; w < num_windows; ++w) {
    const int64_t b0 = nb, r0 = w * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t p = crow[r]; p < crow[r + 1]; ++p) {
        const int64_t c = col[p];
        if (c < 0 || c >= ncols) {
          free(blocks); free(win_start); free(epoch); free(cnt);
          return fail(OR_RUNTIME, "column index out of range");
        }
        if (epoch[c] != w) {
          epoch[c] = w;
          cnt[c] = 0;
          blocks[nb].win = w;
          blocks[nb].col = c;
          blocks[nb].cnt = 0;
          blocks[nb].idx = nb;
          ++nb;
        }
        cnt[c]++;
      }
    for (int64_t b = b0; b < nb; ++b) blocks[b].cnt = cnt[blocks[b].col];
    win_start[w + 1] = nb;
  }

  /* Phase 2 (:1192-1223): stable ascending by count; first k minimising
   * |ratio - a|. */
  block_info* order = ALLOC(block_info, nb);
  memcpy(order, blocks, (size_t)nb * sizeof(block_info));
  qsort(order, (size_t)nb, sizeof(block_info), cmp_block_cnt);
  int64_t* prefix = ALLOC(int64_t, nb + 1);
  for (int64_t i = 0; i < nb; ++i) prefix[i + 1] = prefix[i] + order[i].cnt;
  int64_t best_k = 0;
  double best_diff = INFINITY;
  for (int64_t k = 0; k <= nb; ++k) {
    const int64_t rem = nb - k, nz = prefix[k];
    const double ratio = (nz == 0) ? (rem > 0 ? INFINITY : 0.0) : (double)rem / (double)nz;
    const double diff = fabs(ratio - a);
    if (diff < best_diff) {
      best_diff = diff;
      best_k = k;
    }
  }
  char* moved = ALLOC(char, nb);
  for (int64_t i = 0; i < best_k; ++i) moved[order[i].idx] = 1;

  /* Phase 3a (:1225-1273): BSR over all windows, kept columns ascending. */
  out->crow_window_ptr[0] = 0;
  for (int64_t w = 0; w < num_windows; ++w) {
    int64_t kept = 0;
    for (int64_t b = win_start[w]; b < win_start[w + 1]; ++b) kept += moved[b] ? 0 : 1;
    out->crow_window_ptr[w + 1] = out->crow_window_ptr[w] + kept;
  }
  out->n_crow = num_windows + 1;
  const int64_t n_kept = out->crow_window_ptr[num_windows];
  out->n_unique = n_kept;
  out->n_value = n_kept * W;
  int64_t* slot_epoch = epoch; /* reuse */
  int64_t* slot_of = cnt;
  for (int64_t c = 0; c < ncols; ++c) slot_epoch[c] = -1;
  int64_t* kept_cols = ALLOC(int64_t, nb);
  for (int64_t w = 0; w < num_windows; ++w) {
    int64_t nk = 0;
    for (int64_t b = win_start[w]; b < win_start[w + 1]; ++b)
      if (!moved[b]) kept_cols[nk++] = blocks[b].col;
    qsort(kept_cols, (size_t)nk, sizeof(int64_t), cmp_i64);
    int64_t pos = out->crow_window_ptr[w];
    for (int64_t i = 0; i < nk; ++i) {
      out->unique_col_ids[pos] = kept_cols[i];
      slot_epoch[kept_cols[i]] = w;
      slot_of[kept_cols[i]] = pos;
      ++pos;
    }
    const int64_t r0 = w * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t p = crow[r]; p < crow[r + 1]; ++p) {
        const int64_t c = col[p];
        if (slot_epoch[c] == w)
          memcpy(out->value + (slot_of[c] * W + (r - r0)) * vs, val + p * vs, (size_t)vs);
      }
  }

  /* Phase 3b (:1275-1309): CSR residual over m_pad rows in original order. */
  int64_t* moved_epoch = kept_cols; /* reuse as (window, col) -> moved marker */
  free(moved_epoch);
  moved_epoch = ALLOC(int64_t, ncols);
  for (int64_t c = 0; c < ncols; ++c) moved_epoch[c] = -1;
  int64_t vnnz = 0;
  for (int64_t w = 0; w < num_windows; ++w) {
    for (int64_t b = win_start[w]; b < win_start[w + 1]; ++b)
      if (moved[b]) moved_epoch[blocks[b].col] = w;
    const int64_t r0 = w * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    for (int64_t r = r0; r < r1; ++r) {
      out->vrow_window_ptr[r] = vnnz;
      for (int64_t p = crow[r]; p < crow[r + 1]; ++p) {
        const int64_t c = col[p];
        if (moved_epoch[c] == w) {
          out->vcol_indices[vnnz] = c;
          memcpy(out->vvalue + vnnz * vs, val + p * vs, (size_t)vs);
          ++vnnz;
        }
      }
    }
    for (int64_t r = r1; r < r0 + W; ++r) out->vrow_window_ptr[r] = vnnz;
  }
  out->vrow_window_ptr[m_pad] = vnnz;
  out->n_vrow = m_pad + 1;
  out->n_vnnz = vnnz;

  free(blocks); free(win_start); free(epoch); free(cnt); free(order); free(prefix);
  free(moved); free(moved_epoch);
  return OR_OK;
}

/* ------------------------------------------------------------- taskmapping */

typedef struct {
  or_split_out fwd;
  int64_t* renum_unique; int64_t n_renum_unique;
  int64_t* renum_vcol;   int64_t n_renum_vcol;
  or_split_out tr;       /* transpose_* (empty unless graph layout) */
  int64_t* permutation;  int64_t n_perm;
  int64_t* inv_permutation; int64_t n_inv;
  int64_t packed_rows, packed_layout_supported, marginal_window, marginal_aic_blocks,
      marginal_total_blocks, shared_windows;
  double est_aic, est_aiv, est_max;
} or_preprocess_out;

typedef struct { int64_t id, nnz, nb; double density; } window_stat;

static int cmp_window(const void* a, const void* b) {
  const window_stat* x = (const window_stat*)a;
  const window_stat* y = (const window_stat*)b;
  if (x->density != y->density) return x->density > y->density ? -1 : 1;
  return (x->id > y->id) - (x->id < y->id);
}

/* Buffers of `out` are caller-allocated at upper bounds (nwin = ceil(nrows/16)):
 * fwd.crow nwin+1, fwd.unique nnz, fwd.value 16*nnz (zeroed), fwd.vrow 16*nwin+1,
 * fwd.vcol/vvalue nnz, renum_* nnz, permutation 16*nwin, inv nrows, and tr.* as
 * fwd.  index_max is the largest value of the sparse index type. */
int or_preprocess(const int64_t* crow, const int64_t* col, const unsigned char* val, int64_t vs,
                  int64_t nnz, int64_t nrows, int64_t ncols, int64_t window_size,
                  int graph_layout, int64_t index_max, or_preprocess_out* out) {
  if (window_size != 16) return fail(OR_RUNTIME, "Ascend-SpMM requires a 16-row window");
  const double kAic = 295.0, kAiv = 505.0;
  const int64_t W = 16;
  const int64_t nwin = (nrows + W - 1) / W;
  int rc = OR_OK;

  /* Window statistics (custom_op.cpp:784-806). */
  window_stat* win = ALLOC(window_stat, nwin);
  int64_t* epoch = ALLOC(int64_t, ncols);
  for (int64_t c = 0; c < ncols; ++c) epoch[c] = -1;
  for (int64_t w = 0; w < nwin; ++w) {
    const int64_t r0 = w * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    int64_t wn = 0, wb = 0;
    for (int64_t r = r0; r < r1; ++r) {
      wn += crow[r + 1] - crow[r];
      for (int64_t p = crow[r]; p < crow[r + 1]; ++p) {
        const int64_t c = col[p];
        if (!(c >= 0 && c < ncols)) {
          free(win); free(epoch);
          return fail(OR_RUNTIME, "column index out of range");
        }
        if (epoch[c] != w) {
          epoch[c] = w;
          ++wb;
        }
      }
    }
    win[w].id = w;
    win[w].nnz = wn;
    win[w].nb = wb;
    win[w].density = wb ? (double)wn / (double)wb : 0.0;
  }
  /* Density descending, id ascending (:808-811). */
  qsort(win, (size_t)nwin, sizeof(window_stat), cmp_window);

  /* Marginal window (:813-826). */
  int64_t bpos = -1, prefix_blocks = 0, remaining = nnz;
  for (int64_t pos = 0; pos < nwin; ++pos) {
    const double aic_after = (double)(prefix_blocks + win[pos].nb) / kAic;
    const double aiv_after = (double)(remaining - win[pos].nnz) / kAiv;
    if (aic_after >= aiv_after) {
      bpos = pos;
      break;
    }
    prefix_blocks += win[pos].nb;
    remaining -= win[pos].nnz;
  }

  /* Marginal split (:828-885). */
  int64_t bwin = -1, bblocks = 0, baic = 0;
  double e_aic = 0.0, e_aiv = 0.0, e_max = 0.0;
  char* to_aic = ALLOC(char, ncols);
  if (bpos >= 0) {
    bwin = win[bpos].id;
    bblocks = win[bpos].nb;
    int64_t* occ = ALLOC(int64_t, ncols);
    int64_t* bcols = ALLOC(int64_t, bblocks);
    int64_t nbc = 0;
    const int64_t r0 = bwin * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t p = crow[r]; p < crow[r + 1]; ++p) {
        const int64_t c = col[p];
        if (occ[c]++ == 0) bcols[nbc++] = c;
      }
    if (nbc != bblocks) rc = fail(OR_RUNTIME, "internal boundary-block count mismatch");
    if (rc == OR_OK) rc = or_bucket_sort(bcols, nbc, occ, ncols, W);
    if (rc == OR_OK) {
      const int64_t suffix = remaining - win[bpos].nnz;
      int64_t assigned = 0, best_q = 0;
      double best = INFINITY;
      for (int64_t q = 0; q <= bblocks; ++q) {
        const double aic = (double)(prefix_blocks + q) / kAic;
        const double aiv = (double)(suffix + win[bpos].nnz - assigned) / kAiv;
        const double mx = aic > aiv ? aic : aiv; /* std::max(aic, aiv) */
        if (mx < best) {
          best = mx;
          best_q = q;
          e_aic = aic;
          e_aiv = aiv;
          e_max = mx;
        }
        if (q < bblocks) assigned += occ[bcols[q]];
      }
      baic = best_q;
      for (int64_t q = 0; q < best_q; ++q) to_aic[bcols[q]] = 1;
    }
    free(occ);
    free(bcols);
  }
  if (rc != OR_OK) {
    free(win); free(epoch); free(to_aic);
    return rc;
  }

  /* Window lists (:887-905). */
  int64_t* aic = ALLOC(int64_t, nwin);
  int64_t* aiv = ALLOC(int64_t, nwin);
  int64_t naic = 0, naiv = 0;
  if (bpos < 0) {
    for (int64_t i = 0; i < nwin; ++i) aiv[naiv++] = win[i].id;
  } else {
    for (int64_t i = 0; i < bpos; ++i) aic[naic++] = win[i].id;
    if (baic > 0) aic[naic++] = bwin; else aiv[naiv++] = bwin;
    for (int64_t i = bpos + 1; i < nwin; ++i) aiv[naiv++] = win[i].id;
  }
  const int shared = baic > 0 && baic < bblocks;
  const int64_t aic_padded = naic * W;
  int64_t aic_real = 0;
  for (int64_t i = 0; i < naic; ++i) {
    const int64_t w = aic[i];
    aic_real += ((w + 1) * W < nrows ? (w + 1) * W : nrows) - w * W;
  }
  const int64_t real_extent = aic_padded + (nrows - aic_real);
  const int64_t layout = graph_layout && nrows == ncols ? 1 : 0;
  const int64_t out_rows = layout ? nwin * W : real_extent;

  /* Permutation (:917-940). */
  int64_t* perm = out->permutation;
  int64_t* inv = out->inv_permutation;
  for (int64_t i = 0; i < out_rows; ++i) perm[i] = -1;
  for (int64_t i = 0; i < nrows; ++i) inv[i] = -1;
  for (int64_t s = 0; s < naic; ++s) {
    const int64_t w = aic[s], r0 = w * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    for (int64_t r = r0; r < r1; ++r) {
      perm[s * W + (r - r0)] = r;
      inv[r] = s * W + (r - r0);
    }
  }
  int64_t vrow = aic_padded;
  for (int64_t i = 0; i < naiv; ++i) {
    const int64_t w = aiv[i], r0 = w * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    for (int64_t r = r0; r < r1; ++r) {
      perm[vrow] = r;
      inv[r] = vrow;
      ++vrow;
    }
  }
  out->n_perm = out_rows;
  out->n_inv = nrows;

  /* AIC pack (:942-979): per slot, the distinct columns ascending. */
  or_split_out* f = &out->fwd;
  int64_t* bepoch = epoch;
  for (int64_t c = 0; c < ncols; ++c) bepoch[c] = -1;
  int64_t* bslot = ALLOC(int64_t, ncols);
  int64_t* bc = ALLOC(int64_t, nnz);
  int64_t nunique = 0;
  f->crow_window_ptr[0] = 0;
  for (int64_t s = 0; s < naic; ++s) {
    const int64_t w = aic[s], r0 = w * W, r1 = r0 + W < nrows ? r0 + W : nrows;
    int64_t n = 0;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t p = crow[r]; p < crow[r + 1]; ++p) {
        const int64_t c = col[p];
        if (shared && w == bwin && !to_aic[c]) continue;
        if (bepoch[c] != s) {
          bepoch[c] = s;
          bc[n++] = c;
        }
      }
    qsort(bc, (size_t)n, sizeof(int64_t), cmp_i64);
    for (int64_t i = 0; i < n; ++i) {
      f->unique_col_ids[nunique + i] = bc[i];
      bslot[bc[i]] = nunique + i;
    }
    nunique += n;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t p = crow[r]; p < crow[r + 1]; ++p) {
        const int64_t c = col[p];
        if (shared && w == bwin && !to_aic[c]) continue;
        memcpy(f->value + (bslot[c] * W + (r - r0)) * vs, val + p * vs, (size_t)vs);
      }
    f->crow_window_ptr[s + 1] = nunique;
  }
  f->n_crow = naic + 1;
  f->n_unique = nunique;
  f->n_value = nunique * W;

  /* AIV pack (:981-1001). */
  int64_t vn = 0;
  for (int64_t o = 0; o < out_rows; ++o) {
    f->vrow_window_ptr[o] = vn;
    const int64_t orig = perm[o];
    if (orig < 0) continue;
    const int vector_owned = o >= aic_padded;
    const int residual = shared && orig / W == bwin;
    if (!vector_owned && !residual) continue;
    for (int64_t p = crow[orig]; p < crow[orig + 1]; ++p) {
      const int64_t c = col[p];
      if (residual && to_aic[c]) continue;
      f->vcol_indices[vn] = c;
      memcpy(f->vvalue + vn * vs, val + p * vs, (size_t)vs);
      ++vn;
    }
  }
  f->vrow_window_ptr[out_rows] = vn;
  f->n_vrow = out_rows + 1;
  f->n_vnnz = vn;

  /* Graph layout (:1003-1035). */
  out->n_renum_unique = 0;
  out->n_renum_vcol = 0;
  out->tr.n_crow = out->tr.n_unique = out->tr.n_value = out->tr.n_vrow = out->tr.n_vnnz = 0;
  if (layout) {
    rc = or_renumber(f->unique_col_ids, nunique, inv, nrows, index_max, out->renum_unique);
    if (rc == OR_OK) {
      out->n_renum_unique = nunique;
      rc = or_renumber(f->vcol_indices, vn, inv, nrows, index_max, out->renum_vcol);
    }
    if (rc == OR_OK) {
      out->n_renum_vcol = vn;
      int64_t* rt = ALLOC(int64_t, out_rows + 1);
      int64_t* ct = ALLOC(int64_t, nnz);
      unsigned char* vt = (unsigned char*)calloc((size_t)(nnz > 0 ? nnz : 1), (size_t)vs);
      rc = or_transpose(crow, col, val, vs, nnz, inv, nrows, out_rows, rt, ct, vt);
      if (rc == OR_OK)
        rc = or_hybrid_split(rt, ct, vt, vs, out_rows, out_rows, 295.0 / 505.0, W, &out->tr);
      free(rt); free(ct); free(vt);
    }
  }

  out->packed_rows = out_rows;
  out->packed_layout_supported = layout;
  out->marginal_window = bwin;
  out->marginal_aic_blocks = baic;
  out->marginal_total_blocks = bblocks;
  out->est_aic = e_aic;
  out->est_aiv = e_aiv;
  out->est_max = e_max;
  out->shared_windows = shared ? 1 : 0;

  free(win); free(epoch); free(to_aic); free(aic); free(aiv); free(bslot); free(bc);
  return rc;
}
