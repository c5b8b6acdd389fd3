// extern "C" entry points of libspmm_mi355x: argument validation, workspace
// sizing and dispatch to the kernels.  The checks mirror the reference's
// operator contracts (extension/custom_op.cpp:36-152) at the level of sizes
// and dtypes; tensor-level checks (device, rank, contiguity) live in the torch
// extension that calls this library.
#include <mutex>
#include <string>

#include "common.h"

// Scratch of spmm_csr_run_noalloc: the gather workspace (tail rows and fp32
// partial slots) of callers that cannot allocate.  Each device that loads
// the library holds its own copy until the process ends.  Host code must not
// pass this name to a kernel (on the host it is a stand-in, not a device
// address): its per-device address comes from hipGetSymbolAddress, once per
// device (scratch_on_current_device below).
constexpr size_t kNoallocScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

namespace spmm {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

spmm_status fail(spmm_status code, const std::string& msg) {
  set_error(msg);
  return code;
}

spmm_status check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return SPMM_OK;
  return fail(SPMM_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(err));
}

spmm_status check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

namespace {

spmm_status check_types(int32_t index_type, int32_t value_type, const char* op) {
  if (index_type != SPMM_INDEX_I32 && index_type != SPMM_INDEX_I64)
    return fail(SPMM_ERR_CONTRACT, std::string(op) + ": index arrays must be int32 or int64");
  if (value_type != SPMM_VALUE_F16 && value_type != SPMM_VALUE_F32)
    return fail(SPMM_ERR_CONTRACT, std::string(op) + " supports only FP16 and FP32 dense tensors");
  return SPMM_OK;
}

// Feature-width contract of check_dense_contract (extension/custom_op.cpp:39-57).
spmm_status check_width(int64_t width, int32_t value_type, int64_t alignment, const char* op) {
  const bool half = value_type == SPMM_VALUE_F16;
  const int64_t max_width = half ? 1024 : 512;
  if (width <= 0 || width > max_width)
    return fail(SPMM_ERR_CONTRACT, std::string(op) + " requires 0 < feature width <= " +
                                       std::to_string(max_width) + " for " +
                                       (half ? "FP16" : "FP32") + ", but got " +
                                       std::to_string(width));
  if (width % alignment != 0)
    return fail(SPMM_ERR_CONTRACT,
                std::string(op) + " requires feature width divisible by " +
                    std::to_string(alignment) + ", but got " + std::to_string(width) +
                    ". Pad and crop the dense tensor or use a safe PyTorch fallback.");
  return SPMM_OK;
}

// The kernels move 16-byte (gather) / 8-byte (block) pieces of dense and out.
spmm_status check_aligned(const void* dense, const void* out, const char* op) {
  if ((reinterpret_cast<uintptr_t>(dense) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return fail(SPMM_ERR_CONTRACT, std::string(op) + ": dense and out must be 16-byte aligned");
  return SPMM_OK;
}

// Checks shared by spmm_csr_run and its allocation-free variant (everything
// before the pointers).
spmm_status check_csr_desc(const spmm_csr_desc* d, const char* op) {
  if (d == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "null descriptor");
  if (spmm_status st = check_types(d->index_type, d->value_type, op)) return st;
  if (spmm_status st = check_width(d->width, d->value_type, d->value_type == SPMM_VALUE_F16 ? 16 : 8, op))
    return st;
  if (d->rows < 0 || d->nnz < 0 || d->dense_rows < 0)
    return fail(SPMM_ERR_CONTRACT, std::string(op) + ": negative extent");
  return SPMM_OK;
}

spmm_status check_csr_pointers(const spmm_csr_desc* d, const void* rowptr, const void* col,
                               const void* value, const void* dense, void* out, const char* op) {
  if (rowptr == nullptr || out == nullptr || (d->nnz > 0 && (col == nullptr || value == nullptr)) ||
      (d->dense_rows > 0 && dense == nullptr))
    return fail(SPMM_ERR_INVALID_ARGUMENT, std::string(op) + ": null device pointer");
  return check_aligned(dense, out, op);
}

int64_t elem_bytes(int32_t value_type) { return value_type == SPMM_VALUE_F16 ? 2 : 4; }

// spmm_csr over column slabs of pass_width columns (one pass when the dense
// operand is small): the same gather kernels per slab, rows N apart.
spmm_status csr_passes(const spmm_csr_desc* d, const void* rowptr, const void* col, const void* value,
                       const void* dense, void* out, void* ws, size_t ws_bytes, hipStream_t stream) {
  const int64_t s = elem_bytes(d->value_type);
  const int64_t w = pass_width(d->dense_rows, d->width, s);
  for (int64_t c = 0; c < d->width; c += w) {
    if (spmm_status st = launch_gather(d->index_type, d->value_type, rowptr, col, value, d->nnz, d->rows, 0,
                                       d->rows, static_cast<const char*>(dense) + c * s, d->dense_rows, w,
                                       d->width, static_cast<char*>(out) + c * s, ws, ws_bytes, nullptr, 0, 0,
                                       nullptr, nullptr, nullptr, nullptr, 0, stream))
      return st;
  }
  return SPMM_OK;
}

// Device address of `scratch` on the current device, resolved with
// hipGetSymbolAddress on the first call per device (with that device
// current) and kept; every later call on the device reuses it.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

spmm_status scratch_on_current_device(void** ptr) {
  int dev = -1;
  if (spmm_status st = check_hip(hipGetDevice(&dev), "hipGetDevice")) return st;
  if (dev < 0 || dev >= kMaxDevices) return fail(SPMM_ERR_DEVICE, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    if (spmm_status st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
      return st;
    if (p == nullptr) return fail(SPMM_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned null");
    g_scratch[dev] = p;
  }
  *ptr = g_scratch[dev];
  return SPMM_OK;
}

}  // namespace
}  // namespace spmm

using namespace spmm;

extern "C" {

const char* spmm_last_error(void) { return g_last_error.c_str(); }

const char* spmm_version(void) { return "spmm_mi355x 0.1 gfx950"; }

spmm_status spmm_csr_workspace(const spmm_csr_desc* d, size_t* bytes) {
  clear_error();
  if (d == nullptr || bytes == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "null argument");
  if (spmm_status st = check_types(d->index_type, d->value_type, "spmm_csr")) return st;
  *bytes = gather_workspace_bytes(d->nnz < 0 ? 0 : d->nnz,
                                  pass_width(d->dense_rows, d->width, elem_bytes(d->value_type)));
  return SPMM_OK;
}

spmm_status spmm_csr_run(const spmm_csr_desc* d, const void* rowptr, const void* col,
                         const void* value, const void* dense, void* out, void* workspace,
                         size_t workspace_bytes, spmm_stream stream) {
  clear_error();
  if (spmm_status st = check_csr_desc(d, "spmm_csr")) return st;
  if (d->rows == 0) return SPMM_OK;
  if (spmm_status st = check_csr_pointers(d, rowptr, col, value, dense, out, "spmm_csr")) return st;
  return csr_passes(d, rowptr, col, value, dense, out, workspace, workspace_bytes, as_stream(stream));
}

size_t spmm_csr_noalloc_max_scratch(void) { return kNoallocScratchBytes; }

spmm_status spmm_csr_run_noalloc(const spmm_csr_desc* d, const void* rowptr, const void* col,
                                 const void* value, const void* dense, void* out, spmm_stream stream) {
  clear_error();
  if (spmm_status st = check_csr_desc(d, "spmm_csr_run_noalloc")) return st;
  // The gather's scratch (tail rows, fp32 partial slots) must fit the fixed
  // array; checked before any HIP call.
  const size_t need =
      gather_workspace_bytes(d->nnz, pass_width(d->dense_rows, d->width, elem_bytes(d->value_type)));
  if (need > kNoallocScratchBytes)
    return fail(SPMM_ERR_CONTRACT, "spmm_csr_run_noalloc: this call needs " + std::to_string(need) +
                                       " bytes of scratch, more than the library's fixed " +
                                       std::to_string(kNoallocScratchBytes) +
                                       "; call spmm_csr_run with a workspace instead");
  if (d->rows == 0) return SPMM_OK;
  if (spmm_status st = check_csr_pointers(d, rowptr, col, value, dense, out, "spmm_csr_run_noalloc")) return st;
  void* ws = nullptr;
  if (spmm_status st = scratch_on_current_device(&ws)) return st;
  // Nothing in the scratch needs clearing: every call writes each tail entry
  // and each partial slot before the post pass reads it.
  return csr_passes(d, rowptr, col, value, dense, out, ws, kNoallocScratchBytes, as_stream(stream));
}

size_t spmm_gather_probe_sink(const spmm_csr_desc* d) {
  if (d == nullptr || d->nnz < 0 || d->width <= 0) return 0;
  return gather_probe_sink_floats(d->nnz, d->width, d->value_type);
}

spmm_status spmm_gather_probe(const spmm_csr_desc* d, const void* col, const void* value, const void* dense,
                              float* sink, spmm_stream stream) {
  clear_error();
  if (spmm_status st = check_csr_desc(d, "spmm_gather_probe")) return st;
  if (d->index_type != SPMM_INDEX_I32) return fail(SPMM_ERR_CONTRACT, "spmm_gather_probe: int32 column ids only");
  if (d->nnz == 0) return SPMM_OK;
  if (col == nullptr || value == nullptr || dense == nullptr || sink == nullptr)
    return fail(SPMM_ERR_INVALID_ARGUMENT, "spmm_gather_probe: null device pointer");
  if (spmm_status st = check_aligned(dense, sink, "spmm_gather_probe")) return st;
  return launch_gather_probe(d->value_type, col, value, d->nnz, dense, d->dense_rows, d->width, sink,
                             as_stream(stream));
}

spmm_status spmm_csr_rowscalar_run(const spmm_csr_desc* d, const void* rowptr, const void* col,
                                   const void* value, const void* dense, void* out, spmm_stream stream) {
  clear_error();
  if (d == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "null descriptor");
  if (spmm_status st = check_types(d->index_type, d->value_type, "spmm_csr_rowscalar")) return st;
  if (spmm_status st = check_width(d->width, d->value_type, d->value_type == SPMM_VALUE_F16 ? 16 : 8,
                                   "spmm_csr_rowscalar"))
    return st;
  if (d->rows < 0 || d->nnz < 0 || d->dense_rows < 0)
    return fail(SPMM_ERR_CONTRACT, "spmm_csr_rowscalar: negative extent");
  if (d->rows == 0) return SPMM_OK;
  if (rowptr == nullptr || out == nullptr || (d->nnz > 0 && (col == nullptr || value == nullptr)) ||
      (d->dense_rows > 0 && dense == nullptr))
    return fail(SPMM_ERR_INVALID_ARGUMENT, "spmm_csr_rowscalar: null device pointer");
  if (spmm_status st = check_aligned(dense, out, "spmm_csr_rowscalar")) return st;
  return launch_rowscalar(d->index_type, d->value_type, rowptr, col, value, d->rows, d->nnz, dense,
                          d->dense_rows, d->width, out, as_stream(stream));
}

int64_t spmm_mixed_out_rows(const spmm_mixed_desc* d) {
  if (d == nullptr) return -1;
  const int64_t blocks = 16 * (d->block_windows < 0 ? 0 : d->block_windows);
  const int64_t vec = d->vector_rows < 0 ? 0 : d->vector_rows;
  return blocks > vec ? blocks : vec;
}

namespace {
// Workspace of the mixed operator, for one column pass of w = pass_width
// columns (passes run one after another and reuse it): gather part, then the
// fp32 vector sums of block-window rows ([16*windows][w]), then the pieces of
// windows longer than the block chunk ([ranges][2][16][w]) and one counter per
// overflow range ([ranges] uint32, zeroed by each pass before its block
// kernel).
struct MixedLayout {
  size_t gather = 0, vpart = 0, slots = 0, order = 0;
  int64_t limit = 0, ranges = 0, w = 0;
  explicit MixedLayout(const spmm_mixed_desc* d) {
    w = d->width > 0 ? pass_width(d->dense_rows, d->width, elem_bytes(d->value_type)) : 0;
    gather = align_up(gather_workspace_bytes(d->vector_nnz < 0 ? 0 : d->vector_nnz, w), 256);
    // vpart only when there is a vector part (rows of block windows may then
    // have vector sums to hand over).
    const int64_t windows = d->block_windows > 0 && d->vector_nnz > 0 ? d->block_windows : 0;
    vpart = align_up(static_cast<size_t>(16 * windows) * w * sizeof(float), 256);
    limit = d->block_count < d->block_values / 16 ? d->block_count : d->block_values / 16;
    if (limit < 0) limit = 0;
    ranges = block_overflow_ranges(limit, block_chunk_for(d->value_type, limit));
    slots = align_up(static_cast<size_t>(ranges * 2 * 16) * w * sizeof(float) +
                         static_cast<size_t>(ranges) * sizeof(uint32_t), 256);
    // The block windows' locality order and its sort state (block_order_wanted).
    order = block_order_wanted(d->block_windows, d->vector_nnz, w, d->value_type)
                ? align_up(static_cast<size_t>(order_words(d->block_windows)) * sizeof(int32_t), 256)
                : 0;
  }
  size_t total() const { return gather + vpart + slots + order; }
};
}  // namespace

spmm_status spmm_mixed_workspace(const spmm_mixed_desc* d, size_t* bytes) {
  clear_error();
  if (d == nullptr || bytes == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "null argument");
  if (spmm_status st = check_types(d->index_type, d->value_type, "spmm_ascend_cube")) return st;
  *bytes = MixedLayout(d).total();
  return SPMM_OK;
}

spmm_status spmm_mixed_run(const spmm_mixed_desc* d, const void* Crowptr, const void* Ccol,
                           const void* Cvalue, const void* Vrowptr, const void* Vcol,
                           const void* Vvalue, const void* dense, void* out, void* workspace,
                           size_t workspace_bytes, spmm_stream stream) {
  clear_error();
  if (d == nullptr) return fail(SPMM_ERR_INVALID_ARGUMENT, "null descriptor");
  if (spmm_status st = check_types(d->index_type, d->value_type, "spmm_ascend_cube")) return st;
  if (spmm_status st = check_width(d->width, d->value_type, 16, "spmm_ascend_cube")) return st;
  if (d->block_windows < 0 || d->block_count < 0 || d->block_values < 0 || d->vector_rows < 0 ||
      d->vector_nnz < 0 || d->dense_rows < 0)
    return fail(SPMM_ERR_CONTRACT, "spmm_ascend_cube: negative extent");
  const int64_t out_rows = spmm_mixed_out_rows(d);
  if (out_rows == 0) return SPMM_OK;
  if (out == nullptr || (d->dense_rows > 0 && dense == nullptr) ||
      (d->block_windows > 0 && Crowptr == nullptr) ||
      (d->block_count > 0 && (Ccol == nullptr || Cvalue == nullptr)) ||
      Vrowptr == nullptr ||
      (d->vector_nnz > 0 && (Vcol == nullptr || Vvalue == nullptr)))
    return fail(SPMM_ERR_INVALID_ARGUMENT, "spmm_ascend_cube: null device pointer");
  if (spmm_status st = check_aligned(dense, out, "spmm_ascend_cube")) return st;
  if (reinterpret_cast<uintptr_t>(Cvalue) % 16 != 0)
    return fail(SPMM_ERR_CONTRACT, "spmm_ascend_cube: Cvalue must be 16-byte aligned");
  hipStream_t s = as_stream(stream);
  const MixedLayout lay(d);
  if (workspace == nullptr || workspace_bytes < lay.total())
    return fail(SPMM_ERR_CONTRACT, "spmm_ascend_cube: workspace too small: need " +
                                       std::to_string(lay.total()) + " bytes");
  char* ws = static_cast<char*>(workspace);
  float* vpart = lay.vpart > 0 ? reinterpret_cast<float*>(ws + lay.gather) : nullptr;
  float* slots = reinterpret_cast<float*>(ws + lay.gather + lay.vpart);
  int32_t* order = lay.order > 0 ? reinterpret_cast<int32_t*>(ws + lay.gather + lay.vpart + lay.slots) : nullptr;
  // Vector pass first (it leaves the fp32 vector sums of block-window rows in
  // vpart), then the block part, which adds them and rounds once.  Without
  // vector nonzeros the block kernel writes the zero rows of windows without
  // blocks itself, and the vector pass only covers rows past the windows.
  // With the window order (block_order_wanted), the vector pass's kernel also
  // writes the block windows' locality order, which the block kernel follows.
  // The block kernel's window counters (after the pieces in `slots`) are
  // zeroed by the gather's post pass when it runs (it always does when the
  // gather covers any row); without it, the block kernel sums each long
  // window's pieces in the window's own work-group and uses no counter.
  const int64_t row_lo = d->vector_nnz == 0 ? 16 * d->block_windows : 0;
  const bool gather_runs = out_rows > row_lo;
  // A dense operand much larger than the Infinity Cache is swept in column
  // passes of lay.w columns (pass_width), each pass both parts on its slab.
  uint32_t* counts = reinterpret_cast<uint32_t*>(slots + lay.ranges * 2 * 16 * lay.w);
  const int64_t eb = elem_bytes(d->value_type);
  for (int64_t c = 0; c < d->width; c += lay.w) {
    const void* dense_c = static_cast<const char*>(dense) + c * eb;
    void* out_c = static_cast<char*>(out) + c * eb;
    spmm_status st = launch_gather(d->index_type, d->value_type, Vrowptr, Vcol, Vvalue, d->vector_nnz,
                                   d->vector_rows, row_lo, out_rows, dense_c, d->dense_rows, lay.w, d->width, out_c,
                                   ws, lay.gather, d->block_windows > 0 ? Crowptr : nullptr, d->block_windows,
                                   lay.limit, vpart, Ccol, order, lay.ranges > 0 ? counts : nullptr, lay.ranges, s);
    if (st != SPMM_OK) return st;
    st = launch_block(d->index_type, d->value_type, Crowptr, Ccol, Cvalue, d->block_windows, d->block_count,
                      d->block_values, Vrowptr, d->vector_rows, d->vector_nnz, dense_c, d->dense_rows, lay.w,
                      d->width, out_c, vpart, slots, order, gather_runs, s);
    if (st != SPMM_OK) return st;
  }
  return SPMM_OK;
}

}  // extern "C"
