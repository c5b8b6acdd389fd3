// custom_ops_lib — the PyTorch-ROCm extension behind `spmm_npu`.
//
// It keeps the reference extension's operator surface
// (extension/custom_op.cpp:266-283 TORCH_LIBRARY(myops) schemas and the
// pybind module at :1413-1492): same names, argument order, validation
// messages and output sizing.  Every operator is a thin wrapper that checks
// its tensors, allocates the output on the tensor's device and calls the C ABI
// of libspmm_mi355x.so on the current HIP stream.  There is no host compute
// path: tensors that are not on a GPU are rejected.
#include <torch/extension.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <map>
#include <stdexcept>
#include <string>

#include <ATen/hip/HIPContext.h>

#include "../../../include/spmm_mi355x.h"

namespace {

constexpr int64_t kSpmmHalfMaxDenseWidth = 1024;
constexpr int64_t kSpmmFloatMaxDenseWidth = 512;

inline bool is_gpu(const at::Tensor& tensor) { return tensor.device().is_cuda(); }
#define TORCH_CHECK_GPU(tensor) \
  TORCH_CHECK(is_gpu(tensor), #tensor " must be a GPU tensor (MI355X build; reference: NPU tensor)")

// Same checks and messages as the reference (extension/custom_op.cpp:39-64).
void check_dense_contract(const at::Tensor& dense, int64_t alignment, const char* op_name) {
  TORCH_CHECK(dense.scalar_type() == at::kHalf || dense.scalar_type() == at::kFloat, op_name,
              " supports only FP16 and FP32 dense tensors");
  TORCH_CHECK(dense.is_contiguous(), op_name, " requires a contiguous dense tensor");
  const int64_t width = dense.size(1);
  const bool is_half = dense.scalar_type() == at::kHalf;
  const int64_t max_width = is_half ? kSpmmHalfMaxDenseWidth : kSpmmFloatMaxDenseWidth;
  const char* dtype_name = is_half ? "FP16" : "FP32";
  TORCH_CHECK(width > 0 && width <= max_width, op_name, " requires 0 < feature width <= ",
              max_width, " for ", dtype_name, ", but got ", width);
  TORCH_CHECK(width % alignment == 0, op_name, " requires feature width divisible by ", alignment,
              ", but got ", width,
              ". Pad and crop the dense tensor or use a safe PyTorch fallback.");
}

void check_value_contract(const at::Tensor& value, const at::Tensor& dense, const char* name) {
  TORCH_CHECK(value.scalar_type() == dense.scalar_type(), name,
              " must have the same dtype as dense");
  TORCH_CHECK(value.is_contiguous(), name, " must be contiguous");
}

int32_t index_type_of(const at::Tensor& t, const char* name) {
  if (t.scalar_type() == at::kInt) return SPMM_INDEX_I32;
  if (t.scalar_type() == at::kLong) return SPMM_INDEX_I64;
  TORCH_CHECK(false, name, " must be an int32 or int64 tensor, but got ", t.scalar_type());
  return -1;
}

int32_t value_type_of(const at::Tensor& dense) {
  return dense.scalar_type() == at::kHalf ? SPMM_VALUE_F16 : SPMM_VALUE_F32;
}

// Maps a library status to the exception type the reference raises for the
// same condition (pybind11 turns these into ValueError / IndexError /
// OverflowError / RuntimeError).
void raise_status(spmm_status st, const char* what) {
  if (st == SPMM_OK) return;
  const std::string msg = std::string(what) + ": " + spmm_last_error();
  switch (st) {
    case SPMM_ERR_INVALID_ARGUMENT: throw std::invalid_argument(msg);
    case SPMM_ERR_OUT_OF_RANGE: throw std::out_of_range(msg);
    case SPMM_ERR_OVERFLOW: throw std::overflow_error(msg);
    default: TORCH_CHECK(false, msg);
  }
}

spmm_stream current_stream(const at::Tensor& t) {
  return reinterpret_cast<spmm_stream>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_same_device(const at::Tensor& a, const at::Tensor& b, const char* name) {
  TORCH_CHECK(a.device() == b.device(), name, " must be on the same device as dense");
}

// The kernels read dense and Cvalue in 16-byte pieces; a view at an offset
// that is not a multiple of 16 bytes is copied.
at::Tensor aligned(const at::Tensor& t) {
  return reinterpret_cast<uintptr_t>(t.data_ptr()) % 16 == 0 ? t : t.clone();
}

at::Tensor workspace(const at::Tensor& like, size_t bytes) {
  return at::empty({static_cast<int64_t>(bytes > 0 ? bytes : 1)}, like.options().dtype(at::kByte));
}

}  // namespace

// spmm_csr (reference: spmm_csr_impl_npu, extension/custom_op.cpp:67-88).
at::Tensor spmm_csr_impl(const at::Tensor& rowptr, const at::Tensor& col, const at::Tensor& value,
                         const at::Tensor& dense, const at::Tensor& start) {
  TORCH_CHECK_GPU(rowptr);
  TORCH_CHECK_GPU(col);
  TORCH_CHECK_GPU(value);
  TORCH_CHECK_GPU(dense);
  TORCH_CHECK_GPU(start);
  TORCH_CHECK(rowptr.dim() == 1, "row must be a 1D Tensor, but got: ", rowptr.dim());
  TORCH_CHECK(col.dim() == 1, "col must be a 1D Tensor, but got: ", col.dim());
  TORCH_CHECK(value.dim() == 1, "value must be a 1D Tensor, but got: ", value.dim());
  TORCH_CHECK(dense.dim() == 2, "dense must be a 2D Tensor, but got: ", dense.dim());
  TORCH_CHECK(start.dim() == 1, "start must be a 1D Tensor, but got: ", start.dim());
  check_dense_contract(dense, dense.scalar_type() == at::kHalf ? 16 : 8, "spmm_csr");
  check_value_contract(value, dense, "value");
  const int64_t nnz1 = col.size(0), nnz2 = value.size(0);
  TORCH_CHECK(nnz1 == nnz2, "col and value must be same size, but got different: ", nnz1 - nnz2);
  TORCH_CHECK(rowptr.size(0) >= 1, "row must hold at least one entry");
  const int32_t it = index_type_of(rowptr, "rowptr");
  TORCH_CHECK(index_type_of(col, "col") == it, "rowptr and col must have the same dtype");
  check_same_device(rowptr, dense, "rowptr");
  check_same_device(col, dense, "col");
  check_same_device(value, dense, "value");

  c10::DeviceGuard guard(dense.device());
  const at::Tensor rp = rowptr.contiguous(), cl = col.contiguous();
  const at::Tensor dn = aligned(dense);
  const int64_t M = rowptr.size(0) - 1, D = dense.size(1);
  auto result = at::empty({M, D}, dense.options());
  spmm_csr_desc d{M, nnz1, dense.size(0), D, it, value_type_of(dense)};
  size_t ws_bytes = 0;
  raise_status(spmm_csr_workspace(&d, &ws_bytes), "spmm_csr");
  at::Tensor ws = workspace(dense, ws_bytes);
  raise_status(spmm_csr_run(&d, rp.data_ptr(), cl.data_ptr(), value.data_ptr(), dn.data_ptr(),
                            result.data_ptr(), ws.data_ptr(), ws_bytes, current_stream(dense)),
               "spmm_csr");
  return result;
}

namespace {
at::Tensor run_mixed(const at::Tensor& Crowptr, const at::Tensor& Ccol_ids, const at::Tensor& Cvalue,
                     const at::Tensor& Vrowptr, const at::Tensor& Vcol_ids, const at::Tensor& Vvalue,
                     const at::Tensor& dense, const char* op_name) {
  const int32_t it = index_type_of(Crowptr, "Crowptr");
  TORCH_CHECK(index_type_of(Ccol_ids, "Ccol_ids") == it && index_type_of(Vrowptr, "Vrowptr") == it &&
                  index_type_of(Vcol_ids, "Vcol_ids") == it,
              op_name, ": all index tensors must have the same dtype");
  for (const at::Tensor* t : {&Crowptr, &Ccol_ids, &Cvalue, &Vrowptr, &Vcol_ids, &Vvalue})
    check_same_device(*t, dense, op_name);
  c10::DeviceGuard guard(dense.device());
  const at::Tensor crp = Crowptr.contiguous(), ccl = Ccol_ids.contiguous();
  const at::Tensor vrp = Vrowptr.contiguous(), vcl = Vcol_ids.contiguous();
  const at::Tensor dn = aligned(dense), cv = aligned(Cvalue);
  spmm_mixed_desc d;
  d.block_windows = std::max<int64_t>(Crowptr.size(0) - 1, 0);
  d.block_count = Ccol_ids.size(0);
  d.block_values = Cvalue.size(0);
  d.vector_rows = std::max<int64_t>(Vrowptr.size(0) - 1, 0);
  d.vector_nnz = std::min(Vcol_ids.size(0), Vvalue.size(0));
  d.dense_rows = dense.size(0);
  d.width = dense.size(1);
  d.index_type = it;
  d.value_type = value_type_of(dense);
  // Output rows as in the reference (extension/custom_op.cpp:146).
  const int64_t rows = std::max((Crowptr.size(0) - 1) * 16, Vrowptr.size(0) - 1);
  auto result = at::empty({std::max<int64_t>(rows, 0), dense.size(1)}, dense.options());
  size_t ws_bytes = 0;
  raise_status(spmm_mixed_workspace(&d, &ws_bytes), op_name);
  at::Tensor ws = workspace(dense, ws_bytes);
  raise_status(spmm_mixed_run(&d, crp.data_ptr(), ccl.data_ptr(), cv.data_ptr(), vrp.data_ptr(),
                              vcl.data_ptr(), Vvalue.data_ptr(), dn.data_ptr(), result.data_ptr(),
                              ws.data_ptr(), ws_bytes, current_stream(dense)),
               op_name);
  return result;
}
}  // namespace

// spmm_ascend_cube (reference: spmm_ascend_cube_impl_npu, extension/custom_op.cpp:115-152).
at::Tensor spmm_ascend_cube_impl(const at::Tensor& Crowptr, const at::Tensor& Ccol_ids,
                                 const at::Tensor& Cvalue, const at::Tensor& Vrowptr,
                                 const at::Tensor& Vcol_ids, const at::Tensor& Vvalue,
                                 const at::Tensor& dense, const at::Tensor& Cstart,
                                 const at::Tensor& Vstart) {
  TORCH_CHECK_GPU(Crowptr);
  TORCH_CHECK_GPU(Ccol_ids);
  TORCH_CHECK_GPU(Cvalue);
  TORCH_CHECK_GPU(Vrowptr);
  TORCH_CHECK_GPU(Vcol_ids);
  TORCH_CHECK_GPU(Vvalue);
  TORCH_CHECK_GPU(dense);
  TORCH_CHECK_GPU(Cstart);
  TORCH_CHECK_GPU(Vstart);
  TORCH_CHECK(Crowptr.dim() == 1, "Crow must be a 1D Tensor, but got: ", Crowptr.dim());
  TORCH_CHECK(Ccol_ids.dim() == 1, "Ccol_ids must be a 1D Tensor, but got: ", Ccol_ids.dim());
  TORCH_CHECK(Cvalue.dim() == 1, "Cvalue must be a 1D Tensor, but got: ", Cvalue.dim());
  TORCH_CHECK(Vrowptr.dim() == 1, "Vrow must be a 1D Tensor, but got: ", Vrowptr.dim());
  TORCH_CHECK(Vcol_ids.dim() == 1, "Vcol_ids must be a 1D Tensor, but got: ", Vcol_ids.dim());
  TORCH_CHECK(Vvalue.dim() == 1, "Vvalue must be a 1D Tensor, but got: ", Vvalue.dim());
  TORCH_CHECK(dense.dim() == 2, "dense must be a 2D Tensor, but got: ", dense.dim());
  TORCH_CHECK(Cstart.dim() == 1, "Cstart must be a 1D Tensor, but got: ", Cstart.dim());
  TORCH_CHECK(Vstart.dim() == 1, "Vstart must be a 1D Tensor, but got: ", Vstart.dim());
  check_dense_contract(dense, 16, "spmm_ascend_cube");
  check_value_contract(Cvalue, dense, "Cvalue");
  check_value_contract(Vvalue, dense, "Vvalue");
  return run_mixed(Crowptr, Ccol_ids, Cvalue, Vrowptr, Vcol_ids, Vvalue, dense, "spmm_ascend_cube");
}

// Shared checks of the mixed-op ablation aliases
// (reference: prepare_spmm_mixed_ablation_result, extension/custom_op.cpp:183-227).
at::Tensor mixed_ablation(const at::Tensor& Crowptr, const at::Tensor& Ccol_ids,
                          const at::Tensor& Cvalue, const at::Tensor& Vrowptr,
                          const at::Tensor& Vcol_ids, const at::Tensor& Vvalue,
                          const at::Tensor& dense, const at::Tensor& Cstart,
                          const at::Tensor& Vstart, const char* op_name) {
  TORCH_CHECK_GPU(Crowptr);
  TORCH_CHECK_GPU(Ccol_ids);
  TORCH_CHECK_GPU(Cvalue);
  TORCH_CHECK_GPU(Vrowptr);
  TORCH_CHECK_GPU(Vcol_ids);
  TORCH_CHECK_GPU(Vvalue);
  TORCH_CHECK_GPU(dense);
  TORCH_CHECK_GPU(Cstart);
  TORCH_CHECK_GPU(Vstart);
  TORCH_CHECK(Crowptr.dim() == 1, op_name, ": Crowptr must be one-dimensional");
  TORCH_CHECK(Ccol_ids.dim() == 1, op_name, ": Ccol_ids must be one-dimensional");
  TORCH_CHECK(Cvalue.dim() == 1, op_name, ": Cvalue must be one-dimensional");
  TORCH_CHECK(Vrowptr.dim() == 1, op_name, ": Vrowptr must be one-dimensional");
  TORCH_CHECK(Vcol_ids.dim() == 1, op_name, ": Vcol_ids must be one-dimensional");
  TORCH_CHECK(Vvalue.dim() == 1, op_name, ": Vvalue must be one-dimensional");
  TORCH_CHECK(dense.dim() == 2, op_name, ": dense must be two-dimensional");
  TORCH_CHECK(Cstart.dim() == 1, op_name, ": Cstart must be one-dimensional");
  TORCH_CHECK(Vstart.dim() == 1, op_name, ": Vstart must be one-dimensional");
  check_dense_contract(dense, 16, op_name);
  check_value_contract(Cvalue, dense, "Cvalue");
  check_value_contract(Vvalue, dense, "Vvalue");
  return run_mixed(Crowptr, Ccol_ids, Cvalue, Vrowptr, Vcol_ids, Vvalue, dense, op_name);
}

// The reference's ablation kernels compute the same sums with different
// pipelining (kernels/op_kernel/spmm_ascend_cube_aic_without_pipeline.cpp:6,
// spmm_ascend_cube_aiv_mb.cpp:822,851); on MI355X they share the mixed kernels.
at::Tensor spmm_ascend_cube_aic_without_pipeline_impl(
    const at::Tensor& Crowptr, const at::Tensor& Ccol_ids, const at::Tensor& Cvalue,
    const at::Tensor& Vrowptr, const at::Tensor& Vcol_ids, const at::Tensor& Vvalue,
    const at::Tensor& dense, const at::Tensor& Cstart, const at::Tensor& Vstart) {
  return mixed_ablation(Crowptr, Ccol_ids, Cvalue, Vrowptr, Vcol_ids, Vvalue, dense, Cstart, Vstart,
                        "spmm_ascend_cube_aic_without_pipeline");
}

at::Tensor spmm_ascend_cube_aiv_mb_impl(const at::Tensor& Crowptr, const at::Tensor& Ccol_ids,
                                        const at::Tensor& Cvalue, const at::Tensor& Vrowptr,
                                        const at::Tensor& Vcol_ids, const at::Tensor& Vvalue,
                                        const at::Tensor& dense, const at::Tensor& Cstart,
                                        const at::Tensor& Vstart) {
  return mixed_ablation(Crowptr, Ccol_ids, Cvalue, Vrowptr, Vcol_ids, Vvalue, dense, Cstart, Vstart,
                        "spmm_ascend_cube_aiv_mb");
}

// spmm_csr_aiv_mb_batch (reference: extension/custom_op.cpp:155-181): same
// sums as spmm_csr, so it runs the same gather kernel.
at::Tensor spmm_csr_aiv_mb_batch_impl(const at::Tensor& rowptr, const at::Tensor& col,
                                      const at::Tensor& value, const at::Tensor& dense,
                                      const at::Tensor& start) {
  const char* op_name = "spmm_csr_aiv_mb_batch";
  TORCH_CHECK_GPU(rowptr);
  TORCH_CHECK_GPU(col);
  TORCH_CHECK_GPU(value);
  TORCH_CHECK_GPU(dense);
  TORCH_CHECK_GPU(start);
  TORCH_CHECK(rowptr.dim() == 1, op_name, ": rowptr must be one-dimensional");
  TORCH_CHECK(col.dim() == 1, op_name, ": col must be one-dimensional");
  TORCH_CHECK(value.dim() == 1, op_name, ": value must be one-dimensional");
  TORCH_CHECK(dense.dim() == 2, op_name, ": dense must be two-dimensional");
  TORCH_CHECK(start.dim() == 1, op_name, ": start must be one-dimensional");
  check_dense_contract(dense, dense.scalar_type() == at::kHalf ? 16 : 8, op_name);
  check_value_contract(value, dense, "value");
  TORCH_CHECK(col.size(0) == value.size(0), op_name, ": col and value must have equal length");
  return spmm_csr_impl(rowptr, col, value, dense, start);
}

// spmm_cube, the legacy window-encoded operator (reference: spmm_cube_impl_npu,
// extension/custom_op.cpp:91-113): rowptr indexes 16-row windows, col holds
// (dense row << 4) | row in window.  Output [16 * windows, D].
at::Tensor spmm_cube_impl(const at::Tensor& rowptr, const at::Tensor& col, const at::Tensor& value,
                          const at::Tensor& dense, const at::Tensor& start) {
  TORCH_CHECK_GPU(rowptr);
  TORCH_CHECK_GPU(col);
  TORCH_CHECK_GPU(value);
  TORCH_CHECK_GPU(dense);
  TORCH_CHECK_GPU(start);
  TORCH_CHECK(rowptr.dim() == 1, "row must be a 1D Tensor, but got: ", rowptr.dim());
  TORCH_CHECK(col.dim() == 1, "col must be a 1D Tensor, but got: ", col.dim());
  TORCH_CHECK(value.dim() == 1, "value must be a 1D Tensor, but got: ", value.dim());
  TORCH_CHECK(dense.dim() == 2, "dense must be a 2D Tensor, but got: ", dense.dim());
  TORCH_CHECK(start.dim() == 1, "start must be a 1D Tensor, but got: ", start.dim());
  check_dense_contract(dense, 16, "spmm_cube");
  check_value_contract(value, dense, "value");
  const int64_t nnz1 = col.size(0), nnz2 = value.size(0);
  TORCH_CHECK(nnz1 == nnz2, "col and value must be same size, but got different: ", nnz1 - nnz2);
  TORCH_CHECK(rowptr.size(0) >= 1, "row must hold at least one entry");
  const int32_t it = index_type_of(rowptr, "rowptr");
  TORCH_CHECK(index_type_of(col, "col") == it, "rowptr and col must have the same dtype");
  check_same_device(rowptr, dense, "rowptr");
  check_same_device(col, dense, "col");
  check_same_device(value, dense, "value");

  c10::DeviceGuard guard(dense.device());
  const at::Tensor rp = rowptr.contiguous(), cl = col.contiguous();
  const at::Tensor dn = aligned(dense);
  const int64_t W = rowptr.size(0) - 1, D = dense.size(1);
  auto result = at::empty({16 * W, D}, dense.options());
  spmm_cube_op_desc d{W, nnz1, dense.size(0), D, it, value_type_of(dense)};
  size_t ws_bytes = 0;
  raise_status(spmm_cube_op_workspace(&d, &ws_bytes), "spmm_cube");
  at::Tensor ws = workspace(dense, ws_bytes);
  raise_status(spmm_cube_op_run(&d, rp.data_ptr(), cl.data_ptr(), value.data_ptr(), dn.data_ptr(),
                                result.data_ptr(), ws.data_ptr(), ws_bytes, current_stream(dense)),
               "spmm_cube");
  return result;
}

// Row permutation helpers used by spmm_npu.pack_node_tensor / restore_node_tensor.
at::Tensor pack_rows(const at::Tensor& tensor, const at::Tensor& inv, int64_t packed_rows) {
  TORCH_CHECK_GPU(tensor);
  TORCH_CHECK(inv.device() == tensor.device() && inv.scalar_type() == at::kLong && inv.dim() == 1,
              "pack_rows: inv_permutation must be a 1-D int64 tensor on the tensor's device");
  TORCH_CHECK(tensor.dim() >= 1 && inv.size(0) == tensor.size(0), "pack_rows: one inv entry per row");
  c10::DeviceGuard guard(tensor.device());
  const at::Tensor src = tensor.contiguous(), iv = inv.contiguous();
  std::vector<int64_t> shape(tensor.sizes().begin(), tensor.sizes().end());
  shape[0] = packed_rows;
  auto packed = at::empty(shape, tensor.options());
  const int64_t rows = tensor.size(0);
  const int64_t row_bytes = rows > 0 ? src.numel() / rows * src.element_size()
                                     : (packed_rows > 0 ? packed.numel() / packed_rows * packed.element_size() : 0);
  const size_t ws_bytes = spmm_pack_workspace(packed_rows);
  at::Tensor ws = workspace(tensor, ws_bytes);
  raise_status(spmm_pack_rows(src.data_ptr(), rows, row_bytes, iv.data_ptr<int64_t>(),
                              packed.data_ptr(), packed_rows, ws.data_ptr(), ws_bytes,
                              current_stream(tensor)),
               "pack_node_tensor");
  return packed;
}

at::Tensor restore_rows(const at::Tensor& packed, const at::Tensor& inv) {
  TORCH_CHECK_GPU(packed);
  TORCH_CHECK(inv.device() == packed.device() && inv.scalar_type() == at::kLong && inv.dim() == 1,
              "restore_rows: inv_permutation must be a 1-D int64 tensor on the tensor's device");
  TORCH_CHECK(packed.dim() >= 1, "restore_rows: packed tensor needs a leading dimension");
  c10::DeviceGuard guard(packed.device());
  const at::Tensor src = packed.contiguous(), iv = inv.contiguous();
  std::vector<int64_t> shape(packed.sizes().begin(), packed.sizes().end());
  shape[0] = inv.size(0);
  auto out = at::empty(shape, packed.options());
  const int64_t packed_rows = packed.size(0);
  const int64_t row_bytes = out.size(0) > 0 ? out.numel() / out.size(0) * out.element_size() : 0;
  raise_status(spmm_restore_rows(src.data_ptr(), packed_rows, row_bytes, iv.data_ptr<int64_t>(),
                                 inv.size(0), out.data_ptr(), current_stream(packed)),
               "restore_node_tensor");
  return out;
}

// ---------------------------------------------------------------------------
// Preprocessing (layout conversion and task mapping) on the GPU.
//
// The reference runs these on the host and returns CPU tensors
// (extension/custom_op.cpp:561-592, 714-746, 1112-1137, 1390-1412).  Here
// inputs on the CPU are copied to the current GPU, processed by the library's
// device pipelines and the results copied back to the CPU (so callers that
// expect CPU dicts keep working); inputs already on a GPU give GPU results.
namespace {

struct DeviceCsr {
  at::Tensor crow, col, val;
  bool to_cpu;
  c10::Device device{c10::kCPU};
};

DeviceCsr to_device(const at::Tensor& crow_ptr, const at::Tensor& col_indices, const at::Tensor& values,
                    int64_t nrows, const char* op) {
  TORCH_CHECK(crow_ptr.dim() == 1 && col_indices.dim() == 1 && values.dim() == 1, op,
              ": crow_ptr, col_indices and values must be 1-D");
  TORCH_CHECK(crow_ptr.scalar_type() == at::kInt || crow_ptr.scalar_type() == at::kLong, op,
              ": index tensors must be int32 or int64");
  TORCH_CHECK(col_indices.scalar_type() == crow_ptr.scalar_type(), op,
              ": col_indices must have the dtype of crow_ptr");
  TORCH_CHECK(values.scalar_type() == at::kHalf || values.scalar_type() == at::kFloat ||
                  values.scalar_type() == at::kDouble,
              op, ": values must be float16, float32 or float64");
  if (nrows < 0 || crow_ptr.numel() < nrows + 1)
    throw std::invalid_argument(std::string(op) + ": crow_ptr must hold nrows + 1 entries");
  if (values.numel() < col_indices.numel())
    throw std::invalid_argument(std::string(op) + ": values must hold one entry per column index");
  DeviceCsr d;
  d.to_cpu = !crow_ptr.device().is_cuda();
  if (d.to_cpu) {
    TORCH_CHECK(at::cuda::is_available(), op, " runs on the GPU, and no GPU is available");
    d.device = c10::Device(c10::kCUDA, c10::hip::current_device());
  } else {
    d.device = crow_ptr.device();
  }
  d.crow = crow_ptr.to(d.device).contiguous();
  d.col = col_indices.to(d.device).contiguous();
  d.val = values.to(d.device).contiguous();
  return d;
}

spmm_csr_matrix describe(const DeviceCsr& d, int64_t nrows, int64_t ncols) {
  spmm_csr_matrix m;
  m.rows = nrows;
  m.cols = ncols;
  m.nnz = d.col.numel();
  m.index_type = d.crow.scalar_type() == at::kInt ? SPMM_INDEX_I32 : SPMM_INDEX_I64;
  m.value_type = d.val.scalar_type() == at::kHalf
                     ? SPMM_VALUE_F16
                     : (d.val.scalar_type() == at::kFloat ? SPMM_VALUE_F32 : SPMM_VALUE_F64);
  m.rowptr = d.crow.data_ptr();
  m.col = d.col.data_ptr();
  m.value = d.val.data_ptr();
  return m;
}

at::Tensor idx_tensor(const DeviceCsr& d, int64_t n) { return at::empty({n}, d.crow.options()); }
at::Tensor val_tensor(const DeviceCsr& d, int64_t n) { return at::empty({n}, d.val.options()); }

std::map<std::string, at::Tensor> finish(std::map<std::string, at::Tensor> out, const DeviceCsr& d) {
  if (d.to_cpu)
    for (auto& kv : out) kv.second = kv.second.cpu();
  return out;
}

void* ptr(const at::Tensor& t) { return t.numel() ? t.data_ptr() : nullptr; }

}  // namespace

// csr_to_bcsr (reference: ToBCSR / csr_to_bcsr, extension/custom_op.cpp:594-746).
std::map<std::string, at::Tensor> csr_to_bcsr(at::Tensor crow_ptr, at::Tensor col_indices, at::Tensor values,
                                              int64_t nrows, int64_t ncols, int64_t window_size) {
  DeviceCsr d = to_device(crow_ptr, col_indices, values, nrows, "csr_to_bcsr");
  c10::DeviceGuard guard(d.device);
  const spmm_csr_matrix m = describe(d, nrows, ncols);
  spmm_stream s = current_stream(d.crow);
  const size_t ws_bytes = spmm_bcsr_workspace(&m, window_size);
  at::Tensor ws = workspace(d.crow, ws_bytes);
  int64_t blocks = 0;
  raise_status(spmm_bcsr_plan(&m, window_size, ws.data_ptr(), ws_bytes, s, &blocks), "csr_to_bcsr");
  const int64_t nwin = (nrows + window_size - 1) / window_size;
  std::map<std::string, at::Tensor> out;
  out["crow_window_ptr"] = idx_tensor(d, nwin + 1);
  out["unique_col_ids"] = idx_tensor(d, blocks);
  out["value"] = val_tensor(d, 16 * blocks);
  raise_status(spmm_bcsr_fill(&m, window_size, ws.data_ptr(), ws_bytes, ptr(out["crow_window_ptr"]),
                              ptr(out["unique_col_ids"]), ptr(out["value"]), s),
               "csr_to_bcsr");
  return finish(std::move(out), d);
}

// csr_to_ascend_cube (reference: your_logic_kernel, extension/custom_op.cpp:429-592).
std::map<std::string, at::Tensor> csr_to_ascend_cube(at::Tensor crow_ptr, at::Tensor col_indices,
                                                     at::Tensor values, int64_t nrows, int64_t ncols,
                                                     int64_t window_size) {
  DeviceCsr d = to_device(crow_ptr, col_indices, values, nrows, "csr_to_ascend_cube");
  c10::DeviceGuard guard(d.device);
  const spmm_csr_matrix m = describe(d, nrows, ncols);
  spmm_stream s = current_stream(d.crow);
  const size_t ws_bytes = spmm_cube_workspace(&m, window_size);
  at::Tensor ws = workspace(d.crow, ws_bytes);
  int64_t tiles = 0;
  raise_status(spmm_cube_plan(&m, window_size, ws.data_ptr(), ws_bytes, s, &tiles), "csr_to_ascend_cube");
  const int64_t nwin = (nrows + window_size - 1) / window_size;
  std::map<std::string, at::Tensor> out;
  out["crow_window_ptr"] = idx_tensor(d, nwin + 1);
  out["unique_col_ids"] = idx_tensor(d, 16 * tiles);
  out["value"] = val_tensor(d, 256 * tiles);
  raise_status(spmm_cube_fill(&m, window_size, ws.data_ptr(), ws_bytes, ptr(out["crow_window_ptr"]),
                              ptr(out["unique_col_ids"]), ptr(out["value"]), s),
               "csr_to_ascend_cube");
  return finish(std::move(out), d);
}

// block_level_split (reference: hybrid_split_impl, extension/custom_op.cpp:1146-1348, 1390-1412).
std::map<std::string, at::Tensor> block_level_split(at::Tensor crow_ptr, at::Tensor col_indices,
                                                    at::Tensor values, int64_t nrows, int64_t ncols,
                                                    double a, int64_t window_size) {
  DeviceCsr d = to_device(crow_ptr, col_indices, values, nrows, "block_level_split");
  c10::DeviceGuard guard(d.device);
  const spmm_csr_matrix m = describe(d, nrows, ncols);
  spmm_stream s = current_stream(d.crow);
  const size_t ws_bytes = spmm_hybrid_workspace(&m, window_size);
  at::Tensor ws = workspace(d.crow, ws_bytes);
  int64_t kept = 0, vnnz = 0;
  raise_status(spmm_hybrid_plan(&m, a, window_size, ws.data_ptr(), ws_bytes, s, &kept, &vnnz),
               "block_level_split");
  const int64_t nwin = window_size > 0 ? (nrows + window_size - 1) / window_size : 0;
  std::map<std::string, at::Tensor> out;
  out["crow_window_ptr"] = idx_tensor(d, nwin + 1);
  out["unique_col_ids"] = idx_tensor(d, kept);
  out["value"] = val_tensor(d, kept * window_size);
  out["vrow_window_ptr"] = idx_tensor(d, nwin * window_size + 1);
  out["vcol_indices"] = idx_tensor(d, vnnz);
  out["vvalue"] = val_tensor(d, vnnz);
  raise_status(spmm_hybrid_fill(&m, a, window_size, ws.data_ptr(), ws_bytes, ptr(out["crow_window_ptr"]),
                                ptr(out["unique_col_ids"]), ptr(out["value"]), ptr(out["vrow_window_ptr"]),
                                ptr(out["vcol_indices"]), ptr(out["vvalue"]), s),
               "block_level_split");
  return finish(std::move(out), d);
}

// preprocess (reference: taskmapping, extension/custom_op.cpp:749-1137).
std::map<std::string, at::Tensor> preprocess(at::Tensor crow_ptr, at::Tensor col_indices, at::Tensor values,
                                             int64_t nrows, int64_t ncols, int64_t window_size,
                                             bool graph_layout) {
  DeviceCsr d = to_device(crow_ptr, col_indices, values, nrows, "preprocess");
  c10::DeviceGuard guard(d.device);
  const spmm_csr_matrix m = describe(d, nrows, ncols);
  spmm_stream s = current_stream(d.crow);
  TORCH_CHECK(window_size == 16, "Ascend-SpMM requires a 16-row window");
  const size_t ws_bytes = spmm_taskmap_workspace(&m, window_size, graph_layout ? 1 : 0);
  at::Tensor ws = workspace(d.crow, ws_bytes);
  spmm_taskmap_info info;
  raise_status(spmm_taskmap_plan(&m, window_size, graph_layout ? 1 : 0, ws.data_ptr(), ws_bytes, s, &info),
               "preprocess");
  const bool layout = info.packed_layout_supported != 0;
  std::map<std::string, at::Tensor> out;
  out["crow_window_ptr"] = idx_tensor(d, info.aic_windows + 1);
  out["unique_col_ids"] = idx_tensor(d, info.aic_blocks);
  out["value"] = val_tensor(d, 16 * info.aic_blocks);
  out["vrow_window_ptr"] = idx_tensor(d, info.packed_rows + 1);
  out["vcol_indices"] = idx_tensor(d, info.vector_nnz);
  out["vvalue"] = val_tensor(d, info.vector_nnz);
  out["renumbered_unique_col_ids"] = idx_tensor(d, layout ? info.aic_blocks : 0);
  out["renumbered_vcol_indices"] = idx_tensor(d, layout ? info.vector_nnz : 0);
  out["transpose_crow_window_ptr"] = idx_tensor(d, layout ? info.t_windows + 1 : 0);
  out["transpose_unique_col_ids"] = idx_tensor(d, info.t_blocks);
  out["transpose_value"] = val_tensor(d, 16 * info.t_blocks);
  out["transpose_vrow_window_ptr"] = idx_tensor(d, layout ? info.t_rows + 1 : 0);
  out["transpose_vcol_indices"] = idx_tensor(d, info.t_vector_nnz);
  out["transpose_vvalue"] = val_tensor(d, info.t_vector_nnz);
  const auto i64 = d.crow.options().dtype(at::kLong);
  out["permutation"] = at::empty({info.packed_rows}, i64);
  out["inv_permutation"] = at::empty({nrows}, i64);
  spmm_taskmap_out o;
  o.crow_window_ptr = ptr(out["crow_window_ptr"]);
  o.unique_col_ids = ptr(out["unique_col_ids"]);
  o.value = ptr(out["value"]);
  o.vrow_window_ptr = ptr(out["vrow_window_ptr"]);
  o.vcol_indices = ptr(out["vcol_indices"]);
  o.vvalue = ptr(out["vvalue"]);
  o.renumbered_unique_col_ids = ptr(out["renumbered_unique_col_ids"]);
  o.renumbered_vcol_indices = ptr(out["renumbered_vcol_indices"]);
  o.transpose_crow_window_ptr = ptr(out["transpose_crow_window_ptr"]);
  o.transpose_unique_col_ids = ptr(out["transpose_unique_col_ids"]);
  o.transpose_value = ptr(out["transpose_value"]);
  o.transpose_vrow_window_ptr = ptr(out["transpose_vrow_window_ptr"]);
  o.transpose_vcol_indices = ptr(out["transpose_vcol_indices"]);
  o.transpose_vvalue = ptr(out["transpose_vvalue"]);
  o.permutation = static_cast<int64_t*>(ptr(out["permutation"]));
  o.inv_permutation = static_cast<int64_t*>(ptr(out["inv_permutation"]));
  raise_status(spmm_taskmap_fill(&m, window_size, graph_layout ? 1 : 0, ws.data_ptr(), ws_bytes, &o, s),
               "preprocess");
  auto scalar = [&](int64_t v) { return at::full({1}, v, i64); };
  auto dscalar = [&](double v) { return at::full({1}, v, d.crow.options().dtype(at::kDouble)); };
  out["packed_rows"] = scalar(info.packed_rows);
  out["packed_layout_supported"] = scalar(info.packed_layout_supported);
  out["marginal_window"] = scalar(info.marginal_window);
  out["marginal_aic_blocks"] = scalar(info.marginal_aic_blocks);
  out["marginal_total_blocks"] = scalar(info.marginal_total_blocks);
  out["estimated_aic_cost"] = dscalar(info.estimated_aic_cost);
  out["estimated_aiv_cost"] = dscalar(info.estimated_aiv_cost);
  out["estimated_max_cost"] = dscalar(info.estimated_max_cost);
  out["shared_windows"] = scalar(info.shared_windows);
  return finish(std::move(out), d);
}

// Schemas as in the reference (extension/custom_op.cpp:266-273).
TORCH_LIBRARY(myops, m) {
  m.def("spmm_csr(Tensor rowptr, Tensor col, Tensor value, Tensor dense, Tensor start) -> Tensor");
  m.def("spmm_cube(Tensor rowptr, Tensor col, Tensor value, Tensor dense, Tensor start) -> Tensor");
  m.def("spmm_ascend_cube(Tensor Crowptr, Tensor Ccol_ids, Tensor Cvalue, Tensor Vrowptr, Tensor Vcol_ids, Tensor Vvalue, Tensor dense, Tensor Cstart, Tensor Vstart) -> Tensor");
  m.def("spmm_csr_aiv_mb_batch(Tensor rowptr, Tensor col, Tensor value, Tensor dense, Tensor start) -> Tensor");
  m.def("spmm_ascend_cube_aic_without_pipeline(Tensor Crowptr, Tensor Ccol_ids, Tensor Cvalue, Tensor Vrowptr, Tensor Vcol_ids, Tensor Vvalue, Tensor dense, Tensor Cstart, Tensor Vstart) -> Tensor");
  m.def("spmm_ascend_cube_aiv_mb(Tensor Crowptr, Tensor Ccol_ids, Tensor Cvalue, Tensor Vrowptr, Tensor Vcol_ids, Tensor Vvalue, Tensor dense, Tensor Cstart, Tensor Vstart) -> Tensor");
}

// The reference implements them on PrivateUse1 (the NPU key,
// extension/custom_op.cpp:276-283); on ROCm the GPU key is CUDA.
TORCH_LIBRARY_IMPL(myops, CUDA, m) {
  m.impl("spmm_csr", &spmm_csr_impl);
  m.impl("spmm_cube", &spmm_cube_impl);
  m.impl("spmm_ascend_cube", &spmm_ascend_cube_impl);
  m.impl("spmm_csr_aiv_mb_batch", &spmm_csr_aiv_mb_batch_impl);
  m.impl("spmm_ascend_cube_aic_without_pipeline", &spmm_ascend_cube_aic_without_pipeline_impl);
  m.impl("spmm_ascend_cube_aiv_mb", &spmm_ascend_cube_aiv_mb_impl);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("spmm_csr", &spmm_csr_impl,
        "GPU CSR SpMM; FP16 width divisible by 16 with MAXD=1024, FP32 width divisible by 8 with MAXD=512");
  m.def("spmm_cube", &spmm_cube_impl,
        "GPU window-encoded SpMM (col = (dense row << 4) | row in window) on MFMA; width divisible by 16, MAXD=1024 for FP16 and 512 for FP32");
  m.def("spmm_ascend_cube", &spmm_ascend_cube_impl,
        "GPU mixed block(MFMA)/vector SpMM; width divisible by 16, MAXD=1024 for FP16 and 512 for FP32");
  m.def("spmm_ascend_cube_aic_without_pipeline", &spmm_ascend_cube_aic_without_pipeline_impl,
        "Alias of spmm_ascend_cube (the reference's AIC g=1 ablation)");
  m.def("spmm_ascend_cube_aiv_mb", &spmm_ascend_cube_aiv_mb_impl,
        "Alias of spmm_ascend_cube (the reference's AIV multiple-buffer ablation)");
  m.def("spmm_csr_aiv_mb_batch", &spmm_csr_aiv_mb_batch_impl,
        "Alias of spmm_csr (the reference's AIV batch ablation)");
  m.def("csr_to_ascend_cube", &csr_to_ascend_cube,
        R"doc(
    Convert CSR sparse matrix to Ascend Cube format (16x16 tiles), on the GPU.
    Requires: each row's col_indices must be sorted in ascending order.

    Returns dict with keys:
        crow_window_ptr   Tensor  [nwindows + 1]
        unique_col_ids    Tensor  [total_blocks * 16]
        value             Tensor  [total_blocks * 16 * 16]
    )doc");
  m.def("csr_to_bcsr", &csr_to_bcsr,
        R"doc(
    Convert CSR sparse matrix to BCSR(16 * 1), on the GPU.
    Requires: each row's col_indices must be sorted in ascending order.

    Returns dict with keys:
        crow_window_ptr   Tensor  [nwindows + 1]
        unique_col_ids    Tensor  [total_blocks]
        value             Tensor  [total_blocks * 16]
    )doc");
  m.def("preprocess", &preprocess,
        R"doc(
    Partition coalesced CSR by the calibrated AIC/AIV bandwidths (295/505 GB/s),
    on the GPU, with results identical to the reference's host implementation.
    All dense windows before the marginal window go to the block (MFMA) part,
    all sparse windows after it to the vector part, and only the marginal
    window is split at block granularity, minimising max(block cost, vector cost).
    graph_layout=True on a square graph also returns P*A*P^T (renumbered_*)
    and its fixed-layout transpose P*A^T*P^T (transpose_*).  Keys as the
    reference: packed AIC/AIV tensors, permutation, inv_permutation,
    packed_rows, packed_layout_supported, marginal_window,
    marginal_aic_blocks, marginal_total_blocks, estimated_{aic,aiv,max}_cost,
    shared_windows.
    )doc",
        pybind11::arg("crow_ptr"), pybind11::arg("col_indices"), pybind11::arg("values"),
        pybind11::arg("nrows"), pybind11::arg("ncols"), pybind11::arg("window_size") = 16,
        pybind11::arg("graph_layout") = false);
  m.def("block_level_split", &block_level_split,
        "Split CSR into (16,1)-BSR + CSR hybrid dict by block density (GPU)");
  m.def("pack_rows", &pack_rows, "packed[inv[i]] = tensor[i]; other rows zero (GPU)");
  m.def("restore_rows", &restore_rows, "out[i] = packed[inv[i]] (GPU)");
  m.def("library_version", []() { return std::string(spmm_version()); });
}
