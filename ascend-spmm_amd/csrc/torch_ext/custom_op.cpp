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

#include <stdexcept>
#include <string>

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

// The kernels read dense in 16-byte pieces; a view at an odd offset is copied.
at::Tensor aligned(const at::Tensor& dense) {
  return reinterpret_cast<uintptr_t>(dense.data_ptr()) % 16 == 0 ? dense : dense.clone();
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
  const at::Tensor dn = aligned(dense);
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
  raise_status(spmm_mixed_run(&d, crp.data_ptr(), ccl.data_ptr(), Cvalue.data_ptr(), vrp.data_ptr(),
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

// Schemas as in the reference (extension/custom_op.cpp:266-273); the
// reference's spmm_cube legacy operator is not provided.
TORCH_LIBRARY(myops, m) {
  m.def("spmm_csr(Tensor rowptr, Tensor col, Tensor value, Tensor dense, Tensor start) -> Tensor");
  m.def("spmm_ascend_cube(Tensor Crowptr, Tensor Ccol_ids, Tensor Cvalue, Tensor Vrowptr, Tensor Vcol_ids, Tensor Vvalue, Tensor dense, Tensor Cstart, Tensor Vstart) -> Tensor");
  m.def("spmm_csr_aiv_mb_batch(Tensor rowptr, Tensor col, Tensor value, Tensor dense, Tensor start) -> Tensor");
  m.def("spmm_ascend_cube_aic_without_pipeline(Tensor Crowptr, Tensor Ccol_ids, Tensor Cvalue, Tensor Vrowptr, Tensor Vcol_ids, Tensor Vvalue, Tensor dense, Tensor Cstart, Tensor Vstart) -> Tensor");
  m.def("spmm_ascend_cube_aiv_mb(Tensor Crowptr, Tensor Ccol_ids, Tensor Cvalue, Tensor Vrowptr, Tensor Vcol_ids, Tensor Vvalue, Tensor dense, Tensor Cstart, Tensor Vstart) -> Tensor");
}

// The reference implements them on PrivateUse1 (the NPU key,
// extension/custom_op.cpp:276-283); on ROCm the GPU key is CUDA.
TORCH_LIBRARY_IMPL(myops, CUDA, m) {
  m.impl("spmm_csr", &spmm_csr_impl);
  m.impl("spmm_ascend_cube", &spmm_ascend_cube_impl);
  m.impl("spmm_csr_aiv_mb_batch", &spmm_csr_aiv_mb_batch_impl);
  m.impl("spmm_ascend_cube_aic_without_pipeline", &spmm_ascend_cube_aic_without_pipeline_impl);
  m.impl("spmm_ascend_cube_aiv_mb", &spmm_ascend_cube_aiv_mb_impl);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("spmm_csr", &spmm_csr_impl,
        "GPU CSR SpMM; FP16 width divisible by 16 with MAXD=1024, FP32 width divisible by 8 with MAXD=512");
  m.def("spmm_ascend_cube", &spmm_ascend_cube_impl,
        "GPU mixed block(MFMA)/vector SpMM; width divisible by 16, MAXD=1024 for FP16 and 512 for FP32");
  m.def("spmm_ascend_cube_aic_without_pipeline", &spmm_ascend_cube_aic_without_pipeline_impl,
        "Alias of spmm_ascend_cube (the reference's AIC g=1 ablation)");
  m.def("spmm_ascend_cube_aiv_mb", &spmm_ascend_cube_aiv_mb_impl,
        "Alias of spmm_ascend_cube (the reference's AIV multiple-buffer ablation)");
  m.def("spmm_csr_aiv_mb_batch", &spmm_csr_aiv_mb_batch_impl,
        "Alias of spmm_csr (the reference's AIV batch ablation)");
  m.def("pack_rows", &pack_rows, "packed[inv[i]] = tensor[i]; other rows zero (GPU)");
  m.def("restore_rows", &restore_rows, "out[i] = packed[inv[i]] (GPU)");
  m.def("library_version", []() { return std::string(spmm_version()); });
}
