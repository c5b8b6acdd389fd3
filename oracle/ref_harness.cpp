// ref_harness.cpp — C entry points around the reference's own std-only
// headers, compiled from where they lie under the reference checkout:
//   extension/boundary_bucket_sort.h   (stable_bucket_sort_by_occupancy_desc)
//   extension/packed_column_reindex.h  (renumber_columns_for_packed_layout,
//                                       transpose_into_packed_layout)
// TEST INFRASTRUCTURE ONLY: built into oracle/_ref/ (never committed; the
// built library travels with the working tree to the GPU box like the other
// built libraries, but only the CPU tests load it) and used by tests to pin
// the oracle's restatement of these three functions against the reference's
// code.  Exceptions become status codes:
// 1 invalid_argument, 2 out_of_range, 3 overflow_error.
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "boundary_bucket_sort.h"
#include "packed_column_reindex.h"

#define REF_TRY try {
#define REF_CATCH                                      \
  }                                                    \
  catch (const std::invalid_argument&) { return 1; }   \
  catch (const std::out_of_range&) { return 2; }       \
  catch (const std::overflow_error&) { return 3; }     \
  return 0;

extern "C" {

int ref_bucket_sort(int64_t* columns, int64_t n, const int64_t* occupancy, int64_t nocc,
                    int64_t max_occupancy) {
  REF_TRY
  std::vector<int64_t> cols(columns, columns + n);
  std::vector<int64_t> occ(occupancy, occupancy + nocc);
  ascend_spmm::stable_bucket_sort_by_occupancy_desc(cols, occ, max_occupancy);
  std::memcpy(columns, cols.data(), sizeof(int64_t) * cols.size());
  REF_CATCH
}

int ref_renumber_i32(const int32_t* cols, int64_t n, const int64_t* inv, int64_t ninv,
                     int32_t* out) {
  REF_TRY
  std::vector<int32_t> c(cols, cols + n);
  std::vector<int64_t> iv(inv, inv + ninv);
  std::vector<int32_t> r = ascend_spmm::renumber_columns_for_packed_layout(c, iv);
  std::memcpy(out, r.data(), sizeof(int32_t) * r.size());
  REF_CATCH
}

int ref_renumber_i64(const int64_t* cols, int64_t n, const int64_t* inv, int64_t ninv,
                     int64_t* out) {
  REF_TRY
  std::vector<int64_t> c(cols, cols + n);
  std::vector<int64_t> iv(inv, inv + ninv);
  std::vector<int64_t> r = ascend_spmm::renumber_columns_for_packed_layout(c, iv);
  std::memcpy(out, r.data(), sizeof(int64_t) * r.size());
  REF_CATCH
}

// Values are 32-bit payloads (fp32 bits, or fp16 bits widened by the caller).
int ref_transpose(const int64_t* rowptr, int64_t nrowptr, const int64_t* cols,
                  const uint32_t* vals, int64_t nnz, const int64_t* inv, int64_t ninv,
                  int64_t packed_rows, int64_t* rowptrT, int64_t* colsT, uint32_t* valsT) {
  REF_TRY
  std::vector<int64_t> rp(rowptr, rowptr + nrowptr), c(cols, cols + nnz), iv(inv, inv + ninv);
  std::vector<uint32_t> v(vals, vals + nnz);
  std::vector<int64_t> rt, ct;
  std::vector<uint32_t> vt;
  ascend_spmm::transpose_into_packed_layout(rp, c, v, iv, static_cast<std::size_t>(packed_rows),
                                            rt, ct, vt);
  std::memcpy(rowptrT, rt.data(), sizeof(int64_t) * rt.size());
  if (!ct.empty()) {
    std::memcpy(colsT, ct.data(), sizeof(int64_t) * ct.size());
    std::memcpy(valsT, vt.data(), sizeof(uint32_t) * vt.size());
  }
  REF_CATCH
}

}  // extern "C"
