// csr_matvec.cpp - C++ primitive layer for CSR SpMV.
#include "sparse/csr_matvec/csr_matvec.h"

#include <stdexcept>

#include "common/validate.h"

namespace msx {

void csr_matvec(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                const ArrayView &x, const ArrayView &out, int64_t n_rows, int64_t n_cols,
                const msx_csr_plan *plan, const ExecContext &ctx) {
  // reference: src/sparse/csr_matvec/csr_matvec.cpp:329-345
  if (n_rows < 0 || n_cols < 0)
    throw std::invalid_argument("csr_matvec shape dimensions must be non-negative.");
  if (n_rows >= 2147483647 || n_cols > 2147483647)
    throw std::invalid_argument("csr_matvec shape dimensions must fit in int32.");
  require_rank(data, 1, "csr_matvec data");
  require_rank(indices, 1, "csr_matvec indices");
  require_rank(indptr, 1, "csr_matvec indptr");
  require_rank(x, 1, "csr_matvec x");
  require_same_value_dtype(data, x, "csr_matvec data", "csr_matvec x");
  require_same_index_dtype(indices, indptr, "csr_matvec indices", "csr_matvec indptr");
  require_size(indptr, n_rows + 1, "csr_matvec indptr");
  require_size(x, n_cols, "csr_matvec x");
  if (indices.size() != data.size())
    throw std::invalid_argument("csr_matvec data and indices must have equal length.");
  require_same_device({&data, &indices, &indptr, &x, &out}, "csr_matvec");
  require_rank(out, 1, "csr_matvec out");
  require_size(out, n_rows, "csr_matvec out");
  if (out.dtype != data.dtype)
    throw std::invalid_argument("csr_matvec out must have the dtype of data.");
  for (const ArrayView *a : {&data, &indices, &indptr, &x, &out})
    require_contiguous(*a, "csr_matvec operand");

  const msx_vtype vt = to_vtype(data.dtype);
  const msx_itype it = to_itype(indices.dtype);
  const int64_t nnz = data.size();
  if (data.device >= 0) {
    check_status(msx_csr_spmv(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr, indptr.ptr,
                              x.ptr, out.ptr, plan, ctx.stream),
                 "csr_matvec");
  } else {
    check_status(msx_csr_spmv_cpu(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr, indptr.ptr,
                                  x.ptr, out.ptr, ctx.n_threads),
                 "csr_matvec");
  }
}

}  // namespace msx
