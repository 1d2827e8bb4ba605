// csr_matmul.cpp - C++ primitive layer for CSR SpMM with a dense RHS.
#include "sparse/csr_matmul/csr_matmul.h"

#include <stdexcept>

#include "common/validate.h"

namespace msx {

void csr_matmul(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                const ArrayView &rhs, const ArrayView &out, int64_t n_rows, int64_t n_cols,
                const msx_csr_plan *plan, const ExecContext &ctx) {
  // reference: src/sparse/csr_matmul/csr_matmul.cpp:386-405
  if (n_rows < 0 || n_cols < 0)
    throw std::invalid_argument("csr_matmul shape dimensions must be non-negative.");
  if (n_rows >= 2147483647 || n_cols > 2147483647)
    throw std::invalid_argument("csr_matmul shape dimensions must fit in int32.");
  require_rank(data, 1, "csr_matmul data");
  require_rank(indices, 1, "csr_matmul indices");
  require_rank(indptr, 1, "csr_matmul indptr");
  require_rank(rhs, 2, "csr_matmul rhs");
  require_same_value_dtype(data, rhs, "csr_matmul data", "csr_matmul rhs");
  require_same_index_dtype(indices, indptr, "csr_matmul indices", "csr_matmul indptr");
  require_size(indptr, n_rows + 1, "csr_matmul indptr");
  if (rhs.shape[0] != n_cols)
    throw std::invalid_argument(
        "csr_matmul rhs first dimension must equal the sparse matrix column count.");
  if (indices.size() != data.size())
    throw std::invalid_argument("csr_matmul data and indices must have equal length.");
  require_same_device({&data, &indices, &indptr, &rhs, &out}, "csr_matmul");
  const int64_t k = rhs.shape[1];
  if (out.ndim != 2 || out.shape[0] != n_rows || out.shape[1] != k || out.dtype != data.dtype)
    throw std::invalid_argument("csr_matmul out must be (n_rows, k) with the dtype of data.");
  for (const ArrayView *a : {&data, &indices, &indptr, &rhs, &out})
    require_contiguous(*a, "csr_matmul operand");

  const msx_vtype vt = to_vtype(data.dtype);
  const msx_itype it = to_itype(indices.dtype);
  const int64_t nnz = data.size();
  if (data.device >= 0) {
    check_status(msx_csr_spmm(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr, indptr.ptr, k,
                              rhs.ptr, k, out.ptr, k, plan, ctx.stream),
                 "csr_matmul");
  } else {
    check_status(msx_csr_spmm_cpu(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr, indptr.ptr,
                                  k, rhs.ptr, out.ptr, ctx.n_threads),
                 "csr_matmul");
  }
}

}  // namespace msx
