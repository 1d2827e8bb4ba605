// csr_batched_matmul.cpp - C++ primitive layer for CSR times a batch of dense matrices.
#include "sparse/csr_batched_matmul/csr_batched_matmul.h"

#include <stdexcept>

#include "common/validate.h"

namespace msx {

void csr_batched_matmul(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                        const ArrayView &rhs, const ArrayView &out, int64_t n_rows, int64_t n_cols,
                        const ExecContext &ctx) {
  // reference: src/sparse/csr_batched_matmul/csr_batched_matmul.cpp:441-461
  if (n_rows < 0 || n_cols < 0)
    throw std::invalid_argument("csr_batched_matmul shape dimensions must be non-negative.");
  if (n_rows >= 2147483647 || n_cols > 2147483647)
    throw std::invalid_argument("csr_batched_matmul shape dimensions must fit in int32.");
  require_rank(data, 1, "csr_batched_matmul data");
  require_rank(indices, 1, "csr_batched_matmul indices");
  require_rank(indptr, 1, "csr_batched_matmul indptr");
  require_rank(rhs, 3, "csr_batched_matmul rhs");
  require_same_value_dtype(data, rhs, "csr_batched_matmul data", "csr_batched_matmul rhs");
  require_same_index_dtype(indices, indptr, "csr_batched_matmul indices",
                           "csr_batched_matmul indptr");
  require_size(indptr, n_rows + 1, "csr_batched_matmul indptr");
  if (rhs.shape[1] != n_cols)
    throw std::invalid_argument(
        "csr_batched_matmul rhs sparse dimension must equal the sparse matrix column count.");
  if (indices.size() != data.size())
    throw std::invalid_argument("csr_batched_matmul data and indices must have equal length.");
  require_same_device({&data, &indices, &indptr, &rhs, &out}, "csr_batched_matmul");
  const int64_t batch = rhs.shape[0], k = rhs.shape[2];
  if (out.ndim != 3 || out.shape[0] != batch || out.shape[1] != n_rows || out.shape[2] != k ||
      out.dtype != data.dtype)
    throw std::invalid_argument(
        "csr_batched_matmul out must be (batch, n_rows, k) with the dtype of data.");
  for (const ArrayView *a : {&data, &indices, &indptr, &rhs, &out})
    require_contiguous(*a, "csr_batched_matmul operand");

  const msx_vtype vt = to_vtype(data.dtype);
  const msx_itype it = to_itype(indices.dtype);
  const int64_t nnz = data.size();
  if (data.device >= 0) {
    check_status(msx_csr_batched_spmm(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr,
                                      indptr.ptr, batch, k, rhs.ptr, n_cols * k, k, out.ptr,
                                      n_rows * k, k, ctx.stream),
                 "csr_batched_matmul");
  } else {
    check_status(msx_csr_batched_spmm_cpu(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr,
                                          indptr.ptr, batch, k, rhs.ptr, out.ptr, ctx.n_threads),
                 "csr_batched_matmul");
  }
}

}  // namespace msx
