// csr_batched_matvec.cpp - C++ primitive layer for CSR times a batch of vectors.
#include "sparse/csr_batched_matvec/csr_batched_matvec.h"

#include <stdexcept>

#include "common/validate.h"

namespace msx {

void csr_batched_matvec(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                        const ArrayView &rhs, const ArrayView &out, int64_t n_rows, int64_t n_cols,
                        const ExecContext &ctx) {
  // reference: src/sparse/csr_batched_matvec/csr_batched_matvec.cpp:255-276
  if (n_rows < 0 || n_cols < 0)
    throw std::invalid_argument("csr_batched_matvec shape dimensions must be non-negative.");
  if (n_rows >= 2147483647 || n_cols > 2147483647)
    throw std::invalid_argument("csr_batched_matvec shape dimensions must fit in int32.");
  require_rank(data, 1, "csr_batched_matvec data");
  require_rank(indices, 1, "csr_batched_matvec indices");
  require_rank(indptr, 1, "csr_batched_matvec indptr");
  require_rank(rhs, 2, "csr_batched_matvec rhs");
  require_same_value_dtype(data, rhs, "csr_batched_matvec data", "csr_batched_matvec rhs");
  require_same_index_dtype(indices, indptr, "csr_batched_matvec indices",
                           "csr_batched_matvec indptr");
  require_size(indptr, n_rows + 1, "csr_batched_matvec indptr");
  if (rhs.shape[1] != n_cols)
    throw std::invalid_argument(
        "csr_batched_matvec rhs last dimension must equal the sparse matrix column count.");
  if (indices.size() != data.size())
    throw std::invalid_argument("csr_batched_matvec data and indices must have equal length.");
  require_same_device({&data, &indices, &indptr, &rhs, &out}, "csr_batched_matvec");
  const int64_t batch = rhs.shape[0];
  if (out.ndim != 2 || out.shape[0] != batch || out.shape[1] != n_rows || out.dtype != data.dtype)
    throw std::invalid_argument(
        "csr_batched_matvec out must be (batch, n_rows) with the dtype of data.");
  for (const ArrayView *a : {&data, &indices, &indptr, &rhs, &out})
    require_contiguous(*a, "csr_batched_matvec operand");

  const msx_vtype vt = to_vtype(data.dtype);
  const msx_itype it = to_itype(indices.dtype);
  const int64_t nnz = data.size();
  if (data.device >= 0) {
    check_status(msx_csr_batched_spmv(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr,
                                      indptr.ptr, batch, rhs.ptr, n_cols, out.ptr, n_rows,
                                      ctx.stream),
                 "csr_batched_matvec");
  } else {
    check_status(msx_csr_batched_spmv_cpu(vt, it, n_rows, n_cols, nnz, data.ptr, indices.ptr,
                                          indptr.ptr, batch, rhs.ptr, out.ptr, ctx.n_threads),
                 "csr_batched_matvec");
  }
}

}  // namespace msx
