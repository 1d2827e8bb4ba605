// csr_adjoint.h - C++ primitives of the adjoint side: the CSR transpose, the
// transposed products A^T x / A^T X, and the value gradients of A x / A X.
#pragma once

#include "common/array_view.h"
#include "msx_sparse.h"

namespace msx {

// CSR of A^T into caller-allocated out_data (nnz), out_indices (nnz) and
// out_indptr (n_cols + 1).  Validates like the reference op (reference:
// src/sparse/csr_transpose/csr_transpose.cpp, csr_transpose), then runs
// msx_csr_transpose on ctx.stream or msx_csr_transpose_cpu on the host.
void csr_transpose(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                   const ArrayView &out_data, const ArrayView &out_indices,
                   const ArrayView &out_indptr, int64_t n_rows, int64_t n_cols,
                   const ExecContext &ctx);

// y = A^T x, x of length n_rows, y of length n_cols (reference:
// src/sparse/csr_matvec_transpose/csr_matvec_transpose.cpp,
// csr_matvec_transpose).
void csr_matvec_transpose(const ArrayView &data, const ArrayView &indices,
                          const ArrayView &indptr, const ArrayView &x, const ArrayView &out,
                          int64_t n_rows, int64_t n_cols, const ExecContext &ctx);

// Y = A^T X, X of shape (n_rows, k), Y of shape (n_cols, k) (reference:
// src/sparse/csr_matmul_transpose/csr_matmul_transpose.cpp,
// csr_matmul_transpose).
void csr_matmul_transpose(const ArrayView &data, const ArrayView &indices,
                          const ArrayView &indptr, const ArrayView &rhs, const ArrayView &out,
                          int64_t n_rows, int64_t n_cols, const ExecContext &ctx);

// out[p] = cot[row(p)] * x[col(p)] (reference:
// src/sparse/csr_matvec_data_vjp/csr_matvec_data_vjp.cpp, csr_matvec_data_vjp).
// plan: a GPU plan of the matrix (nullptr: none); a panel plan serves the
// gather of x from LDS.
void csr_matvec_data_vjp(const ArrayView &indices, const ArrayView &indptr, const ArrayView &x,
                         const ArrayView &cotangent, const ArrayView &out, int64_t n_rows,
                         int64_t n_cols, const ExecContext &ctx,
                         const msx_csr_plan *plan = nullptr);

// out[p] = sum_q cot[row(p), q] * X[col(p), q] (reference:
// src/sparse/csr_matmul_data_vjp/csr_matmul_data_vjp.cpp, csr_matmul_data_vjp).
void csr_matmul_data_vjp(const ArrayView &indices, const ArrayView &indptr, const ArrayView &rhs,
                         const ArrayView &cotangent, const ArrayView &out, int64_t n_rows,
                         int64_t n_cols, const ExecContext &ctx);

}  // namespace msx
