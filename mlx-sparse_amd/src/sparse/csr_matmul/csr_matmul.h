// csr_matmul.h - C++ primitive: CSR sparse matrix x dense row-major matrix.
#pragma once

#include "common/array_view.h"
#include "msx_sparse.h"

namespace msx {

// Y = A X for CSR buffers of shape (n_rows, n_cols) and a rank-2 X of shape
// (n_cols, k).  Validates like the reference op constructor (reference:
// src/sparse/csr_matmul/csr_matmul.cpp:383-418), then runs msx_csr_spmm on
// ctx.stream or msx_csr_spmm_cpu on the host.  All operands contiguous (the
// binding copies non-contiguous inputs, as mx::contiguous does in the
// reference); `out` is a caller-allocated contiguous (n_rows, k) array.
void csr_matmul(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                const ArrayView &rhs, const ArrayView &out, int64_t n_rows, int64_t n_cols,
                const msx_csr_plan *plan, const ExecContext &ctx);

}  // namespace msx
