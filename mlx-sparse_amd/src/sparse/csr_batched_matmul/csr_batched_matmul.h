// csr_batched_matmul.h - C++ primitive: CSR matrix times a batch of dense matrices.
#pragma once

#include "common/array_view.h"
#include "msx_sparse.h"

namespace msx {

// Y[b] = A X[b] for CSR buffers of shape (n_rows, n_cols), X of shape
// (batch, n_cols, k) and Y of shape (batch, n_rows, k).  Validates like the
// reference op constructor (reference:
// src/sparse/csr_batched_matmul/csr_batched_matmul.cpp:438-475), then runs
// msx_csr_batched_spmm on ctx.stream or msx_csr_batched_spmm_cpu on the
// host.  All operands contiguous; `out` is caller-allocated.
void csr_batched_matmul(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                        const ArrayView &rhs, const ArrayView &out, int64_t n_rows, int64_t n_cols,
                        const ExecContext &ctx);

}  // namespace msx
