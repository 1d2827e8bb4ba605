// csr_matvec.h - C++ primitive: CSR sparse matrix x dense vector.
#pragma once

#include "common/array_view.h"
#include "msx_sparse.h"

namespace msx {

// y = A x for CSR buffers (data, indices, indptr) of shape (n_rows, n_cols).
// Validates like the reference op constructor (reference:
// src/sparse/csr_matvec/csr_matvec.cpp:326-356; texts from
// src/common/common.cpp:104-177), then runs on the arrays' device: a HIP
// device through msx_csr_spmv on ctx.stream (asynchronous), or the host
// through msx_csr_spmv_cpu.  `out` is a caller-allocated contiguous rank-1
// array of n_rows values of data's dtype on the same device.  `plan` (device
// path only, may be NULL) must come from this indptr.
void csr_matvec(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                const ArrayView &x, const ArrayView &out, int64_t n_rows, int64_t n_cols,
                const msx_csr_plan *plan, const ExecContext &ctx);

}  // namespace msx
