// csr_cg.h - C++ primitives of the conjugate gradient solvers.
#pragma once

#include "common/array_view.h"
#include "msx_sparse.h"

namespace msx {

// x (caller-allocated, n) from x0 for A x = b, A square float32 CSR (n x n).
// Validates like the reference op (reference: src/linalg/cg/cg.cpp:330-372,
// csr_cg; src/preconditioners/pcg/pcg.cpp, csr_pcg_jacobi), then runs the
// device solver on ctx.stream (with `plan`, nullable) or the host loop.
// `inv_diag` null: plain CG; else Jacobi-preconditioned CG.
msx_solver_result csr_cg(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                         const ArrayView &b, const ArrayView &x0, const ArrayView *inv_diag,
                         const ArrayView &x, int64_t n_rows, int64_t n_cols, float rtol,
                         float atol, int64_t maxiter, const msx_csr_plan *plan,
                         const ExecContext &ctx);

}  // namespace msx
