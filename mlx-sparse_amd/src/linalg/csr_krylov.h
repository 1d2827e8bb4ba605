// csr_krylov.h - C++ primitives of the BiCGSTAB and MINRES solvers.
#pragma once

#include "common/array_view.h"
#include "msx_sparse.h"

namespace msx {

enum class Krylov { BiCGSTAB, MINRES, GMRES };

// x (caller-allocated, n) from x0 for A x = b (MINRES: (A - shift I) x = b),
// A square float32 CSR (n x n).  Validates like the reference ops
// (reference: src/linalg/bicgstab/bicgstab.cpp:440-480 csr_bicgstab,
// src/linalg/minres/minres.cpp csr_minres, src/linalg/gmres/gmres.cpp:223-263
// csr_gmres), then runs the device solver on ctx.stream (with `plan`,
// nullable) or the host loop.  `restart`: GMRES's cycle length (> 0).
// `inv_diag` non-null: the Jacobi-preconditioned loop (reference:
// src/preconditioners/bicgstab/bicgstab.cpp:607-635 csr_bicgstab_jacobi,
// minres/minres.cpp:418-440 csr_minres_jacobi, gmres/gmres.cpp:750-790
// csr_gmres_jacobi).
msx_solver_result csr_krylov(Krylov kind, const ArrayView &data, const ArrayView &indices,
                             const ArrayView &indptr, const ArrayView &b, const ArrayView &x0,
                             const ArrayView &x, int64_t n_rows, int64_t n_cols, float rtol,
                             float atol, int64_t maxiter, float shift, const msx_csr_plan *plan,
                             const ExecContext &ctx, int64_t restart = 0,
                             const ArrayView *inv_diag = nullptr);

}  // namespace msx
