// csr_krylov.cpp - C++ primitive layer of the BiCGSTAB and MINRES solvers.
#include "linalg/csr_krylov.h"

#include <stdexcept>
#include <string>

#include "common/validate.h"

namespace msx {

msx_solver_result csr_krylov(Krylov kind, const ArrayView &data, const ArrayView &indices,
                             const ArrayView &indptr, const ArrayView &b, const ArrayView &x0,
                             const ArrayView &x, int64_t n_rows, int64_t n_cols, float rtol,
                             float atol, int64_t maxiter, float shift, const msx_csr_plan *plan,
                             const ExecContext &ctx, int64_t restart,
                             const ArrayView *inv_diag) {
  // reference: src/linalg/bicgstab/bicgstab.cpp:440-480 (require_* calls
  // of csr_bicgstab), src/linalg/minres/minres.cpp (csr_minres),
  // src/linalg/gmres/gmres.cpp:223-263 (csr_gmres)
  const std::string op = std::string(kind == Krylov::BiCGSTAB ? "csr_bicgstab"
                                     : kind == Krylov::MINRES ? "csr_minres"
                                                              : "csr_gmres") +
                         (inv_diag ? "_jacobi" : "");
  if (n_rows <= 0 || n_cols <= 0 || n_rows != n_cols || n_rows >= 2147483647)
    throw std::invalid_argument(op + " requires a non-empty square matrix.");
  if (kind == Krylov::GMRES && (restart <= 0 || maxiter < 0))
    throw std::invalid_argument(op + " requires restart > 0 and maxiter >= 0.");
  if (maxiter < 0) throw std::invalid_argument(op + " maxiter must be non-negative.");
  if (maxiter > 2147483647) throw std::invalid_argument(op + " maxiter must fit in int32.");
  require_rank(data, 1, (op + " data").c_str());
  require_rank(indices, 1, (op + " indices").c_str());
  require_rank(indptr, 1, (op + " indptr").c_str());
  require_rank(b, 1, (op + " b").c_str());
  require_rank(x0, 1, (op + " x0").c_str());
  for (const auto *a : {&data, &b, &x0})
    if (a->dtype != DType::Float32)
      throw std::invalid_argument(op + (a == &data ? " data" : a == &b ? " b" : " x0") +
                                  " currently requires dtype float32.");
  require_same_index_dtype(indices, indptr, (op + " indices").c_str(), (op + " indptr").c_str());
  require_size(indptr, n_rows + 1, (op + " indptr").c_str());
  require_size(b, n_rows, (op + " b").c_str());
  require_size(x0, n_cols, (op + " x0").c_str());
  if (indices.size() != data.size())
    throw std::invalid_argument(op + " data and indices must have equal length.");
  if (inv_diag) {
    // reference: src/preconditioners/bicgstab/bicgstab.cpp:615-617,
    // minres/minres.cpp:418-440, gmres/gmres.cpp:750-790
    require_rank(*inv_diag, 1, (op + " inv_diag").c_str());
    if (inv_diag->dtype != DType::Float32)
      throw std::invalid_argument(op + " inv_diag currently requires dtype float32.");
    require_size(*inv_diag, n_rows, (op + " inv_diag").c_str());
  }
  if (x.ndim != 1 || x.shape[0] != n_rows || x.dtype != DType::Float32)
    throw std::invalid_argument(op + " output buffer has the wrong shape or dtype.");
  require_same_device({&data, &indices, &indptr, &b, &x0, &x}, op.c_str());
  if (inv_diag) require_same_device({&data, inv_diag}, op.c_str());
  for (const ArrayView *a : {&data, &indices, &indptr, &b, &x0, &x})
    require_contiguous(*a, (op + " operand").c_str());
  if (inv_diag) require_contiguous(*inv_diag, (op + " operand").c_str());
  const auto *inv = inv_diag ? static_cast<const float *>(inv_diag->ptr) : nullptr;

  const msx_itype it = to_itype(indices.dtype);
  const auto *d = static_cast<const float *>(data.ptr);
  const auto *bb = static_cast<const float *>(b.ptr);
  const auto *xx0 = static_cast<const float *>(x0.ptr);
  auto *xx = static_cast<float *>(x.ptr);
  msx_solver_result res{};
  const int64_t nnz = data.size();
  if (kind == Krylov::BiCGSTAB && inv) {
    if (data.device >= 0)
      check_status(msx_csr_bicgstab_jacobi(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0,
                                           inv, xx, rtol, atol, maxiter, plan, &res, ctx.stream),
                   op.c_str());
    else
      check_status(msx_csr_bicgstab_jacobi_cpu(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb,
                                               xx0, inv, xx, rtol, atol, maxiter, &res),
                   op.c_str());
  } else if (kind == Krylov::BiCGSTAB) {
    if (data.device >= 0)
      check_status(msx_csr_bicgstab(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, xx, rtol,
                                    atol, maxiter, plan, &res, ctx.stream),
                   op.c_str());
    else
      check_status(msx_csr_bicgstab_cpu(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, xx,
                                        rtol, atol, maxiter, &res),
                   op.c_str());
  } else if (kind == Krylov::MINRES && inv) {
    if (data.device >= 0)
      check_status(msx_csr_minres_jacobi(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, inv,
                                         xx, rtol, atol, maxiter, shift, plan, &res, ctx.stream),
                   op.c_str());
    else
      check_status(msx_csr_minres_jacobi_cpu(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0,
                                             inv, xx, rtol, atol, maxiter, shift, &res),
                   op.c_str());
  } else if (kind == Krylov::GMRES && inv) {
    if (data.device >= 0)
      check_status(msx_csr_gmres_jacobi(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, inv,
                                        xx, rtol, atol, restart, maxiter, plan, &res, ctx.stream),
                   op.c_str());
    else
      check_status(msx_csr_gmres_jacobi_cpu(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0,
                                            inv, xx, rtol, atol, restart, maxiter, &res),
                   op.c_str());
  } else if (kind == Krylov::GMRES) {
    if (data.device >= 0)
      check_status(msx_csr_gmres(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, xx, rtol,
                                 atol, restart, maxiter, plan, &res, ctx.stream),
                   op.c_str());
    else
      check_status(msx_csr_gmres_cpu(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, xx,
                                     rtol, atol, restart, maxiter, &res),
                   op.c_str());
  } else {
    if (data.device >= 0)
      check_status(msx_csr_minres(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, xx, rtol,
                                  atol, maxiter, shift, plan, &res, ctx.stream),
                   op.c_str());
    else
      check_status(msx_csr_minres_cpu(it, n_rows, nnz, d, indices.ptr, indptr.ptr, bb, xx0, xx,
                                      rtol, atol, maxiter, shift, &res),
                   op.c_str());
  }
  return res;
}

}  // namespace msx
