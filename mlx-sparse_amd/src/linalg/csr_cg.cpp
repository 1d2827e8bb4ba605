// csr_cg.cpp - C++ primitive layer of the conjugate gradient solvers.
#include "linalg/csr_cg.h"

#include <stdexcept>
#include <string>

#include "common/validate.h"

namespace msx {
namespace {

void require_float32(const ArrayView &a, const std::string &name) {
  // reference: src/linalg/common/common.h:413-418 (require_linalg_float32)
  if (a.dtype != DType::Float32)
    throw std::invalid_argument(name + " currently requires dtype float32.");
}

}  // namespace

msx_solver_result csr_cg(const ArrayView &data, const ArrayView &indices, const ArrayView &indptr,
                         const ArrayView &b, const ArrayView &x0, const ArrayView *inv_diag,
                         const ArrayView &x, int64_t n_rows, int64_t n_cols, float rtol,
                         float atol, int64_t maxiter, const msx_csr_plan *plan,
                         const ExecContext &ctx) {
  // reference: src/linalg/cg/cg.cpp:330-358
  const std::string op = inv_diag ? "csr_pcg_jacobi" : "csr_cg";
  if (n_rows <= 0 || n_cols <= 0 || n_rows != n_cols || n_rows >= 2147483647)
    throw std::invalid_argument(op + " requires a non-empty square matrix.");
  if (maxiter < 0) throw std::invalid_argument(op + " maxiter must be non-negative.");
  if (maxiter > 2147483647) throw std::invalid_argument(op + " maxiter must fit in int32.");
  require_rank(data, 1, (op + " data").c_str());
  require_rank(indices, 1, (op + " indices").c_str());
  require_rank(indptr, 1, (op + " indptr").c_str());
  require_rank(b, 1, (op + " b").c_str());
  require_rank(x0, 1, (op + " x0").c_str());
  require_float32(data, op + " data");
  require_float32(b, op + " b");
  require_float32(x0, op + " x0");
  require_same_index_dtype(indices, indptr, (op + " indices").c_str(), (op + " indptr").c_str());
  require_size(indptr, n_rows + 1, (op + " indptr").c_str());
  require_size(b, n_rows, (op + " b").c_str());
  require_size(x0, n_cols, (op + " x0").c_str());
  if (indices.size() != data.size())
    throw std::invalid_argument(op + " data and indices must have equal length.");
  if (inv_diag) {
    require_rank(*inv_diag, 1, "csr_pcg_jacobi inverse diagonal");
    require_float32(*inv_diag, "csr_pcg_jacobi inverse diagonal");
    require_size(*inv_diag, n_rows, "csr_pcg_jacobi inverse diagonal");
  }
  if (x.ndim != 1 || x.shape[0] != n_rows || x.dtype != DType::Float32)
    throw std::invalid_argument(op + " output buffer has the wrong shape or dtype.");
  require_same_device({&data, &indices, &indptr, &b, &x0, &x}, op.c_str());
  if (inv_diag) require_same_device({&data, inv_diag}, op.c_str());
  for (const ArrayView *a : {&data, &indices, &indptr, &b, &x0, &x})
    require_contiguous(*a, (op + " operand").c_str());
  if (inv_diag) require_contiguous(*inv_diag, (op + " operand").c_str());

  const msx_itype it = to_itype(indices.dtype);
  const auto *d = static_cast<const float *>(data.ptr);
  const auto *bb = static_cast<const float *>(b.ptr);
  const auto *xx0 = static_cast<const float *>(x0.ptr);
  auto *xx = static_cast<float *>(x.ptr);
  msx_solver_result res{};
  if (data.device >= 0) {
    if (inv_diag)
      check_status(msx_csr_pcg_jacobi(it, n_rows, data.size(), d, indices.ptr, indptr.ptr, bb, xx0,
                                      static_cast<const float *>(inv_diag->ptr), xx, rtol, atol,
                                      maxiter, plan, &res, ctx.stream),
                   op.c_str());
    else
      check_status(msx_csr_cg(it, n_rows, data.size(), d, indices.ptr, indptr.ptr, bb, xx0, xx,
                              rtol, atol, maxiter, plan, &res, ctx.stream),
                   op.c_str());
  } else {
    if (inv_diag)
      check_status(msx_csr_pcg_jacobi_cpu(it, n_rows, data.size(), d, indices.ptr, indptr.ptr, bb,
                                          xx0, static_cast<const float *>(inv_diag->ptr), xx, rtol,
                                          atol, maxiter, &res),
                   op.c_str());
    else
      check_status(msx_csr_cg_cpu(it, n_rows, data.size(), d, indices.ptr, indptr.ptr, bb, xx0, xx,
                                  rtol, atol, maxiter, &res),
                   op.c_str());
  }
  return res;
}

}  // namespace msx
