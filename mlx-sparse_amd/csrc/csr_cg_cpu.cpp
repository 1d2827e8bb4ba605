// csr_cg_cpu.cpp - the `use_cpu()` conjugate gradient solvers: the
// reference's sequential loops, one thread, float32 values.
//
//   msx_csr_cg_cpu          csr_cg_cpu_impl (reference: src/linalg/cg/cg.cpp:75-246)
//   msx_csr_pcg_jacobi_cpu  csr_pcg_jacobi_cpu_impl (src/preconditioners/pcg/pcg.cpp:71-236)
//
// The solver SpMV sums each row from 0.0f in stored order (reference
// src/linalg/common/common.h:35-45); columns outside [0, n) add nothing.
#include <stdint.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <string>
#include <vector>

#include "msx_sparse.h"

namespace msx {
msx_status fail(msx_status code, const std::string &msg);
void clear_error();
}  // namespace msx

namespace {

template <class I>
void solver_spmv(int64_t n, const float *data, const I *indices, const I *indptr, const float *x,
                 float *out) {
  for (int64_t r = 0; r < n; ++r) {
    float acc = 0.0f;
    for (int64_t p = static_cast<int64_t>(indptr[r]); p < static_cast<int64_t>(indptr[r + 1]); ++p) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      if (c >= 0 && c < n) acc += data[p] * x[c];
    }
    out[r] = acc;
  }
}

bool fin(float v) { return std::isfinite(v); }

double dot(const std::vector<float> &a, const std::vector<float> &b) {
  double acc = 0.0;
  for (size_t i = 0; i < a.size(); ++i) acc += static_cast<double>(a[i]) * static_cast<double>(b[i]);
  return acc;
}

template <class I>
void cg(int64_t n, const float *data, const I *indices, const I *indptr, const float *b,
        const float *x0, float *x, float rtol, float atol, int64_t maxiter,
        msx_solver_result *res) {
  std::vector<float> r(n), p(n), ap(n);
  std::copy(x0, x0 + n, x);
  solver_spmv(n, data, indices, indptr, x, ap.data());
  double b_norm2 = 0.0, rr = 0.0;
  bool finite = true;
  for (int64_t i = 0; i < n; ++i) {
    r[i] = b[i] - ap[i];
    p[i] = r[i];
    b_norm2 += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    rr += static_cast<double>(r[i]) * static_cast<double>(r[i]);
    finite = finite && fin(r[i]) && fin(ap[i]) && fin(b[i]) && fin(x[i]);
  }
  const float residual_norm = static_cast<float>(std::sqrt(std::max(rr, 0.0)));
  const float b_norm = static_cast<float>(std::sqrt(std::max(b_norm2, 0.0)));
  const float tol = std::max(atol, rtol * b_norm);
  const double eps = FLT_EPSILON;
  res->reserved = 0;
  if (!finite || !std::isfinite(rr) || !fin(residual_norm) || !fin(b_norm)) {
    *res = {-3, 0, residual_norm, 0};
    return;
  }
  if (residual_norm <= tol) {
    *res = {0, 0, residual_norm, 0};
    return;
  }
  int32_t status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
  int32_t completed = 0;
  for (int64_t k = 1; k <= maxiter; ++k) {
    solver_spmv(n, data, indices, indptr, p.data(), ap.data());
    double denom = 0.0;
    finite = true;
    for (int64_t i = 0; i < n; ++i) {
      denom += static_cast<double>(p[i]) * static_cast<double>(ap[i]);
      finite = finite && fin(p[i]) && fin(ap[i]);
    }
    if (!finite || !std::isfinite(denom)) {
      status = -3;
      completed = static_cast<int32_t>(k - 1);
      break;
    }
    if (std::abs(denom) <= eps) {
      const double scale = std::sqrt(std::max(dot(p, p) * dot(ap, ap), 0.0));
      const double dtol = std::min(eps, eps * eps * std::max(1.0, scale));
      if (!std::isfinite(scale)) {
        status = -3;
        completed = static_cast<int32_t>(k - 1);
        break;
      }
      if (std::abs(denom) <= dtol) {
        status = -1;
        completed = static_cast<int32_t>(k - 1);
        break;
      }
    }
    const double alpha = rr / denom;
    if (!std::isfinite(alpha)) {
      status = -3;
      completed = static_cast<int32_t>(k - 1);
      break;
    }
    finite = true;
    double rr_new = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const double xc = static_cast<double>(x[i]) + alpha * static_cast<double>(p[i]);
      const double rc = static_cast<double>(r[i]) - alpha * static_cast<double>(ap[i]);
      const float xf = static_cast<float>(xc), rf = static_cast<float>(rc);
      if (!std::isfinite(xc) || !std::isfinite(rc) || !fin(xf) || !fin(rf)) {
        finite = false;
        continue;
      }
      x[i] = xf;
      r[i] = rf;
      rr_new += static_cast<double>(rf) * static_cast<double>(rf);
    }
    const float r_norm = static_cast<float>(std::sqrt(std::max(rr_new, 0.0)));
    completed = static_cast<int32_t>(k);
    if (!finite || !std::isfinite(rr_new) || !fin(r_norm)) {
      status = -3;
      break;
    }
    if (r_norm <= tol) {
      status = 0;
      rr = rr_new;
      break;
    }
    const double beta = rr_new / rr;
    if (!std::isfinite(beta)) {
      status = -3;
      break;
    }
    for (int64_t i = 0; i < n; ++i) {
      const double pc = static_cast<double>(r[i]) + beta * static_cast<double>(p[i]);
      const float pf = static_cast<float>(pc);
      if (!std::isfinite(pc) || !fin(pf)) {
        status = -3;
        break;
      }
      p[i] = pf;
    }
    if (status < 0) break;
    rr = rr_new;
  }
  *res = {status, completed, static_cast<float>(std::sqrt(std::max(rr, 0.0))), 0};
}

template <class I>
void pcg_jacobi(int64_t n, const float *data, const I *indices, const I *indptr, const float *b,
                const float *x0, const float *inv_diag, float *x, float rtol, float atol,
                int64_t maxiter, msx_solver_result *res) {
  std::vector<float> r(n), z(n), p(n), ap(n);
  std::copy(x0, x0 + n, x);
  solver_spmv(n, data, indices, indptr, x, ap.data());
  double b_norm2 = 0.0;
  bool finite = true;
  for (int64_t i = 0; i < n; ++i) {
    const float ri = b[i] - ap[i];
    const float zi = inv_diag[i] * ri;
    r[i] = ri;
    z[i] = zi;
    p[i] = zi;
    b_norm2 += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    finite = finite && fin(ri) && fin(zi) && fin(inv_diag[i]);
  }
  float true_rr = static_cast<float>(dot(r, r));
  float rho = static_cast<float>(dot(r, z));
  const float b_norm = static_cast<float>(std::sqrt(std::max(b_norm2, 0.0)));
  const float tol = std::max(atol, rtol * b_norm);
  const float true_residual = std::sqrt(std::max(true_rr, 0.0f));
  if (!finite || !fin(true_rr) || !fin(rho)) {
    *res = {-3, 0, true_residual, 0};
    return;
  }
  if (true_residual <= tol) {
    *res = {0, 0, true_residual, 0};
    return;
  }
  if (rho <= 0.0f) {
    *res = {-2, 0, true_residual, 0};
    return;
  }
  const float eps = FLT_EPSILON;
  int32_t status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
  int32_t completed = 0;
  for (int64_t k = 1; k <= maxiter; ++k) {
    solver_spmv(n, data, indices, indptr, p.data(), ap.data());
    const float denom = static_cast<float>(dot(p, ap));
    const float p2 = static_cast<float>(dot(p, p));
    const float ap2 = static_cast<float>(dot(ap, ap));
    const float scale = std::sqrt(std::max(p2 * ap2, 0.0f));
    const float dtol = eps * std::max(1.0f, scale);
    if (!fin(denom) || !fin(scale) || std::abs(denom) <= dtol) {
      status = -1;
      completed = static_cast<int32_t>(k - 1);
      break;
    }
    const float alpha = rho / denom;
    if (!fin(alpha)) {
      status = -3;
      completed = static_cast<int32_t>(k - 1);
      break;
    }
    double acc = 0.0;
    finite = true;
    for (int64_t i = 0; i < n; ++i) {
      x[i] += alpha * p[i];
      const float ri = r[i] - alpha * ap[i];
      const float zi = inv_diag[i] * ri;
      r[i] = ri;
      z[i] = zi;
      acc += static_cast<double>(ri) * static_cast<double>(ri);
      finite = finite && fin(x[i]) && fin(ri) && fin(zi);
    }
    true_rr = static_cast<float>(acc);
    const float r_norm = std::sqrt(std::max(true_rr, 0.0f));
    completed = static_cast<int32_t>(k);
    if (!finite || !fin(true_rr) || !fin(r_norm)) {
      status = -3;
      break;
    }
    if (r_norm <= tol) {
      status = 0;
      break;
    }
    const float rho_new = static_cast<float>(dot(r, z));
    if (!fin(rho_new) || rho_new <= 0.0f) {
      status = -2;
      break;
    }
    const float beta = rho_new / rho;
    if (!fin(beta)) {
      status = -3;
      break;
    }
    for (int64_t i = 0; i < n; ++i) p[i] = z[i] + beta * p[i];
    rho = rho_new;
  }
  *res = {status, completed, std::sqrt(std::max(true_rr, 0.0f)), 0};
}

msx_status check(const char *op, msx_itype it, int64_t n, int64_t nnz, const void *data,
                 const void *indices, const void *indptr, const void *b, const void *x0, void *x,
                 int64_t maxiter, msx_solver_result *result) {
  using msx::fail;
  if (it != MSX_I32 && it != MSX_I64)
    return fail(MSX_ETYPE, std::string(op) + " requires int32 or int64 indices.");
  if (n <= 0 || n >= 2147483647)
    return fail(MSX_EINVAL, std::string(op) + " requires a non-empty square matrix.");
  if (maxiter < 0) return fail(MSX_EINVAL, std::string(op) + " maxiter must be non-negative.");
  if (maxiter > 2147483647) return fail(MSX_EINVAL, std::string(op) + " maxiter must fit in int32.");
  if (nnz < 0) return fail(MSX_EINVAL, std::string(op) + " nnz must be non-negative.");
  if (indptr == nullptr || b == nullptr || x0 == nullptr || x == nullptr || result == nullptr ||
      (nnz > 0 && (data == nullptr || indices == nullptr)))
    return fail(MSX_EINVAL, std::string(op) + " buffers must be non-NULL.");
  return MSX_OK;
}

}  // namespace

extern "C" msx_status msx_csr_cg_cpu(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                     const void *indices, const void *indptr, const float *b,
                                     const float *x0, float *x, float rtol, float atol,
                                     int64_t maxiter, msx_solver_result *result) {
  msx::clear_error();
  const msx_status st = check("csr_cg", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  try {
    if (it == MSX_I32)
      cg(n, data, static_cast<const int32_t *>(indices), static_cast<const int32_t *>(indptr), b, x0,
         x, rtol, atol, maxiter, result);
    else
      cg(n, data, static_cast<const int64_t *>(indices), static_cast<const int64_t *>(indptr), b, x0,
         x, rtol, atol, maxiter, result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_cg: out of host memory.");
  }
  return MSX_OK;
}

extern "C" msx_status msx_csr_pcg_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                             const float *data, const void *indices,
                                             const void *indptr, const float *b, const float *x0,
                                             const float *inv_diag, float *x, float rtol,
                                             float atol, int64_t maxiter,
                                             msx_solver_result *result) {
  msx::clear_error();
  const msx_status st =
      check("csr_pcg_jacobi", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  if (inv_diag == nullptr) return msx::fail(MSX_EINVAL, "csr_pcg_jacobi inverse diagonal is NULL.");
  try {
    if (it == MSX_I32)
      pcg_jacobi(n, data, static_cast<const int32_t *>(indices),
                 static_cast<const int32_t *>(indptr), b, x0, inv_diag, x, rtol, atol, maxiter,
                 result);
    else
      pcg_jacobi(n, data, static_cast<const int64_t *>(indices),
                 static_cast<const int64_t *>(indptr), b, x0, inv_diag, x, rtol, atol, maxiter,
                 result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_pcg_jacobi: out of host memory.");
  }
  return MSX_OK;
}
