// csr_gmres_cpu.cpp - the `use_cpu()` restarted GMRES: the reference's
// sequential loop, one thread, float32 values.
//
//   msx_csr_gmres_cpu  csr_gmres_impl (reference:
//                      src/linalg/gmres/gmres.cpp:58-220) over the CPU
//                      Arnoldi factorisation (src/linalg/arnoldi/
//                      arnoldi.cpp:79-159, csr_arnoldi_cpu_impl)
//   msx_csr_gmres_jacobi_cpu  csr_gmres_jacobi_impl over
//                      csr_arnoldi_jacobi_cpu_impl (reference:
//                      src/preconditioners/gmres/gmres.cpp:342-748)
//
// Each cycle: the true residual r = b - A x and beta = ||r||; `steps`
// Arnoldi steps from r / beta, each one SpMV and two passes of modified
// Gram-Schmidt (each coefficient a double sum of float products, subtracted
// in float); the (used + 1) x used least-squares problem in double on the
// host (msx_hessenberg.h); x += V y with each row's update summed in double.
// The solver SpMV sums each row from 0.0f in stored order (reference
// src/linalg/common/common.h:35-45); columns outside [0, n) add nothing.
#include <stdint.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <limits>
#include <new>
#include <string>
#include <vector>

#include "msx_hessenberg.h"
#include "msx_sparse.h"

namespace msx {
msx_status fail(msx_status code, const std::string &msg);
void clear_error();
}  // namespace msx

namespace {

using Vec = std::vector<float>;

template <class I>
void spmv(int64_t n, const float *data, const I *indices, const I *indptr, const float *x,
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

// norm_float (common.h:56-73): float(sqrt(max(float(double sum), 0))).
float norm(const float *v, int64_t n) {
  double acc = 0.0;
  for (int64_t i = 0; i < n; ++i) acc += static_cast<double>(v[i]) * static_cast<double>(v[i]);
  const float f = static_cast<float>(acc);
  return std::sqrt(f < 0.0f ? 0.0f : f);
}

bool finite(float v) { return std::isfinite(v); }

// inv_diag non-null: GMRES with the Jacobi preconditioner M = diag(inv_diag)
// (reference src/preconditioners/gmres/gmres.cpp:342-748): each cycle starts
// from z0 = M r (beta = ||z0||, at most FLT_EPSILON: -1) over the Arnoldi
// basis of M A; ||r|| decides convergence; the least-squares solution is
// not tested on its own.
template <class I>
struct Gmres {
  int64_t n;
  const float *data;
  const I *indices;
  const I *indptr;
  const float *inv_diag;

  // b - A x into r; norm_float(r); `ok` = r and the norm finite.
  float residual(const float *b, const float *x, Vec &ax, Vec &r, bool &ok) const {
    spmv(n, data, indices, indptr, x, ax.data());
    ok = true;
    for (int64_t i = 0; i < n; ++i) {
      r[i] = b[i] - ax[i];
      ok = ok && finite(r[i]);
    }
    const float nr = norm(r.data(), n);
    ok = ok && finite(nr);
    return nr;
  }

  // k Arnoldi steps from v0 (arnoldi.cpp:99-158): basis vectors V[0..k]
  // (each n floats), h (k + 1) x k row-major; returns the steps taken.
  // Jacobi (gmres.cpp:342-447 there): w = M (A q); no step for a non-finite
  // v0 or inverse diagonal entry, none when a new norm is not finite.
  int64_t arnoldi(const Vec &v0, int64_t k, std::vector<Vec> &V, Vec &h, Vec &w) const {
    std::fill(h.begin(), h.begin() + (k + 1) * k, 0.0f);
    double vv = 0.0;
    bool inputs_ok = true;
    for (int64_t i = 0; i < n; ++i) {
      vv += static_cast<double>(v0[i]) * static_cast<double>(v0[i]);
      if (inv_diag) inputs_ok = inputs_ok && finite(v0[i]) && finite(inv_diag[i]);
    }
    const float v_norm = static_cast<float>(std::sqrt(vv < 0.0 ? 0.0 : vv));
    const float eps = FLT_EPSILON;
    if (inv_diag && (!inputs_ok || !finite(v_norm))) return 0;
    for (int64_t i = 0; i < n; ++i)
      V[0][i] = v_norm <= eps ? (i == 0 ? 1.0f : 0.0f) : v0[i] / v_norm;
    int64_t used = 0;
    for (int64_t j = 0; j < k; ++j) {
      spmv(n, data, indices, indptr, V[j].data(), w.data());
      if (inv_diag)
        for (int64_t i = 0; i < n; ++i) w[i] = w[i] * inv_diag[i];
      for (int pass = 0; pass < 2; ++pass)
        for (int64_t c = 0; c <= j; ++c) {
          const float *q = V[c].data();
          double coeff = 0.0;
          for (int64_t i = 0; i < n; ++i) {
            const float prod = q[i] * w[i];
            coeff += static_cast<double>(prod);
          }
          const float cf = static_cast<float>(coeff);
          h[c * k + j] += cf;
          for (int64_t i = 0; i < n; ++i) w[i] -= cf * q[i];
        }
      const float h_next = norm(w.data(), n);
      h[(j + 1) * k + j] = h_next;
      used = j + 1;
      if (inv_diag && !finite(h_next)) return 0;
      if (h_next <= eps) break;
      float *next = V[j + 1].data();
      for (int64_t i = 0; i < n; ++i) next[i] = w[i] / h_next;
    }
    return used;
  }

  void solve(const float *b, const float *x0, float *x, float rtol, float atol, int64_t restart,
             int64_t maxiter, msx_solver_result *res) const {
    std::copy(x0, x0 + n, x);
    const float b_norm = norm(b, n);
    const float scaled = rtol * b_norm;
    const float tol = atol > scaled ? atol : scaled;
    int64_t iters = 0;
    int32_t status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
    float residual_norm = std::numeric_limits<float>::infinity();
    bool inputs_ok = finite(b_norm) && finite(tol);
    for (int64_t i = 0; i < n; ++i)
      inputs_ok = inputs_ok && finite(x[i]) && finite(b[i]) && (!inv_diag || finite(inv_diag[i]));
    if (!inputs_ok) {
      *res = {-3, 0, residual_norm, 0};
      return;
    }
    const int64_t kcap = std::max<int64_t>(1, std::min({restart, maxiter, n}));
    Vec r(n), ax(n), v0(n), w(n), h((kcap + 1) * kcap), z0(inv_diag ? n : 0);
    std::vector<Vec> V(static_cast<size_t>(kcap + 1), Vec(n, 0.0f));
    std::vector<double> y;
    while (iters < maxiter) {
      bool ok = true;
      float beta = residual(b, x, ax, r, ok);
      residual_norm = beta;
      if (inv_diag) {
        for (int64_t i = 0; i < n; ++i) {
          z0[i] = inv_diag[i] * r[i];
          ok = ok && finite(z0[i]);
        }
      }
      if (!ok) {
        status = -3;
        break;
      }
      if (residual_norm <= tol) {
        status = 0;
        break;
      }
      if (inv_diag) {
        beta = norm(z0.data(), n);
        if (!finite(beta) || beta <= FLT_EPSILON) {
          status = -1;
          break;
        }
      }
      const int64_t steps = std::min({restart, maxiter - iters, n});
      const Vec &start = inv_diag ? z0 : r;
      for (int64_t i = 0; i < n; ++i) v0[i] = start[i] / beta;
      for (int64_t c = 1; c <= steps; ++c) std::fill(V[c].begin(), V[c].end(), 0.0f);
      const int64_t used = arnoldi(v0, steps, V, h, w);
      if (used == 0) {
        status = -1;
        break;
      }
      std::vector<double> hu(static_cast<size_t>((used + 1) * used));
      bool bad = false;
      for (int64_t row = 0; row <= used; ++row)
        for (int64_t col = 0; col < used; ++col) {
          hu[row * used + col] = static_cast<double>(h[row * steps + col]);
          bad = bad || !std::isfinite(hu[row * used + col]);
        }
      if (bad) {
        status = -3;
        break;
      }
      std::vector<double> e1(static_cast<size_t>(used + 1), 0.0);
      e1[0] = static_cast<double>(beta);
      if (!msx::hessenberg_least_squares(std::move(hu), std::move(e1), used, y)) {
        status = -1;
        break;
      }
      if (!inv_diag)
        for (double v : y) bad = bad || !std::isfinite(v);
      if (bad) {
        status = -3;
        break;
      }
      for (int64_t i = 0; i < n && !bad; ++i) {
        double update = 0.0;
        for (int64_t c = 0; c < used; ++c) update += static_cast<double>(V[c][i]) * y[c];
        if (!std::isfinite(update)) {
          bad = true;
          break;
        }
        x[i] += static_cast<float>(update);
        bad = !finite(x[i]);
      }
      if (bad) {
        status = -3;
        break;
      }
      iters += used;
      if (iters >= maxiter) {
        residual_norm = residual(b, x, ax, r, ok);
        if (!ok) status = -3;
        else if (residual_norm <= tol) status = 0;
        break;
      }
    }
    if (maxiter == 0 && status > 0) {
      bool ok = true;
      residual_norm = residual(b, x, ax, r, ok);
      if (!ok) status = -3;
      else if (residual_norm <= tol) status = 0;
    }
    *res = {status, static_cast<int32_t>(iters), residual_norm, 0};
  }
};

}  // namespace

extern "C" msx_status msx_csr_gmres_cpu(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                        const void *indices, const void *indptr, const float *b,
                                        const float *x0, float *x, float rtol, float atol,
                                        int64_t restart, int64_t maxiter,
                                        msx_solver_result *result) {
  msx::clear_error();
  if (it != MSX_I32 && it != MSX_I64)
    return msx::fail(MSX_ETYPE, "csr_gmres requires int32 or int64 indices.");
  if (n <= 0 || n >= 2147483647) return msx::fail(MSX_EINVAL, "csr_gmres requires a non-empty square matrix.");
  if (restart <= 0 || maxiter < 0)
    return msx::fail(MSX_EINVAL, "csr_gmres requires restart > 0 and maxiter >= 0.");
  if (maxiter > 2147483647) return msx::fail(MSX_EINVAL, "csr_gmres maxiter must fit in int32.");
  if (nnz < 0) return msx::fail(MSX_EINVAL, "csr_gmres nnz must be non-negative.");
  if (indptr == nullptr || b == nullptr || x0 == nullptr || x == nullptr || result == nullptr ||
      (nnz > 0 && (data == nullptr || indices == nullptr)))
    return msx::fail(MSX_EINVAL, "csr_gmres buffers must be non-NULL.");
  try {
    if (it == MSX_I32)
      Gmres<int32_t>{n, data, static_cast<const int32_t *>(indices),
                     static_cast<const int32_t *>(indptr), nullptr}
          .solve(b, x0, x, rtol, atol, restart, maxiter, result);
    else
      Gmres<int64_t>{n, data, static_cast<const int64_t *>(indices),
                     static_cast<const int64_t *>(indptr), nullptr}
          .solve(b, x0, x, rtol, atol, restart, maxiter, result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_gmres could not allocate its workspace.");
  }
  return MSX_OK;
}

extern "C" msx_status msx_csr_gmres_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                               const float *data, const void *indices,
                                               const void *indptr, const float *b,
                                               const float *x0, const float *inv_diag, float *x,
                                               float rtol, float atol, int64_t restart,
                                               int64_t maxiter, msx_solver_result *result) {
  msx::clear_error();
  if (it != MSX_I32 && it != MSX_I64)
    return msx::fail(MSX_ETYPE, "csr_gmres_jacobi requires int32 or int64 indices.");
  if (n <= 0 || n >= 2147483647)
    return msx::fail(MSX_EINVAL, "csr_gmres_jacobi requires a non-empty square matrix.");
  if (restart <= 0 || maxiter < 0)
    return msx::fail(MSX_EINVAL, "csr_gmres_jacobi requires restart > 0 and maxiter >= 0.");
  if (maxiter > 2147483647)
    return msx::fail(MSX_EINVAL, "csr_gmres_jacobi maxiter must fit in int32.");
  if (nnz < 0) return msx::fail(MSX_EINVAL, "csr_gmres_jacobi nnz must be non-negative.");
  if (indptr == nullptr || b == nullptr || x0 == nullptr || x == nullptr || result == nullptr ||
      inv_diag == nullptr || (nnz > 0 && (data == nullptr || indices == nullptr)))
    return msx::fail(MSX_EINVAL, "csr_gmres_jacobi buffers must be non-NULL.");
  try {
    if (it == MSX_I32)
      Gmres<int32_t>{n, data, static_cast<const int32_t *>(indices),
                     static_cast<const int32_t *>(indptr), inv_diag}
          .solve(b, x0, x, rtol, atol, restart, maxiter, result);
    else
      Gmres<int64_t>{n, data, static_cast<const int64_t *>(indices),
                     static_cast<const int64_t *>(indptr), inv_diag}
          .solve(b, x0, x, rtol, atol, restart, maxiter, result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_gmres_jacobi could not allocate its workspace.");
  }
  return MSX_OK;
}
