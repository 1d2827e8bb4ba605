// csr_krylov_cpu.cpp - the `use_cpu()` BiCGSTAB and MINRES solvers: the
// reference's sequential loops, one thread, float32 values.
//
//   msx_csr_bicgstab_cpu  csr_bicgstab_cpu_impl (reference:
//                         src/linalg/bicgstab/bicgstab.cpp:80-362)
//   msx_csr_bicgstab_jacobi_cpu  left_preconditioned_bicgstab_host with the
//                         Jacobi apply (reference:
//                         src/preconditioners/bicgstab/bicgstab.cpp:140-521)
//   msx_csr_minres_jacobi_cpu  csr_minres_jacobi_cpu_impl (reference:
//                         src/preconditioners/minres/minres.cpp:93-330)
//   msx_csr_minres_cpu    csr_minres_cpu_impl (reference:
//                         src/linalg/minres/minres.cpp:68-312)
//
// Vectors are float; dot products are sequential double sums; scalars are
// double; each vector update is formed in double and rounded once, except
// MINRES's float updates of A v, which the reference writes in float.  The
// solver SpMV sums each row from 0.0f in stored order (reference
// src/linalg/common/common.h:35-45); columns outside [0, n) add nothing.
#include <stdint.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <string>
#include <utility>
#include <vector>

#include "msx_sparse.h"

namespace msx {
msx_status fail(msx_status code, const std::string &msg);
void clear_error();
}  // namespace msx

namespace {

using Vec = std::vector<float>;

template <class I>
struct Csr {
  int64_t n;
  const float *data;
  const I *indices;
  const I *indptr;
  void apply(const float *x, float *out) const {
    for (int64_t r = 0; r < n; ++r) {
      float acc = 0.0f;
      for (int64_t p = static_cast<int64_t>(indptr[r]); p < static_cast<int64_t>(indptr[r + 1]);
           ++p) {
        const int64_t c = static_cast<int64_t>(indices[p]);
        if (c >= 0 && c < n) acc += data[p] * x[c];
      }
      out[r] = acc;
    }
  }
};

bool fin(float v) { return std::isfinite(v); }
bool fin(double v) { return std::isfinite(v); }

double dot(const Vec &a, const Vec &b) {
  double acc = 0.0;
  for (size_t i = 0; i < a.size(); ++i) acc += static_cast<double>(a[i]) * static_cast<double>(b[i]);
  return acc;
}

// The reference's breakdown test for a dot product (bicgstab.cpp:43-49):
// |value| <= FLT_EPSILON * max(1, sqrt(lhs_norm2 * rhs_norm2)).
bool near_zero(double value, double lhs_norm2, double rhs_norm2) {
  const double scale = std::sqrt(std::max(lhs_norm2 * rhs_norm2, 0.0));
  return !fin(scale) || std::fabs(value) <= static_cast<double>(FLT_EPSILON) * std::max(1.0, scale);
}

template <class I>
void bicgstab(const Csr<I> &A, const float *b, const float *x0, float *x, float rtol, float atol,
              int64_t maxiter, msx_solver_result *res) {
  const int64_t n = A.n;
  Vec r(n), r_hat(n), p(n, 0.0f), v(n, 0.0f), s(n), t(n), ax(n);
  std::copy(x0, x0 + n, x);
  double bb = 0.0;
  bool inputs_finite = true;
  for (int64_t i = 0; i < n; ++i) {
    bb += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    inputs_finite = inputs_finite && fin(b[i]) && fin(x[i]);
  }
  const float b_norm = static_cast<float>(std::sqrt(std::max(bb, 0.0)));
  const float tol = std::max(atol, rtol * b_norm);
  // dst = b - A x; the norm as float and whether everything stayed finite
  auto residual_into = [&](Vec &dst, bool &ok) {
    A.apply(x, ax.data());
    double rr = 0.0;
    ok = true;
    for (int64_t i = 0; i < n; ++i) {
      const float ri = b[i] - ax[i];
      ok = ok && fin(ri) && fin(ax[i]) && fin(x[i]);
      dst[i] = ri;
      rr += static_cast<double>(ri) * static_cast<double>(ri);
    }
    const float norm = static_cast<float>(std::sqrt(std::max(rr, 0.0)));
    ok = ok && fin(rr) && fin(norm);
    return norm;
  };
  bool ok = true;
  float residual = residual_into(r, ok);
  r_hat = r;
  res->reserved = 0;
  if (!inputs_finite || !fin(b_norm) || !fin(tol) || !ok) {
    *res = {-3, 0, residual, 0};
    return;
  }
  if (residual <= tol) {
    *res = {0, 0, residual, 0};
    return;
  }
  int32_t status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
  int32_t done = 0;
  double rho_prev = 1.0, alpha = 1.0, omega = 1.0;
  const double eps = FLT_EPSILON;
  for (int64_t k = 1; k <= maxiter; ++k) {
    const int32_t before = static_cast<int32_t>(k - 1);
    const double rho = dot(r_hat, r), hh = dot(r_hat, r_hat), rr = dot(r, r);
    if (!fin(rho) || !fin(hh) || !fin(rr)) {
      status = -3, done = before;
      break;
    }
    if (near_zero(rho, hh, rr)) {
      status = -1, done = before;
      break;
    }
    if (k == 1) {
      p = r;
    } else {
      if (std::fabs(omega) <= eps) {
        status = -1, done = before;
        break;
      }
      const double beta = (rho / rho_prev) * (alpha / omega);
      if (!fin(beta)) {
        status = -3, done = before;
        break;
      }
      bool pf = true;
      for (int64_t i = 0; i < n; ++i) {
        const double pi = static_cast<double>(r[i]) +
                          beta * (static_cast<double>(p[i]) - omega * static_cast<double>(v[i]));
        p[i] = static_cast<float>(pi);
        pf = pf && fin(pi) && fin(p[i]);
      }
      if (!pf) {
        status = -3, done = before;
        break;
      }
    }
    A.apply(p.data(), v.data());
    const double hv = dot(r_hat, v), vv = dot(v, v);
    if (!fin(hv) || !fin(vv)) {
      status = -3, done = before;
      break;
    }
    if (near_zero(hv, hh, vv)) {
      status = -1, done = before;
      break;
    }
    alpha = rho / hv;
    if (!fin(alpha)) {
      status = -3, done = before;
      break;
    }
    double ss = 0.0;
    bool sf = true;
    for (int64_t i = 0; i < n; ++i) {
      const double si = static_cast<double>(r[i]) - alpha * static_cast<double>(v[i]);
      const double xi = static_cast<double>(x[i]) + alpha * static_cast<double>(p[i]);
      s[i] = static_cast<float>(si);
      x[i] = static_cast<float>(xi);
      ss += si * si;
      sf = sf && fin(si) && fin(xi) && fin(s[i]) && fin(x[i]);
    }
    done = static_cast<int32_t>(k);
    const float s_norm = static_cast<float>(std::sqrt(std::max(ss, 0.0)));
    if (!sf || !fin(ss) || !fin(s_norm)) {
      status = -3;
      break;
    }
    if (s_norm <= tol) {  // confirm on the true residual (written to ax)
      bool tf = true;
      const float true_norm = residual_into(ax, tf);
      if (!tf || true_norm <= tol) {
        status = tf ? 0 : -3;
        residual = true_norm;
        break;
      }
    }
    A.apply(s.data(), t.data());
    const double ts = dot(t, s), tt = dot(t, t);
    if (!fin(ts) || !fin(tt)) {
      status = -3;
      break;
    }
    if (near_zero(tt, tt, 1.0)) {
      status = -1;
      break;
    }
    omega = ts / tt;
    if (!fin(omega)) {
      status = -3;
      break;
    }
    double rn = 0.0;
    bool rf = true;
    for (int64_t i = 0; i < n; ++i) {
      const double xi = static_cast<double>(x[i]) + omega * static_cast<double>(s[i]);
      const double ri = static_cast<double>(s[i]) - omega * static_cast<double>(t[i]);
      x[i] = static_cast<float>(xi);
      r[i] = static_cast<float>(ri);
      rn += ri * ri;
      rf = rf && fin(xi) && fin(ri) && fin(x[i]) && fin(r[i]);
    }
    residual = static_cast<float>(std::sqrt(std::max(rn, 0.0)));
    if (!rf || !fin(rn) || !fin(residual)) {
      status = -3;
      break;
    }
    if (residual <= tol) {  // the true residual replaces r
      bool tf = true;
      residual = residual_into(r, tf);
      if (!tf || residual <= tol) {
        status = tf ? 0 : -3;
        break;
      }
    }
    if (std::fabs(omega) <= eps) {
      status = -1;
      break;
    }
    rho_prev = rho;
  }
  if (status > 0 || status == -1) {
    bool tf = true;
    residual = residual_into(r, tf);
    if (!tf) status = -3;
    else if (residual <= tol) status = 0;
  }
  *res = {status, done, residual, 0};
}

template <class I>
void minres(const Csr<I> &A, const float *b, const float *x0, const float *inv_diag, float *x,
            float rtol, float atol, int64_t maxiter, float shift, msx_solver_result *res) {
  const int64_t n = A.n;
  Vec r1(n, 0.0f), r2(n, 0.0f), v(n, 0.0f), w(n, 0.0f), w2(n, 0.0f), av(n, 0.0f);
  // Jacobi (inv_diag non-null, src/preconditioners/minres/minres.cpp:93-330):
  // y = M r2 in float, a non-positive inverse diagonal entry or preconditioned
  // product gives -2
  Vec y(inv_diag ? n : 0, 0.0f);
  const int32_t beta_fail = inv_diag ? -2 : -1;
  auto precondition = [&]() -> const Vec & {
    if (!inv_diag) return r2;
    for (int64_t i = 0; i < n; ++i) y[i] = inv_diag[i] * r2[i];
    return y;
  };
  std::copy(x0, x0 + n, x);
  double bb = 0.0;
  for (int64_t i = 0; i < n; ++i) bb += static_cast<double>(b[i]) * static_cast<double>(b[i]);
  const float b_norm = static_cast<float>(std::sqrt(std::max(bb, 0.0)));
  const float tol = std::max(atol, rtol * b_norm);
  // ||b - (A - shift I) x||, A x left in `work` (minres.cpp:68-91)
  auto true_residual = [&](Vec &work, bool &ok) {
    A.apply(x, work.data());
    double rr = 0.0;
    ok = true;
    for (int64_t i = 0; i < n; ++i) {
      const float ai = work[i] - shift * x[i];
      const float ri = b[i] - ai;
      rr += static_cast<double>(ri) * static_cast<double>(ri);
      ok = ok && fin(ai) && fin(ri);
    }
    const float norm = static_cast<float>(std::sqrt(std::max(rr, 0.0)));
    ok = ok && fin(norm);
    return norm;
  };
  res->reserved = 0;
  int32_t status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
  int32_t done = 0;
  bool ok = true;
  float residual = true_residual(av, ok);
  if (!ok) {
    *res = {-3, 0, residual, 0};
    return;
  }
  if (inv_diag) {
    for (int64_t i = 0; i < n; ++i) {
      if (!(inv_diag[i] > 0.0f)) {
        *res = {-2, 0, residual, 0};
        return;
      }
    }
  }
  if (residual <= tol || maxiter == 0) {
    *res = {residual <= tol ? 0 : status, 0, residual, 0};
    return;
  }
  // r2 = b - (A - shift I) x, y = M r2 (plain: y is r2 throughout)
  for (int64_t i = 0; i < n; ++i) r2[i] = b[i] - (av[i] - shift * x[i]);
  const Vec *yv = &precondition();
  double beta_sq = static_cast<double>(static_cast<float>(dot(r2, *yv)));
  if (!fin(beta_sq) || beta_sq <= 0.0) {
    *res = {beta_fail, 0, residual, 0};
    return;
  }
  const double eps = FLT_EPSILON;
  double beta = std::sqrt(beta_sq), oldb = 0.0, dbar = 0.0, epsln = 0.0, phibar = beta;
  double cs = -1.0, sn = 0.0;
  for (int64_t k = 1; k <= maxiter; ++k) {
    if (!fin(beta) || beta <= eps) {
      status = beta_fail;
      break;
    }
    const double inv_beta = 1.0 / beta;
    const Vec &yy = inv_diag ? y : r2;
    for (int64_t i = 0; i < n; ++i) v[i] = static_cast<float>(inv_beta * static_cast<double>(yy[i]));
    A.apply(v.data(), av.data());
    for (int64_t i = 0; i < n; ++i) av[i] -= shift * v[i];
    if (k >= 2) {
      if (!fin(oldb) || std::fabs(oldb) <= eps) {
        status = -1;
        break;
      }
      const float prev_scale = static_cast<float>(beta / oldb);
      for (int64_t i = 0; i < n; ++i) av[i] -= prev_scale * r1[i];
    }
    const double alfa = static_cast<double>(static_cast<float>(dot(v, av)));
    if (!fin(alfa)) {
      status = -3;
      break;
    }
    const float diag_scale = static_cast<float>(alfa / beta);
    for (int64_t i = 0; i < n; ++i) av[i] -= diag_scale * r2[i];
    // the Lanczos vectors move on: r1 <- r2 <- A v (the old r1 is scratch)
    std::swap(r1, r2);
    std::swap(r2, av);
    yv = &precondition();
    oldb = beta;
    beta_sq = static_cast<double>(static_cast<float>(dot(r2, *yv)));
    if (!fin(beta_sq) || beta_sq < 0.0) {
      status = beta_fail;
      break;
    }
    beta = std::sqrt(std::max(beta_sq, 0.0));
    // the next Givens rotation of the Lanczos tridiagonal
    const double oldeps = epsln;
    const double delta = cs * dbar + sn * alfa;
    const double gbar = sn * dbar - cs * alfa;
    epsln = sn * beta;
    dbar = -cs * beta;
    double gamma = std::hypot(gbar, beta);
    if (!fin(gamma)) {
      status = -3;
      break;
    }
    gamma = std::max(gamma, eps);
    cs = gbar / gamma;
    sn = beta / gamma;
    const double phi = cs * phibar;
    phibar = sn * phibar;
    if (!fin(phi) || !fin(phibar)) {
      status = -3;
      break;
    }
    bool wf = true;
    for (int64_t i = 0; i < n; ++i) {
      const double older = w2[i], old = w[i];
      w2[i] = w[i];
      w[i] = static_cast<float>((static_cast<double>(v[i]) - oldeps * older - delta * old) / gamma);
      x[i] += static_cast<float>(phi * static_cast<double>(w[i]));
      wf = wf && fin(w[i]) && fin(x[i]);
    }
    done = static_cast<int32_t>(k);
    if (!wf) {
      status = -3;
      break;
    }
    residual = true_residual(av, ok);
    if (!ok) {
      status = -3;
      break;
    }
    if (residual <= tol) {
      status = 0;
      break;
    }
    if (beta <= eps) {
      status = -1;
      break;
    }
  }
  *res = {status, done, residual, 0};
}

// BiCGSTAB with the Jacobi preconditioner M = diag(inv_diag): the
// reference's left_preconditioned_bicgstab_host with the Jacobi apply
// (src/preconditioners/bicgstab/bicgstab.cpp:140-521).  Against bicgstab
// above: ||b|| rounded to float before its square root (norm_float,
// src/linalg/common/common.h:56-73); x advances along p_hat = M p and
// s_hat = M s, which the SpMVs take; a failed true-residual evaluation ends
// the solve with -3 and leaves the reported residual as it was (+inf before
// the first iteration); the reported residual follows ||s|| after the s
// update.
template <class I>
struct JacobiBicgstab {
  const Csr<I> &A;
  const float *b;
  const float *inv_diag;
  float *x;
  int64_t n;
  Vec ax;

  // true_residual_into (bicgstab.cpp:166-192); false where the reference throws
  bool true_residual(float *dst, float *norm) {
    A.apply(x, ax.data());
    for (int64_t i = 0; i < n; ++i)
      if (!fin(ax[i])) return false;
    double rr = 0.0;
    bool ok = true;
    for (int64_t i = 0; i < n; ++i) {
      const float ri = b[i] - ax[i];
      dst[i] = ri;
      rr += static_cast<double>(ri) * static_cast<double>(ri);
      ok = ok && fin(ri);
    }
    const float nv = static_cast<float>(std::sqrt(std::max(rr, 0.0)));
    if (!ok || !fin(rr) || !fin(nv)) return false;
    *norm = nv;
    return true;
  }
  bool apply(const Vec &src, Vec &out) const {
    bool ok = true;
    for (int64_t i = 0; i < n; ++i) {
      out[i] = inv_diag[i] * src[i];
      ok = ok && fin(out[i]);
    }
    return ok;
  }
};

template <class I>
void bicgstab_jacobi(const Csr<I> &A, const float *b, const float *x0, const float *inv_diag,
                     float *x, float rtol, float atol, int64_t maxiter, msx_solver_result *res) {
  const int64_t n = A.n;
  Vec r(n, 0.0f), r_hat(n, 0.0f), p(n, 0.0f), p_hat(n, 0.0f), v(n, 0.0f), s(n, 0.0f),
      s_hat(n, 0.0f), t(n, 0.0f);
  JacobiBicgstab<I> J{A, b, inv_diag, x, n, Vec(n, 0.0f)};
  std::copy(x0, x0 + n, x);
  int32_t status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1, done = 0;
  float residual = INFINITY;
  double bb = 0.0;
  bool inputs_finite = true;
  for (int64_t i = 0; i < n; ++i) {
    bb += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    inputs_finite = inputs_finite && fin(b[i]) && fin(x[i]);
  }
  const float bbf = static_cast<float>(bb);
  const float b_norm = std::sqrt(bbf < 0.0f ? 0.0f : bbf);
  const float tol = std::max(atol, rtol * b_norm);
  auto all_finite = [n](const Vec &a) {
    for (int64_t i = 0; i < n; ++i)
      if (!fin(a[i])) return false;
    return true;
  };
  if (!inputs_finite || !fin(b_norm) || !fin(tol) || !J.true_residual(r.data(), &residual)) {
    *res = {-3, 0, residual, 0};
    return;
  }
  r_hat = r;
  if (residual <= tol) {
    *res = {0, 0, residual, 0};
    return;
  }
  double rho_prev = 1.0, alpha = 1.0, omega = 1.0;
  const double eps = static_cast<double>(FLT_EPSILON);
  for (int64_t k = 1; k <= maxiter; ++k) {
    const auto prev = static_cast<int32_t>(k - 1);
    const double rho = dot(r_hat, r), hh = dot(r_hat, r_hat), rr = dot(r, r);
    if (!fin(rho) || !fin(hh) || !fin(rr)) {
      status = -3, done = prev;
      break;
    }
    if (near_zero(rho, hh, rr)) {
      status = -1, done = prev;
      break;
    }
    if (k == 1) {
      p = r;
    } else {
      if (std::fabs(omega) <= eps) {
        status = -1, done = prev;
        break;
      }
      const double beta = (rho / rho_prev) * (alpha / omega);
      if (!fin(beta)) {
        status = -3, done = prev;
        break;
      }
      bool ok = true;
      for (int64_t i = 0; i < n; ++i) {
        const double pi = static_cast<double>(r[i]) +
                          beta * (static_cast<double>(p[i]) - omega * static_cast<double>(v[i]));
        p[i] = static_cast<float>(pi);
        ok = ok && fin(pi) && fin(p[i]);
      }
      if (!ok) {
        status = -3, done = prev;
        break;
      }
    }
    if (!J.apply(p, p_hat)) {
      status = -3, done = prev;
      break;
    }
    A.apply(p_hat.data(), v.data());
    if (!all_finite(v)) {
      status = -3, done = prev;
      break;
    }
    const double hv = dot(r_hat, v), vv = dot(v, v);
    if (!fin(hv) || !fin(vv)) {
      status = -3, done = prev;
      break;
    }
    if (near_zero(hv, hh, vv)) {
      status = -1, done = prev;
      break;
    }
    alpha = rho / hv;
    if (!fin(alpha)) {
      status = -3, done = prev;
      break;
    }
    double ss = 0.0;
    bool ok = true;
    for (int64_t i = 0; i < n; ++i) {
      const double si = static_cast<double>(r[i]) - alpha * static_cast<double>(v[i]);
      const double xi = static_cast<double>(x[i]) + alpha * static_cast<double>(p_hat[i]);
      s[i] = static_cast<float>(si);
      x[i] = static_cast<float>(xi);
      ss += si * si;
      ok = ok && fin(si) && fin(xi) && fin(s[i]) && fin(x[i]);
    }
    done = static_cast<int32_t>(k);
    residual = static_cast<float>(std::sqrt(std::max(ss, 0.0)));
    if (!ok || !fin(ss) || !fin(residual)) {
      status = -3;
      break;
    }
    if (residual <= tol) {
      float tn = 0.0f;
      if (!J.true_residual(t.data(), &tn)) {
        status = -3;
        break;
      }
      if (tn <= tol) {
        status = 0, residual = tn;
        break;
      }
    }
    if (!J.apply(s, s_hat)) {
      status = -3;
      break;
    }
    A.apply(s_hat.data(), t.data());
    if (!all_finite(t)) {
      status = -3;
      break;
    }
    const double ts = dot(t, s), tt = dot(t, t);
    if (!fin(ts) || !fin(tt)) {
      status = -3;
      break;
    }
    if (near_zero(tt, tt, 1.0)) {
      status = -1;
      break;
    }
    omega = ts / tt;
    if (!fin(omega)) {
      status = -3;
      break;
    }
    double rn = 0.0;
    ok = true;
    for (int64_t i = 0; i < n; ++i) {
      const double xi = static_cast<double>(x[i]) + omega * static_cast<double>(s_hat[i]);
      const double ri = static_cast<double>(s[i]) - omega * static_cast<double>(t[i]);
      x[i] = static_cast<float>(xi);
      r[i] = static_cast<float>(ri);
      rn += ri * ri;
      ok = ok && fin(xi) && fin(ri) && fin(x[i]) && fin(r[i]);
    }
    residual = static_cast<float>(std::sqrt(std::max(rn, 0.0)));
    if (!ok || !fin(rn) || !fin(residual)) {
      status = -3;
      break;
    }
    if (residual <= tol) {
      float tn = 0.0f;
      if (!J.true_residual(r.data(), &tn)) {
        status = -3;
        break;
      }
      residual = tn;
      if (tn <= tol) {
        status = 0;
        break;
      }
    }
    if (std::fabs(omega) <= eps) {
      status = -1;
      break;
    }
    rho_prev = rho;
  }
  if (status > 0 || status == -1) {
    float tn = 0.0f;
    if (!J.true_residual(r.data(), &tn)) {
      status = -3;
    } else {
      residual = tn;
      if (tn <= tol) status = 0;
    }
  }
  *res = {status, done, residual, 0};
}

msx_status check(const char *op, msx_itype it, int64_t n, int64_t nnz, const void *data,
                 const void *indices, const void *indptr, const void *b, const void *x0, void *x,
                 int64_t maxiter, msx_solver_result *result) {
  if (it != MSX_I32 && it != MSX_I64)
    return msx::fail(MSX_ETYPE, std::string(op) + " requires int32 or int64 indices.");
  if (n <= 0) return msx::fail(MSX_EINVAL, std::string(op) + " requires a non-empty square matrix.");
  if (maxiter < 0) return msx::fail(MSX_EINVAL, std::string(op) + " maxiter must be non-negative.");
  if (nnz < 0) return msx::fail(MSX_EINVAL, std::string(op) + " nnz must be non-negative.");
  if (indptr == nullptr || b == nullptr || x0 == nullptr || x == nullptr || result == nullptr ||
      (nnz > 0 && (data == nullptr || indices == nullptr)))
    return msx::fail(MSX_EINVAL, std::string(op) + " buffers must be non-NULL.");
  return MSX_OK;
}

}  // namespace

extern "C" msx_status msx_csr_bicgstab_cpu(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                           const void *indices, const void *indptr, const float *b,
                                           const float *x0, float *x, float rtol, float atol,
                                           int64_t maxiter, msx_solver_result *result) {
  msx::clear_error();
  const msx_status st =
      check("csr_bicgstab", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  try {
    if (it == MSX_I32)
      bicgstab(Csr<int32_t>{n, data, static_cast<const int32_t *>(indices),
                            static_cast<const int32_t *>(indptr)},
               b, x0, x, rtol, atol, maxiter, result);
    else
      bicgstab(Csr<int64_t>{n, data, static_cast<const int64_t *>(indices),
                            static_cast<const int64_t *>(indptr)},
               b, x0, x, rtol, atol, maxiter, result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_bicgstab: out of host memory.");
  }
  return MSX_OK;
}

extern "C" msx_status msx_csr_bicgstab_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                                  const float *data, const void *indices,
                                                  const void *indptr, const float *b,
                                                  const float *x0, const float *inv_diag, float *x,
                                                  float rtol, float atol, int64_t maxiter,
                                                  msx_solver_result *result) {
  msx::clear_error();
  msx_status st =
      check("csr_bicgstab_jacobi", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  if (inv_diag == nullptr)
    return msx::fail(MSX_EINVAL, "csr_bicgstab_jacobi buffers must be non-NULL.");
  try {
    if (it == MSX_I32)
      bicgstab_jacobi(Csr<int32_t>{n, data, static_cast<const int32_t *>(indices),
                                   static_cast<const int32_t *>(indptr)},
                      b, x0, inv_diag, x, rtol, atol, maxiter, result);
    else
      bicgstab_jacobi(Csr<int64_t>{n, data, static_cast<const int64_t *>(indices),
                                   static_cast<const int64_t *>(indptr)},
                      b, x0, inv_diag, x, rtol, atol, maxiter, result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_bicgstab_jacobi: out of host memory.");
  }
  return MSX_OK;
}

extern "C" msx_status msx_csr_minres_cpu(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                         const void *indices, const void *indptr, const float *b,
                                         const float *x0, float *x, float rtol, float atol,
                                         int64_t maxiter, float shift,
                                         msx_solver_result *result) {
  msx::clear_error();
  const msx_status st =
      check("csr_minres", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  try {
    if (it == MSX_I32)
      minres(Csr<int32_t>{n, data, static_cast<const int32_t *>(indices),
                          static_cast<const int32_t *>(indptr)},
             b, x0, nullptr, x, rtol, atol, maxiter, shift, result);
    else
      minres(Csr<int64_t>{n, data, static_cast<const int64_t *>(indices),
                          static_cast<const int64_t *>(indptr)},
             b, x0, nullptr, x, rtol, atol, maxiter, shift, result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_minres: out of host memory.");
  }
  return MSX_OK;
}

extern "C" msx_status msx_csr_minres_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                                const float *data, const void *indices,
                                                const void *indptr, const float *b,
                                                const float *x0, const float *inv_diag, float *x,
                                                float rtol, float atol, int64_t maxiter,
                                                float shift, msx_solver_result *result) {
  msx::clear_error();
  msx_status st =
      check("csr_minres_jacobi", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  if (inv_diag == nullptr)
    return msx::fail(MSX_EINVAL, "csr_minres_jacobi buffers must be non-NULL.");
  try {
    if (it == MSX_I32)
      minres(Csr<int32_t>{n, data, static_cast<const int32_t *>(indices),
                          static_cast<const int32_t *>(indptr)},
             b, x0, inv_diag, x, rtol, atol, maxiter, shift, result);
    else
      minres(Csr<int64_t>{n, data, static_cast<const int64_t *>(indices),
                          static_cast<const int64_t *>(indptr)},
             b, x0, inv_diag, x, rtol, atol, maxiter, shift, result);
  } catch (const std::bad_alloc &) {
    return msx::fail(MSX_ENOMEM, "csr_minres_jacobi: out of host memory.");
  }
  return MSX_OK;
}
