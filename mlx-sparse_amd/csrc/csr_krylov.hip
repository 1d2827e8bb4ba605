// csr_krylov.hip - BiCGSTAB and MINRES on a square float32 CSR matrix, with
// the loop resident on the device.
//
// The reference runs both GPU solvers in one 256-thread threadgroup
// (reference: src/linalg/bicgstab/bicgstab.metal:54-320,
// src/linalg/minres/minres.metal:71-140).  Here every step is device-wide:
// the path's SpMV with the matrix's plan, then fused vector passes whose
// double partial sums feed the next pass (msx_solver.h: every workgroup adds
// the partials in workgroup order and takes the same scalar decision, so no
// workgroup waits on another and a solve is reproducible run to run).  The
// scalar rules (tolerances, breakdown tests, status codes) follow the
// reference's CPU loops: src/linalg/bicgstab/bicgstab.cpp:80-362
// (csr_bicgstab_cpu_impl) and src/linalg/minres/minres.cpp:93-312
// (csr_minres_cpu_impl).
//
// BiCGSTAB, per iteration k:
//   bi_p   the previous iteration's residual test (the r-check), rho, the
//          breakdown tests, beta, p = r + beta (p - omega v)
//   v = A p
//   bi_v   r_hat.v, v.v
//   bi_s   alpha; s = r - alpha v, x += alpha p; s.s
//   t = A s
//   bi_t   the s-check (||s|| under the tolerance); t.s, t.t
//   bi_r   omega; x += omega s, r = s - omega t; r.r, r_hat.r
// When ||s|| or ||r|| falls under the tolerance the reference confirms on
// the true residual b - A x: the device pauses the loop there, and the host
// computes that residual on the device (SpMV + bi_resid + bi_check) and
// resumes or ends the solve.  This happens near convergence only.
//
// MINRES, per iteration k (the reference computes the true residual of
// every iterate):
//   mr_v   the previous iterate's residual test; v = r2 / beta
//   av = A v
//   mr_a   av -= shift v (and (beta / oldb) r1); v.av
//   mr_b   av -= (alfa / beta) r2, the next Lanczos vector; its norm
//   mr_x   the next Givens rotation (every workgroup, same sums); w, x
//   q = A x
//   mr_r   b - (q - shift x); its norm
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <string>
#include <utility>

#include "msx_device.h"
#include "msx_internal.h"
#include "msx_solver.h"
#include "msx_sparse.h"

namespace msx {
namespace {

using namespace solver;

constexpr double kEps = static_cast<double>(FLT_EPSILON);

// The reference's breakdown test of a dot product (bicgstab.cpp:43-49).
__device__ inline bool near_zero(double value, double lhs_norm2, double rhs_norm2) {
  const double scale = sqrt(max0(lhs_norm2 * rhs_norm2));
  return !fin(scale) || fabs(value) <= kEps * fmax(1.0, scale);
}

__device__ inline bool lead() { return blockIdx.x == 0 && threadIdx.x == 0; }

// ---------------------------------------------------------------------------
// BiCGSTAB

enum Pause : int32_t { kNoPause = 0, kSCheck = 1, kRCheck = 2 };

struct BiState {
  double rho[2];  // rho of iteration k at rho[k & 1]
  double alpha;   // of the last bi_s, read by the next bi_p
  double omega;   // of the last bi_r, read by the next bi_p and the checks
  double hh;      // r_hat . r_hat
  float tol;
  float residual;     // the reported residual norm
  int32_t status;     // 0, maxiter, -1, -3
  int32_t completed;  // completed iterations
  int32_t running;    // 1 while iterating
  int32_t pause;      // Pause: a true-residual check the host must run
  int32_t pause_it;   // the iteration it belongs to
};

__device__ inline void bi_stop(BiState *st, int32_t status, int32_t completed) {
  st->status = status;
  st->completed = completed;
  st->running = 0;
}

// r = r_hat = b - A x.  Slots: b.b, non-finite count, r.r (twice: rho and
// r.r of the first iteration, r_hat = r).
__global__ void __launch_bounds__(kSolverThreads)
    bi_start(const float *__restrict__ b, const float *__restrict__ x, const float *__restrict__ ax,
             float *__restrict__ r, float *__restrict__ r_hat, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const float ri = b[i] - ax[i];
    r[i] = ri;
    r_hat[i] = ri;
    v[0] += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    if (!(fin(ri) && fin(ax[i]) && fin(b[i]) && fin(x[i]))) v[1] += 1.0;
    v[2] += static_cast<double>(ri) * static_cast<double>(ri);
  })
  v[3] = v[2];
  write_partials(v, part);
}

// bicgstab.cpp:123-167.  J (the Jacobi loop, preconditioners/bicgstab/
// bicgstab.cpp:150-200): ||b|| rounded to float before its square root, and
// a failed start reports an infinite residual.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    bi_decide_start(const double *part, int nparts, float rtol, float atol, int64_t maxiter,
                    BiState *st) {
  double t[kSlots];
  read_totals(part, nparts, t);
  if (threadIdx.x != 0) return;
  const float b_norm = J ? sqrtf(max0(static_cast<float>(t[0])))
                         : static_cast<float>(sqrt(max0(t[0])));
  const float scaled = rtol * b_norm;
  st->tol = atol > scaled ? atol : scaled;
  st->residual = static_cast<float>(sqrt(max0(t[2])));
  st->hh = t[2];
  st->rho[0] = st->rho[1] = 1.0;
  st->alpha = st->omega = 1.0;
  st->pause = kNoPause;
  st->pause_it = 0;
  st->completed = 0;
  if (t[1] != 0.0 || !fin(b_norm) || !fin(st->tol) || !fin(t[2]) || !fin(st->residual)) {
    if (J) st->residual = INFINITY;
    bi_stop(st, -3, 0);
  } else if (st->residual <= st->tol) {
    bi_stop(st, 0, 0);
  } else {
    st->status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
    st->running = maxiter > 0 ? 1 : 0;
  }
}

// The r-check that closes iteration k (bicgstab.cpp:328-355) from the
// update pass's slots (r.r of the unrounded updates, non-finite count):
// returns false when the loop stops or pauses there.
__device__ inline bool bi_close(const double (&t)[kSlots], int32_t k, BiState *st) {
  const float res = static_cast<float>(sqrt(max0(t[0])));
  const bool ld = lead();
  if (t[1] != 0.0 || !fin(t[0]) || !fin(res)) {
    if (ld) {
      st->residual = res;
      bi_stop(st, -3, k);
    }
    return false;
  }
  if (res <= st->tol) {
    if (ld) {
      st->residual = res;
      st->pause = kRCheck;
      st->pause_it = k;
      st->running = 0;
    }
    return false;
  }
  if (fabs(st->omega) <= kEps) {
    if (ld) {
      st->residual = res;
      bi_stop(st, -1, k);
    }
    return false;
  }
  return true;
}

// Iteration k's first pass (bicgstab.cpp:180-230).  `dots`: slots 2 and 3
// are r_hat.r and r.r; with `close_prev`, slots 0 and 1 close iteration
// k - 1 first.  J: also p_hat = inv_diag p (its non-finite entries counted
// with p's).
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    bi_p(const float *__restrict__ r, float *__restrict__ p, const float *__restrict__ v,
         const float *__restrict__ inv_diag, float *__restrict__ p_hat, int64_t n, int32_t k,
         int close_prev, const double *dots, double *part, int nparts, BiState *st) {
  if (!st->running) return;
  constexpr int NV = J ? 4 : 3;
  double pin[kSlots];
  load_partials(dots, nparts, pin);
  const float *vec[NV];
  vec[0] = r, vec[1] = p, vec[2] = v;
  if constexpr (J) vec[3] = inv_diag;
  Round<NV> first;
  load_round<NV>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  if (close_prev && !bi_close(t, k - 1, st)) return;
  if (close_prev && lead()) st->residual = static_cast<float>(sqrt(max0(t[0])));
  const double rho = t[2], rr = t[3], hh = st->hh;
  int32_t verdict = 1;
  double beta = 0.0, omega = st->omega;
  if (!fin(rho) || !fin(hh) || !fin(rr)) verdict = -3;
  else if (near_zero(rho, hh, rr)) verdict = -1;
  else if (k > 1) {
    if (fabs(omega) <= kEps) {
      verdict = -1;
    } else {
      beta = (rho / st->rho[(k - 1) & 1]) * (st->alpha / omega);
      if (!fin(beta)) verdict = -3;
    }
  }
  if (verdict != 1) {
    if (lead()) bi_stop(st, verdict, k - 1);
    return;
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  // J: p_hat = inv_diag p in float (the Jacobi apply, bicgstab.cpp:500-507)
  auto hat = [&](int64_t i, float pf, const float(&e)[NV]) {
    if constexpr (J) {
      const float ph = e[NV - 1] * pf;
      p_hat[i] = ph;
      if (!fin(ph)) acc[1] += 1.0;
    }
  };
  if (k == 1) {
    for_rounds<NV>(vec, n, first, [&](int64_t i, const float(&e)[NV]) {
      p[i] = e[0];
      hat(i, e[0], e);
    });
  } else {
    for_rounds<NV>(vec, n, first, [&](int64_t i, const float(&e)[NV]) {
      const double pi = static_cast<double>(e[0]) +
                        beta * (static_cast<double>(e[1]) - omega * static_cast<double>(e[2]));
      const float pf = static_cast<float>(pi);
      p[i] = pf;
      if (!fin(pi) || !fin(pf)) acc[1] += 1.0;
      hat(i, pf, e);
    });
  }
  write_partials(acc, part);
  if (lead()) st->rho[k & 1] = rho;
}

// The p pass's non-finite count, then r_hat.v and v.v.
__global__ void __launch_bounds__(kSolverThreads)
    bi_v(const float *__restrict__ r_hat, const float *__restrict__ v, int64_t n, int32_t k,
         const double *p_part, double *part, int nparts, BiState *st) {
  if (!st->running) return;
  double pin[kSlots];
  load_partials(p_part, nparts, pin);
  const float *const vec[2] = {r_hat, v};
  Round<2> first;
  load_round<2>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  if (t[1] != 0.0) {
    if (lead()) bi_stop(st, -3, k - 1);
    return;
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<2>(vec, n, first, [&](int64_t, const float(&e)[2]) {
    const double vi = e[1];
    acc[0] += static_cast<double>(e[0]) * vi;
    acc[1] += vi * vi;
  });
  write_partials(acc, part);
}

// alpha (bicgstab.cpp:232-255); s = r - alpha v, x += alpha p; s.s of the
// unrounded s, non-finite count.  J: `p` is p_hat, and s_hat = inv_diag s
// is written too (slot 2: its non-finite count).
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    bi_s(const float *__restrict__ r, const float *__restrict__ v, const float *__restrict__ p,
         const float *__restrict__ inv_diag, float *__restrict__ x, float *__restrict__ s,
         float *__restrict__ s_hat, int64_t n, int32_t k, const double *v_part, double *part,
         int nparts, BiState *st) {
  if (!st->running) return;
  constexpr int NV = J ? 5 : 4;
  double pin[kSlots];
  load_partials(v_part, nparts, pin);
  const float *vec[NV];
  vec[0] = r, vec[1] = v, vec[2] = x, vec[3] = p;
  if constexpr (J) vec[4] = inv_diag;
  Round<NV> first;
  load_round<NV>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  const double hv = t[0], vv = t[1];
  int32_t verdict = 1;
  double alpha = 0.0;
  if (!fin(hv) || !fin(vv)) verdict = -3;
  else if (near_zero(hv, st->hh, vv)) verdict = -1;
  else {
    alpha = st->rho[k & 1] / hv;
    if (!fin(alpha)) verdict = -3;
  }
  if (verdict != 1) {
    if (lead()) bi_stop(st, verdict, k - 1);
    return;
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<NV>(vec, n, first, [&](int64_t i, const float(&e)[NV]) {
    const double si = static_cast<double>(e[0]) - alpha * static_cast<double>(e[1]);
    const double xi = static_cast<double>(e[2]) + alpha * static_cast<double>(e[3]);
    const float sf = static_cast<float>(si), xf = static_cast<float>(xi);
    s[i] = sf;
    x[i] = xf;
    acc[0] += si * si;
    if (!(fin(si) && fin(xi) && fin(sf) && fin(xf))) acc[1] += 1.0;
    if constexpr (J) {
      const float sh = e[NV - 1] * sf;
      s_hat[i] = sh;
      if (!fin(sh)) acc[2] += 1.0;
    }
  });
  write_partials(acc, part);
  if (lead()) {
    st->alpha = alpha;
    st->completed = k;
  }
}

// The s-check (bicgstab.cpp:270-287; skipped when the host has already
// run it), then t.s and t.t.  J: the reported residual becomes ||s||
// (preconditioners/bicgstab/bicgstab.cpp:314), and a non-finite s_hat ends
// the solve after the check.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    bi_t(const float *__restrict__ s, const float *__restrict__ t_vec, int64_t n, int32_t k,
         int check, const double *s_part, double *part, int nparts, BiState *st) {
  if (!st->running) return;
  double pin[kSlots] = {0.0, 0.0, 0.0, 0.0};
  if (check || J) load_partials(s_part, nparts, pin);
  const float *const vec[2] = {s, t_vec};
  Round<2> first;
  load_round<2>(vec, first_base(), n, first);
  double t[kSlots] = {0.0, 0.0, 0.0, 0.0};
  if (check || J) reduce_partials(pin, nparts, t);
  if (check) {
    const float s_norm = static_cast<float>(sqrt(max0(t[0])));
    if (J && lead()) st->residual = s_norm;
    if (t[1] != 0.0 || !fin(t[0]) || !fin(s_norm)) {
      if (lead()) bi_stop(st, -3, k);
      return;
    }
    if (s_norm <= st->tol) {
      if (lead()) {
        st->pause = kSCheck;
        st->pause_it = k;
        st->running = 0;
      }
      return;
    }
  }
  if (J && t[2] != 0.0) {
    if (lead()) bi_stop(st, -3, k);
    return;
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<2>(vec, n, first, [&](int64_t, const float(&e)[2]) {
    const double ti = e[1];
    acc[0] += ti * static_cast<double>(e[0]);
    acc[1] += ti * ti;
  });
  write_partials(acc, part);
}

// omega (bicgstab.cpp:290-305); x += omega s, r = s - omega t.  Slots: r.r
// of the unrounded r, non-finite count, r_hat.r and r.r of the stored r
// (the next iteration's rho and r.r).  J: x += omega s_hat.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    bi_r(const float *__restrict__ s, const float *__restrict__ t_vec,
         const float *__restrict__ s_hat, float *__restrict__ x, float *__restrict__ r,
         const float *__restrict__ r_hat, int64_t n, int32_t k, const double *t_part,
         double *part, int nparts, BiState *st) {
  if (!st->running) return;
  constexpr int NV = J ? 5 : 4;
  double pin[kSlots];
  load_partials(t_part, nparts, pin);
  const float *vec[NV];
  vec[0] = x, vec[1] = s, vec[2] = t_vec, vec[3] = r_hat;
  if constexpr (J) vec[4] = s_hat;
  constexpr int kStep = J ? 4 : 1;  // x advances along s_hat (J) or s
  Round<NV> first;
  load_round<NV>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  const double ts = t[0], tt = t[1];
  int32_t verdict = 1;
  double omega = 0.0;
  if (!fin(ts) || !fin(tt)) verdict = -3;
  else if (near_zero(tt, tt, 1.0)) verdict = -1;
  else {
    omega = ts / tt;
    if (!fin(omega)) verdict = -3;
  }
  if (verdict != 1) {
    if (lead()) bi_stop(st, verdict, k);
    return;
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<NV>(vec, n, first, [&](int64_t i, const float(&e)[NV]) {
    const double xi = static_cast<double>(e[0]) + omega * static_cast<double>(e[kStep]);
    const double ri = static_cast<double>(e[1]) - omega * static_cast<double>(e[2]);
    const float xf = static_cast<float>(xi), rf = static_cast<float>(ri);
    x[i] = xf;
    r[i] = rf;
    acc[0] += ri * ri;
    if (!(fin(xi) && fin(ri) && fin(xf) && fin(rf))) acc[1] += 1.0;
    acc[2] += static_cast<double>(e[3]) * static_cast<double>(rf);
    acc[3] += static_cast<double>(rf) * static_cast<double>(rf);
  });
  write_partials(acc, part);
  if (lead()) st->omega = omega;
}

// One workgroup after the last launched iteration k: closes it.
__global__ void __launch_bounds__(kSolverThreads)
    bi_finish(const double *r_part, int nparts, int32_t k, BiState *st) {
  if (!st->running) return;
  double t[kSlots];
  read_totals(r_part, nparts, t);
  if (!bi_close(t, k, st)) return;
  if (threadIdx.x == 0) {
    st->residual = static_cast<float>(sqrt(max0(t[0])));
    st->running = 0;
  }
}

// dst = b - A x (A x in ax).  Slots: dst.dst, non-finite count, r_hat.dst,
// dst.dst - the layout bi_p reads when the loop resumes with dst as r.  J
// counts the entries of A x and dst only (bicgstab.cpp:166-192 there).
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    bi_resid(const float *__restrict__ b, const float *__restrict__ ax, const float *__restrict__ x,
             const float *__restrict__ r_hat, float *__restrict__ dst, int64_t n, double *part) {
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const float a = ax[i];
    const float ri = b[i] - a;
    dst[i] = ri;
    acc[0] += static_cast<double>(ri) * static_cast<double>(ri);
    if (!(fin(ri) && fin(a) && (J || fin(x[i])))) acc[1] += 1.0;
    acc[2] += static_cast<double>(r_hat[i]) * static_cast<double>(ri);
  })
  acc[3] = acc[0];
  write_partials(acc, part);
}

// The host-driven true-residual checks (bicgstab.cpp:274-287, 319-332,
// 340-350): kind kSCheck / kRCheck resume the loop (running = 1) when the
// true residual is above the tolerance; kind 3 is the check after the loop.
// J: a failed evaluation (the reference's exception) leaves the reported
// residual as it was.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    bi_check(const double *part, int nparts, int32_t kind, BiState *st) {
  double t[kSlots];
  read_totals(part, nparts, t);
  if (threadIdx.x != 0) return;
  const float norm = static_cast<float>(sqrt(max0(t[0])));
  const bool finite = t[1] == 0.0 && fin(t[0]) && fin(norm);
  const int32_t k = st->pause_it;
  st->pause = kNoPause;
  if (kind == 3) {
    if (!J || finite) st->residual = norm;
    if (!finite) st->status = -3;
    else if (norm <= st->tol) st->status = 0;
    return;
  }
  if (!finite) {
    if (!J) st->residual = norm;
    bi_stop(st, -3, k);
  } else if (norm <= st->tol) {
    st->residual = norm;
    bi_stop(st, 0, k);
  } else if (kind == kRCheck) {
    st->residual = norm;
    if (fabs(st->omega) <= kEps) bi_stop(st, -1, k);
    else st->running = 1;
  } else {
    st->running = 1;
  }
}

// ---------------------------------------------------------------------------
// MINRES

struct Givens {
  double beta, oldb, dbar, epsln, phibar, cs, sn;
};

struct MrState {
  Givens g[2];  // after iteration k at g[k & 1] (g[0]: the start)
  float tol;
  float residual;  // the last true residual
  int32_t status, completed, running;
};

__device__ inline void mr_stop(MrState *st, int32_t status, int32_t completed) {
  st->status = status;
  st->completed = completed;
  st->running = 0;
}

// r2 = b - (A x - shift x) (minres.cpp:68-91, 186-191).  Slots: b.b, r2.r2,
// non-finite count; J (the Jacobi loop, preconditioners/minres/
// minres.cpp:93-330): also y = inv_diag r2 and slot 3 r2.y.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    mr_start(const float *__restrict__ b, const float *__restrict__ x, const float *__restrict__ ax,
             float shift, const float *__restrict__ inv_diag, float *__restrict__ r2,
             float *__restrict__ y, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const float ai = ax[i] - shift * x[i];
    const float ri = b[i] - ai;
    r2[i] = ri;
    v[0] += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    v[1] += static_cast<double>(ri) * static_cast<double>(ri);
    if (!(fin(ai) && fin(ri))) v[2] += 1.0;
    if constexpr (J) {
      const float yi = inv_diag[i] * ri;
      y[i] = yi;
      v[3] += static_cast<double>(ri) * static_cast<double>(yi);
    }
  })
  write_partials(v, part);
}

// The Jacobi loop's preconditioner test (minres.cpp:160-166 there): slot 0
// counts the inverse diagonal entries that are not > 0.
__global__ void __launch_bounds__(kSolverThreads)
    mr_diag_check(const float *__restrict__ inv_diag, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    if (!(inv_diag[i] > 0.0f)) v[0] += 1.0;
  })
  write_partials(v, part);
}

// minres.cpp:160-210.  J: a preconditioner entry not > 0 stops the start
// with -2 (after the non-finite test, before the convergence test); beta
// from r2.y, and its failure is -2.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    mr_decide_start(const double *part, const double *diag_part, int nparts, float rtol,
                    float atol, int64_t maxiter, MrState *st) {
  double t[kSlots], dg[kSlots] = {0.0, 0.0, 0.0, 0.0};
  read_totals(part, nparts, t);
  if (J) read_totals(diag_part, nparts, dg);
  if (threadIdx.x != 0) return;
  const float b_norm = static_cast<float>(sqrt(max0(t[0])));
  const float scaled = rtol * b_norm;
  st->tol = atol > scaled ? atol : scaled;
  st->residual = static_cast<float>(sqrt(max0(t[1])));
  st->completed = 0;
  const int32_t budget = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
  if (t[2] != 0.0 || !fin(st->residual)) {
    mr_stop(st, -3, 0);
    return;
  }
  if (J && dg[0] != 0.0) {
    mr_stop(st, -2, 0);
    return;
  }
  if (st->residual <= st->tol) {
    mr_stop(st, 0, 0);
    return;
  }
  if (maxiter == 0) {
    mr_stop(st, budget, 0);
    return;
  }
  const double beta_sq = static_cast<double>(static_cast<float>(J ? t[3] : t[1]));
  if (!fin(beta_sq) || beta_sq <= 0.0) {
    mr_stop(st, J ? -2 : -1, 0);
    return;
  }
  const double beta = sqrt(beta_sq);
  st->g[0] = Givens{beta, 0.0, 0.0, 0.0, beta, -1.0, 0.0};
  st->status = budget;
  st->running = 1;
}

// The true-residual test that ends iteration k (minres.cpp:285-300), from
// the residual pass's slots (r.r, non-finite count).
__device__ inline bool mr_close(const double (&t)[kSlots], int32_t k, MrState *st) {
  const float res = static_cast<float>(sqrt(max0(t[0])));
  int32_t verdict = 1;
  if (t[1] != 0.0 || !fin(res)) verdict = -3;
  else if (res <= st->tol) verdict = 0;
  else if (st->g[k & 1].beta <= kEps) verdict = -1;
  if (lead()) st->residual = res;
  if (verdict != 1) {
    if (lead()) mr_stop(st, verdict, k);
    return false;
  }
  return true;
}

// Closes iteration k - 1, then v = r2 / beta (minres.cpp:212-222); J: `r2`
// is y = M r2, and a failed beta test is -2.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    mr_v(const float *__restrict__ r2, float *__restrict__ v, int64_t n, int32_t k,
         const double *res_part, int nparts, MrState *st) {
  if (!st->running) return;
  double pin[kSlots] = {0.0, 0.0, 0.0, 0.0};
  if (k > 1) load_partials(res_part, nparts, pin);
  const float *const vec[1] = {r2};
  Round<1> first;
  load_round<1>(vec, first_base(), n, first);
  if (k > 1) {
    double t[kSlots];
    reduce_partials(pin, nparts, t);
    if (!mr_close(t, k - 1, st)) return;
  }
  const double beta = st->g[(k - 1) & 1].beta;
  if (!fin(beta) || beta <= kEps) {
    if (lead()) mr_stop(st, J ? -2 : -1, k - 1);
    return;
  }
  const double inv_beta = 1.0 / beta;
  for_rounds<1>(vec, n, first, [&](int64_t i, const float(&e)[1]) {
    v[i] = static_cast<float>(inv_beta * static_cast<double>(e[0]));
  });
}

// av -= shift v, av -= (beta / oldb) r1 from the second iteration on
// (minres.cpp:224-236); v.av.
__global__ void __launch_bounds__(kSolverThreads)
    mr_a(const float *__restrict__ v, float *__restrict__ av, const float *__restrict__ r1,
         float shift, int64_t n, int32_t k, double *part, MrState *st) {
  if (!st->running) return;
  const Givens g = st->g[(k - 1) & 1];
  float prev_scale = 0.0f;
  if (k >= 2) {
    if (!fin(g.oldb) || fabs(g.oldb) <= kEps) {
      if (lead()) mr_stop(st, -1, k - 1);
      return;
    }
    prev_scale = static_cast<float>(g.beta / g.oldb);
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  if (k >= 2) {
    MSX_SOLVER_LOOP({
      float a = av[i] - shift * v[i];
      a = a - prev_scale * r1[i];
      av[i] = a;
      acc[0] += static_cast<double>(v[i]) * static_cast<double>(a);
    })
  } else {
    MSX_SOLVER_LOOP({
      const float a = av[i] - shift * v[i];
      av[i] = a;
      acc[0] += static_cast<double>(v[i]) * static_cast<double>(a);
    })
  }
  write_partials(acc, part);
}

// alfa; av -= (alfa / beta) r2 (minres.cpp:238-246); the new r2's norm.
// J: also y = inv_diag av, and the sum is av.y.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    mr_b(float *__restrict__ av, const float *__restrict__ r2, const float *__restrict__ inv_diag,
         float *__restrict__ y, int64_t n, int32_t k, const double *a_part, double *part,
         int nparts, MrState *st) {
  if (!st->running) return;
  constexpr int NV = J ? 3 : 2;
  double pin[kSlots];
  load_partials(a_part, nparts, pin);
  const float *vec[NV];
  vec[0] = av, vec[1] = r2;
  if constexpr (J) vec[2] = inv_diag;
  Round<NV> first;
  load_round<NV>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  const double alfa = static_cast<double>(static_cast<float>(t[0]));
  if (!fin(alfa)) {
    if (lead()) mr_stop(st, -3, k - 1);
    return;
  }
  const float diag_scale = static_cast<float>(alfa / st->g[(k - 1) & 1].beta);
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<NV>(vec, n, first, [&](int64_t i, const float(&e)[NV]) {
    const float a = e[0] - diag_scale * e[1];
    av[i] = a;
    if constexpr (J) {
      const float yi = e[2] * a;
      y[i] = yi;
      acc[0] += static_cast<double>(a) * static_cast<double>(yi);
    } else {
      acc[0] += static_cast<double>(a) * static_cast<double>(a);
    }
  });
  write_partials(acc, part);
}

// The next Givens rotation (minres.cpp:248-275), then w and x
// (minres.cpp:277-290).  The new w is written over w2 (the host swaps the
// two).  Slots: non-finite count.  J: a failed beta test is -2.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    mr_x(const float *__restrict__ v, const float *__restrict__ w, float *__restrict__ w2,
         float *__restrict__ x, int64_t n, int32_t k, const double *a_part,
         const double *b_part, double *part, int nparts, MrState *st) {
  if (!st->running) return;
  double pa[kSlots], pb[kSlots];
  load_partials(a_part, nparts, pa);
  load_partials(b_part, nparts, pb);
  const float *const vec[4] = {v, w, w2, x};
  Round<4> first;
  load_round<4>(vec, first_base(), n, first);
  double ta[kSlots], tb[kSlots];
  reduce_partials(pa, nparts, ta);
  reduce_partials(pb, nparts, tb);
  const Givens g = st->g[(k - 1) & 1];
  const double alfa = static_cast<double>(static_cast<float>(ta[0]));
  const double beta_sq = static_cast<double>(static_cast<float>(tb[0]));
  if (!fin(beta_sq) || beta_sq < 0.0) {
    if (lead()) mr_stop(st, J ? -2 : -1, k - 1);
    return;
  }
  Givens h;
  h.oldb = g.beta;
  h.beta = sqrt(max0(beta_sq));
  const double oldeps = g.epsln;
  const double delta = g.cs * g.dbar + g.sn * alfa;
  const double gbar = g.sn * g.dbar - g.cs * alfa;
  h.epsln = g.sn * h.beta;
  h.dbar = -g.cs * h.beta;
  double gamma = hypot(gbar, h.beta);
  if (!fin(gamma)) {
    if (lead()) mr_stop(st, -3, k - 1);
    return;
  }
  gamma = fmax(gamma, kEps);
  h.cs = gbar / gamma;
  h.sn = h.beta / gamma;
  const double phi = h.cs * g.phibar;
  h.phibar = h.sn * g.phibar;
  if (!fin(phi) || !fin(h.phibar)) {
    if (lead()) mr_stop(st, -3, k - 1);
    return;
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<4>(vec, n, first, [&](int64_t i, const float(&e)[4]) {
    const double older = e[2], old = e[1];
    const float wn =
        static_cast<float>((static_cast<double>(e[0]) - oldeps * older - delta * old) / gamma);
    const float xn = e[3] + static_cast<float>(phi * static_cast<double>(wn));
    w2[i] = wn;
    x[i] = xn;
    if (!(fin(wn) && fin(xn))) acc[0] += 1.0;
  });
  write_partials(acc, part);
  if (lead()) {
    st->g[k & 1] = h;
    st->completed = k;
  }
}

// The x pass's non-finite count, then b - (A x - shift x) (A x in ax).
// Slots: r.r, non-finite count.
__global__ void __launch_bounds__(kSolverThreads)
    mr_r(const float *__restrict__ b, const float *__restrict__ x, const float *__restrict__ ax,
         float shift, int64_t n, int32_t k, const double *x_part, double *part, int nparts,
         MrState *st) {
  if (!st->running) return;
  double pin[kSlots];
  load_partials(x_part, nparts, pin);
  const float *const vec[3] = {b, x, ax};
  Round<3> first;
  load_round<3>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  if (t[0] != 0.0) {
    if (lead()) mr_stop(st, -3, k);
    return;
  }
  double acc[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<3>(vec, n, first, [&](int64_t, const float(&e)[3]) {
    const float ai = e[2] - shift * e[1];
    const float ri = e[0] - ai;
    acc[0] += static_cast<double>(ri) * static_cast<double>(ri);
    if (!(fin(ai) && fin(ri))) acc[1] += 1.0;
  });
  write_partials(acc, part);
}

// One workgroup after the last launched iteration k: closes it.
__global__ void __launch_bounds__(kSolverThreads)
    mr_finish(const double *res_part, int nparts, int32_t k, MrState *st) {
  if (!st->running) return;
  double t[kSlots];
  read_totals(res_part, nparts, t);
  if (!mr_close(t, k, st)) return;
  if (threadIdx.x == 0) st->running = 0;
}

__global__ void copy_vec(const float *__restrict__ src, float *__restrict__ dst, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kSolverThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kSolverThreads)
    dst[i] = src[i];
}

__global__ void zero_vec(float *__restrict__ dst, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kSolverThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kSolverThreads)
    dst[i] = 0.0f;
}

// ---------------------------------------------------------------------------
// Host side

struct System {
  int64_t n, nnz;
  msx_itype it;
  const float *data;
  const void *indices, *indptr;
  const msx_csr_plan *plan;
  hipStream_t stream;
  dim3 grid, block;
  int nparts;
};

msx_status spmv(const System &s, const float *x, float *y) {
  return launch_spmv(MSX_F32, s.it, s.n, s.n, s.nnz, s.data, s.indices, s.indptr, x, y, s.plan,
                     s.stream);
}

// Scratch from the stream-ordered allocator: `nvec` vectors of n floats, a
// 256-byte state block and `nparts` partial-sum arrays.
struct Scratch {
  char *base = nullptr;
  hipStream_t stream = nullptr;
  size_t vec = 0;
  ~Scratch() {
    if (base) (void)hipFreeAsync(base, stream);
  }
  msx_status alloc(int64_t n, int nvec, int npart_arrays) {
    vec = (static_cast<size_t>(n) * sizeof(float) + 255) / 256 * 256;
    const size_t part_bytes = sizeof(double) * kSlots * kSolverMaxBlocks;
    MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&base),
                               nvec * vec + 256 + npart_arrays * part_bytes, stream));
    nv = nvec;
    return MSX_OK;
  }
  float *vector(int i) const { return reinterpret_cast<float *>(base + i * vec); }
  void *state() const { return base + nv * vec; }
  double *part(int i) const {
    return reinterpret_cast<double *>(base + nv * vec + 256 +
                                      i * sizeof(double) * kSlots * kSolverMaxBlocks);
  }
  int nv = 0;
};

template <class State>
msx_status read_state(const System &s, const State *dev, State *host) {
  MSX_HIP_TRY(hipMemcpyAsync(host, dev, sizeof(State), hipMemcpyDeviceToHost, s.stream));
  MSX_HIP_TRY(hipStreamSynchronize(s.stream));
  return MSX_OK;
}

// J: the Jacobi loop, inv_diag non-null (p_hat and s_hat in two more
// vectors; the SpMVs take them).
template <bool J>
msx_status bicgstab(const System &s, const float *b, const float *x0, const float *inv_diag,
                    float *x, float rtol, float atol, int64_t maxiter,
                    msx_solver_result *result) {
  const int64_t n = s.n;
  Scratch sc;
  sc.stream = s.stream;
  msx_status e = sc.alloc(n, J ? 9 : 7, 7);
  if (e != MSX_OK) return e;
  float *r = sc.vector(0), *r_hat = sc.vector(1), *p = sc.vector(2), *v = sc.vector(3),
        *sv = sc.vector(4), *tv = sc.vector(5), *ax = sc.vector(6);
  float *p_hat = J ? sc.vector(7) : p, *s_hat = J ? sc.vector(8) : sv;
  auto *st = static_cast<BiState *>(sc.state());
  double *start_part = sc.part(0), *p_part = sc.part(1), *v_part = sc.part(2),
         *s_part = sc.part(3), *t_part = sc.part(4), *r_part = sc.part(5),
         *chk_part = sc.part(6);
  const int np = s.nparts;
  BiState host{};

  hipLaunchKernelGGL(copy_vec, s.grid, s.block, 0, s.stream, x0, x, n);
  hipLaunchKernelGGL(zero_vec, s.grid, s.block, 0, s.stream, v, n);
  MSX_HIP_TRY(hipGetLastError());
  if ((e = spmv(s, x, ax)) != MSX_OK) return e;
  hipLaunchKernelGGL(bi_start, s.grid, s.block, 0, s.stream, b, x, ax, r, r_hat, n, start_part);
  hipLaunchKernelGGL(bi_decide_start<J>, dim3(1), s.block, 0, s.stream, start_part, np, rtol,
                     atol, maxiter, st);
  MSX_HIP_TRY(hipGetLastError());
  if ((e = read_state(s, st, &host)) != MSX_OK) return e;

  // the true residual b - A x into dst, then its check of kind `kind`
  auto true_check = [&](float *dst, int32_t kind) -> msx_status {
    msx_status es = spmv(s, x, ax);
    if (es != MSX_OK) return es;
    hipLaunchKernelGGL(bi_resid<J>, s.grid, s.block, 0, s.stream, b, ax, x, r_hat, dst, n,
                       chk_part);
    hipLaunchKernelGGL(bi_check<J>, dim3(1), s.block, 0, s.stream, chk_part, np, kind, st);
    MSX_HIP_TRY(hipGetLastError());
    return read_state(s, st, &host);
  };
  // the rest of iteration k after its s-check
  auto second_half = [&](int32_t k, int check) -> msx_status {
    msx_status es = spmv(s, s_hat, tv);
    if (es != MSX_OK) return es;
    hipLaunchKernelGGL(bi_t<J>, s.grid, s.block, 0, s.stream, sv, tv, n, k, check, s_part, t_part,
                       np, st);
    hipLaunchKernelGGL(bi_r<J>, s.grid, s.block, 0, s.stream, sv, tv, s_hat, x, r, r_hat, n, k,
                       t_part, r_part, np, st);
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  };

  int64_t next = 1;    // next iteration to launch
  int close_prev = 0;  // whether bi_p(next) closes iteration next - 1
  const double *dots = start_part;
  BatchSchedule schedule;  // its residual: the last iteration closed on the device
  int64_t batch = schedule.next(0, host.residual, host.tol);  // the start's state
  for (;;) {
    if (host.running) {
      const int64_t last = std::min(maxiter, next + batch - 1);
      for (int64_t k = next; k <= last; ++k) {
        const auto kk = static_cast<int32_t>(k);
        hipLaunchKernelGGL(bi_p<J>, s.grid, s.block, 0, s.stream, r, p, v, inv_diag, p_hat, n, kk,
                           close_prev, dots, p_part, np, st);
        MSX_HIP_TRY(hipGetLastError());
        if ((e = spmv(s, p_hat, v)) != MSX_OK) return e;
        hipLaunchKernelGGL(bi_v, s.grid, s.block, 0, s.stream, r_hat, v, n, kk, p_part, v_part,
                           np, st);
        hipLaunchKernelGGL(bi_s<J>, s.grid, s.block, 0, s.stream, r, v, p_hat, inv_diag, x, sv,
                           s_hat, n, kk, v_part, s_part, np, st);
        MSX_HIP_TRY(hipGetLastError());
        if ((e = second_half(kk, 1)) != MSX_OK) return e;
        close_prev = 1;
        dots = r_part;
      }
      if (last == maxiter)
        hipLaunchKernelGGL(bi_finish, dim3(1), s.block, 0, s.stream, r_part, np,
                           static_cast<int32_t>(last), st);
      MSX_HIP_TRY(hipGetLastError());
      if ((e = read_state(s, st, &host)) != MSX_OK) return e;
      next = last + 1;
      batch = schedule.next(last, host.residual, host.tol);
      continue;
    }
    if (host.pause == kNoPause) break;
    // a paused check: the true residual decides (the reference's branches)
    const int32_t k = host.pause_it;
    batch = 1;
    if (host.pause == kSCheck) {
      // the reference writes this residual to a scratch vector (its A x)
      if ((e = true_check(tv, kSCheck)) != MSX_OK) return e;
      if (!host.running) break;
      if ((e = second_half(k, 0)) != MSX_OK) return e;
      if (k == maxiter) hipLaunchKernelGGL(bi_finish, dim3(1), s.block, 0, s.stream, r_part, np, k, st);
      MSX_HIP_TRY(hipGetLastError());
      if ((e = read_state(s, st, &host)) != MSX_OK) return e;
      next = k + 1;
      close_prev = 1;
      dots = r_part;
    } else {
      // the true residual replaces r
      if ((e = true_check(r, kRCheck)) != MSX_OK) return e;
      if (!host.running || k == maxiter) break;  // k == maxiter: the budget ends here
      next = k + 1;
      close_prev = 0;  // the check's own sums give rho and r.r of the new r
      dots = chk_part;
    }
  }
  // the budget ran out or a breakdown: the reference's final true-residual check
  if (host.status > 0 || host.status == -1) {
    if ((e = true_check(r, 3)) != MSX_OK) return e;
  }
  if ((e = read_state(s, st, &host)) != MSX_OK) return e;
  *result = {host.status, host.completed, host.residual, 0};
  return MSX_OK;
}

// J: the Jacobi loop, inv_diag non-null (y = M r2 in one more vector).
template <bool J>
msx_status minres(const System &s, const float *b, const float *x0, const float *inv_diag,
                  float *x, float rtol, float atol, int64_t maxiter, float shift,
                  msx_solver_result *result) {
  const int64_t n = s.n;
  Scratch sc;
  sc.stream = s.stream;
  msx_status e = sc.alloc(n, J ? 8 : 7, J ? 6 : 5);
  if (e != MSX_OK) return e;
  float *r1 = sc.vector(0), *r2 = sc.vector(1), *av = sc.vector(2), *v = sc.vector(3),
        *w = sc.vector(4), *w2 = sc.vector(5), *q = sc.vector(6);
  float *y = J ? sc.vector(7) : nullptr;
  auto *st = static_cast<MrState *>(sc.state());
  double *start_part = sc.part(0), *a_part = sc.part(1), *b_part = sc.part(2),
         *x_part = sc.part(3), *res_part = sc.part(4);
  double *diag_part = J ? sc.part(5) : start_part;
  const int np = s.nparts;
  MrState host{};

  hipLaunchKernelGGL(copy_vec, s.grid, s.block, 0, s.stream, x0, x, n);
  for (float *z : {r1, w, w2}) hipLaunchKernelGGL(zero_vec, s.grid, s.block, 0, s.stream, z, n);
  MSX_HIP_TRY(hipGetLastError());
  if ((e = spmv(s, x, av)) != MSX_OK) return e;
  hipLaunchKernelGGL(mr_start<J>, s.grid, s.block, 0, s.stream, b, x, av, shift, inv_diag, r2, y,
                     n, start_part);
  if (J) hipLaunchKernelGGL(mr_diag_check, s.grid, s.block, 0, s.stream, inv_diag, n, diag_part);
  hipLaunchKernelGGL(mr_decide_start<J>, dim3(1), s.block, 0, s.stream, start_part, diag_part, np,
                     rtol, atol, maxiter, st);
  MSX_HIP_TRY(hipGetLastError());
  if ((e = read_state(s, st, &host)) != MSX_OK) return e;
  int64_t next = 1;
  BatchSchedule schedule;  // its residual: the last iteration tested on the device
  int64_t batch = schedule.next(0, host.residual, host.tol);  // the start's state
  while (host.running && next <= maxiter) {
    const int64_t last = std::min(maxiter, next + batch - 1);
    for (int64_t k = next; k <= last; ++k) {
      const auto kk = static_cast<int32_t>(k);
      hipLaunchKernelGGL(mr_v<J>, s.grid, s.block, 0, s.stream, J ? y : r2, v, n, kk, res_part,
                         np, st);
      MSX_HIP_TRY(hipGetLastError());
      if ((e = spmv(s, v, av)) != MSX_OK) return e;
      hipLaunchKernelGGL(mr_a, s.grid, s.block, 0, s.stream, v, av, r1, shift, n, kk, a_part, st);
      hipLaunchKernelGGL(mr_b<J>, s.grid, s.block, 0, s.stream, av, r2, inv_diag, y, n, kk, a_part,
                         b_part, np, st);
      hipLaunchKernelGGL(mr_x<J>, s.grid, s.block, 0, s.stream, v, w, w2, x, n, kk, a_part, b_part,
                         x_part, np, st);
      MSX_HIP_TRY(hipGetLastError());
      // the Lanczos vectors move on (r1 <- r2 <- av) and w2 <- w <- new w
      std::swap(r1, r2);
      std::swap(r2, av);
      std::swap(w, w2);
      if ((e = spmv(s, x, q)) != MSX_OK) return e;
      hipLaunchKernelGGL(mr_r, s.grid, s.block, 0, s.stream, b, x, q, shift, n, kk, x_part,
                         res_part, np, st);
      MSX_HIP_TRY(hipGetLastError());
    }
    if (last == maxiter)
      hipLaunchKernelGGL(mr_finish, dim3(1), s.block, 0, s.stream, res_part, np,
                         static_cast<int32_t>(last), st);
    MSX_HIP_TRY(hipGetLastError());
    if ((e = read_state(s, st, &host)) != MSX_OK) return e;
    next = last + 1;
    batch = schedule.next(last, host.residual, host.tol);
  }
  *result = {host.status, host.completed, host.residual, 0};
  return MSX_OK;
}

msx_status check(const char *op, msx_itype it, int64_t n, int64_t nnz, const void *data,
                 const void *indices, const void *indptr, const void *b, const void *x0, void *x,
                 int64_t maxiter, msx_solver_result *result) {
  if (!valid_itype(it)) return fail(MSX_ETYPE, std::string(op) + " requires int32 or int64 indices.");
  if (n <= 0 || n >= 2147483647)
    return fail(MSX_EINVAL, std::string(op) + " requires a non-empty square matrix.");
  if (maxiter < 0) return fail(MSX_EINVAL, std::string(op) + " maxiter must be non-negative.");
  if (maxiter > 2147483647) return fail(MSX_EINVAL, std::string(op) + " maxiter must fit in int32.");
  if (nnz < 0 || nnz >= 2147483647)
    return fail(MSX_EINVAL, std::string(op) + " supports at most 2^31 - 2 stored values.");
  if (indptr == nullptr || b == nullptr || x0 == nullptr || x == nullptr || result == nullptr ||
      (nnz > 0 && (data == nullptr || indices == nullptr)))
    return fail(MSX_EINVAL, std::string(op) + " buffers must be non-NULL.");
  return MSX_OK;
}

}  // namespace
}  // namespace msx

using namespace msx;

extern "C" msx_status msx_csr_bicgstab(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                       const void *indices, const void *indptr, const float *b,
                                       const float *x0, float *x, float rtol, float atol,
                                       int64_t maxiter, const msx_csr_plan *plan,
                                       msx_solver_result *result, void *stream) {
  clear_error();
  msx_status st = check("csr_bicgstab", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  st = check_plan("csr_bicgstab", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const uint32_t blocks = blocks_for(n);
  const System s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                 dim3(blocks), dim3(kSolverThreads), static_cast<int>(blocks)};
  return bicgstab<false>(s, b, x0, nullptr, x, rtol, atol, maxiter, result);
}

extern "C" msx_status msx_csr_bicgstab_jacobi(msx_itype it, int64_t n, int64_t nnz,
                                              const float *data, const void *indices,
                                              const void *indptr, const float *b,
                                              const float *x0, const float *inv_diag, float *x,
                                              float rtol, float atol, int64_t maxiter,
                                              const msx_csr_plan *plan, msx_solver_result *result,
                                              void *stream) {
  clear_error();
  msx_status st =
      check("csr_bicgstab_jacobi", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  if (inv_diag == nullptr)
    return fail(MSX_EINVAL, "csr_bicgstab_jacobi buffers must be non-NULL.");
  st = check_plan("csr_bicgstab_jacobi", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const uint32_t blocks = blocks_for(n);
  const System s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                 dim3(blocks), dim3(kSolverThreads), static_cast<int>(blocks)};
  return bicgstab<true>(s, b, x0, inv_diag, x, rtol, atol, maxiter, result);
}

extern "C" msx_status msx_csr_minres(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                     const void *indices, const void *indptr, const float *b,
                                     const float *x0, float *x, float rtol, float atol,
                                     int64_t maxiter, float shift, const msx_csr_plan *plan,
                                     msx_solver_result *result, void *stream) {
  clear_error();
  msx_status st = check("csr_minres", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  st = check_plan("csr_minres", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const uint32_t blocks = blocks_for(n);
  const System s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                 dim3(blocks), dim3(kSolverThreads), static_cast<int>(blocks)};
  return minres<false>(s, b, x0, nullptr, x, rtol, atol, maxiter, shift, result);
}

extern "C" msx_status msx_csr_minres_jacobi(msx_itype it, int64_t n, int64_t nnz,
                                            const float *data, const void *indices,
                                            const void *indptr, const float *b, const float *x0,
                                            const float *inv_diag, float *x, float rtol,
                                            float atol, int64_t maxiter, float shift,
                                            const msx_csr_plan *plan, msx_solver_result *result,
                                            void *stream) {
  clear_error();
  msx_status st =
      check("csr_minres_jacobi", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  if (inv_diag == nullptr) return fail(MSX_EINVAL, "csr_minres_jacobi buffers must be non-NULL.");
  st = check_plan("csr_minres_jacobi", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const uint32_t blocks = blocks_for(n);
  const System s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                 dim3(blocks), dim3(kSolverThreads), static_cast<int>(blocks)};
  return minres<true>(s, b, x0, inv_diag, x, rtol, atol, maxiter, shift, result);
}
