// csr_gmres.hip - restarted GMRES on a square float32 CSR matrix, the
// Arnoldi factorisation on the device.
//
// The reference runs the restart loop on the host around a GPU Arnoldi
// kernel of one 256-thread threadgroup (reference:
// src/linalg/gmres/gmres.cpp:58-220, src/linalg/arnoldi/arnoldi.cpp:184-225,
// arnoldi.metal).  Here every Arnoldi step is device-wide: the path's SpMV
// with the matrix's plan, then modified Gram-Schmidt with two sweeps over
// the basis, as the reference's CPU Arnoldi (arnoldi.cpp:118-146), two
// projections per pass over w: a pass subtracts the previous pair's
// projections from w and forms the dot products of the next pair's columns
// with w and with each other, from which the second coefficient of the pair
// is the sequential one in exact arithmetic (gm_pair).  Every workgroup
// adds the previous pass's double partials in the same order (msx_solver.h),
// so all of them subtract the same float coefficients.
//
// Per cycle (the host loop of gmres.cpp:86-207):
//   gm_resid   r = b - A x; r.r, its non-finite count, b.b, non-finite b, x
//   (host)     beta = ||r||: stop (converged / non-finite) or go on
//   gm_v0norm  (r / beta).(r / beta)
//   gm_start   V0 = (r / beta) / ||r / beta|| (e0 when that norm <= eps);
//              clears h and the cycle state
//   step j:    w = A V_j; gm_pair m = 0 .. j + 1; gm_norm
//              (h[j+1][j] = ||w||; V_{j+1} = w / ||w|| unless ||w|| <= eps,
//              which ends the cycle's steps: later passes return at once)
//   (host)     reads h and the steps taken, solves the (used + 1) x used
//              least-squares problem in double (msx_hessenberg.h)
//   gm_update  x' = x + V y, each row's update a double sum in column
//              order; the first non-finite row is recorded
//   then the next cycle's gm_resid runs on x' (one host read per cycle
//   covers the residual and that record).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>
#include <limits>
#include <string>
#include <utility>
#include <vector>

#include "msx_device.h"
#include "msx_hessenberg.h"
#include "msx_internal.h"
#include "msx_solver.h"
#include "msx_sparse.h"

namespace msx {
namespace {

using namespace solver;

constexpr float kEpsF = FLT_EPSILON;

struct GmState {
  int32_t stop_at;  // the step whose ||w|| <= eps ended the cycle (INT_MAX: none)
  int32_t used;     // Arnoldi steps taken in this cycle
  unsigned long long bad;  // first non-finite row of the update: 2 row + kind (~0: none)
};

__device__ inline bool lead() { return blockIdx.x == 0 && threadIdx.x == 0; }

// r = b - A x.  Slots: r.r, non-finite r count, b.b, non-finite b or x count.
// J (the Jacobi loop, preconditioners/gmres/gmres.cpp:572-748): also
// z = inv_diag r; slot 2 holds z.z instead (a double sum of float squares:
// non-finite exactly when some z is) and slot 3 also counts inv_diag.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    gm_resid(const float *__restrict__ b, const float *__restrict__ x,
             const float *__restrict__ ax, const float *__restrict__ inv_diag,
             float *__restrict__ r, float *__restrict__ z, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const float bi = b[i], xi = x[i];
    const float ri = bi - ax[i];
    r[i] = ri;
    v[0] += static_cast<double>(ri) * static_cast<double>(ri);
    if constexpr (J) {
      const float di = inv_diag[i];
      const float zi = di * ri;
      z[i] = zi;
      if (!fin(ri)) v[1] += 1.0;
      v[2] += static_cast<double>(zi) * static_cast<double>(zi);
      if (!(fin(bi) && fin(xi) && fin(di))) v[3] += 1.0;
    } else {
      if (!fin(ri)) v[1] += 1.0;
      v[2] += static_cast<double>(bi) * static_cast<double>(bi);
      if (!(fin(bi) && fin(xi))) v[3] += 1.0;
    }
  })
  write_partials(v, part);
}

// Slot 0: v.v (the Jacobi loop's ||b||).
__global__ void __launch_bounds__(kSolverThreads)
    gm_sumsq(const float *__restrict__ vec, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({ v[0] += static_cast<double>(vec[i]) * static_cast<double>(vec[i]); })
  write_partials(v, part);
}

// The totals of a pass's partials, for the host.
__global__ void __launch_bounds__(kSolverThreads)
    gm_totals(const double *part, int nparts, double *out) {
  double t[kSlots];
  read_totals(part, nparts, t);
  if (threadIdx.x < kSlots) out[threadIdx.x] = t[threadIdx.x];
}

// (r / beta).(r / beta): the norm the reference's Arnoldi takes of its start
// vector (arnoldi.cpp:104-109); slot 1 counts its non-finite entries.
__global__ void __launch_bounds__(kSolverThreads)
    gm_v0norm(const float *__restrict__ r, float beta, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const float vi = r[i] / beta;
    v[0] += static_cast<double>(vi) * static_cast<double>(vi);
    if (!fin(vi)) v[1] += 1.0;
  })
  write_partials(v, part);
}

// V0 and a fresh cycle: h (hn floats) cleared, state reset.  J: a start
// vector with a non-finite entry or norm takes no step (the Jacobi
// Arnoldi's input test, gmres.cpp:382-391 there): every step returns at
// once and the cycle reports zero steps.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    gm_start(const float *__restrict__ r, float beta, const double *part, int nparts,
             float *__restrict__ v0, int64_t n, float *__restrict__ h, int64_t hn, GmState *st) {
  double t[kSlots];
  read_totals(part, nparts, t);
  const float v_norm = static_cast<float>(sqrt(max0(t[0])));
  const bool unit = v_norm <= kEpsF;
  const bool no_steps = J && (t[1] != 0.0 || !fin(v_norm));
  MSX_SOLVER_LOOP({
    const float vi = r[i] / beta;
    v0[i] = unit ? (i == 0 ? 1.0f : 0.0f) : vi / v_norm;
  })
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kSolverThreads + threadIdx.x; i < hn;
       i += static_cast<int64_t>(gridDim.x) * kSolverThreads)
    h[i] = 0.0f;
  if (lead()) {
    st->stop_at = no_steps ? -1 : INT_MAX;
    st->used = 0;
    st->bad = ~0ull;
  }
}

// Gram-Schmidt pass m of Arnoldi step j (ncol = j + 1 columns).  The two
// sweeps project w onto the columns in the order 0..j, 0..j; pass m takes
// the pair of projections 2m and 2m + 1 of that list (columns a = 2m % ncol
// and b = (2m + 1) % ncol) and the last pass (m = ncol) takes w.w.
//   - m > 0: the previous pair's coefficients come from the previous
//     pass's totals: c_a = d_a rounded to float, c_b = (d_b - c_a g)
//     rounded to float, where d_a = w.q_a, d_b = w.q_b and g = q_a.q_b
//     were summed before either projection left w - the value of
//     (w - c_a q_a).q_b in exact arithmetic, so one pass does the work of
//     two sequential ones; both go into h and leave w in the sequential
//     order (w = w - c_a q_a, then w = w - c_b q_b, float operations);
//   - then d_a, d_b and g of this pair (double sums of float products).
// The previous pass's partials, then a thread's first kUnroll elements of
// every stream, are loaded before the partials are reduced, so that the
// reduction (its wave sums and barriers) overlaps the element loads.  J:
// pass 0 first scales w = A v_j by inv_diag in float (the Jacobi Arnoldi's
// w = M A q, gmres.cpp:413-415 there) and writes it back.
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    gm_pair(const float *__restrict__ V, int64_t ld, float *__restrict__ w,
            const float *__restrict__ inv_diag, int64_t n, int32_t j, int32_t m,
            const double *part_in, int nparts, double *part_out, float *__restrict__ h, int64_t k,
            const GmState *st) {
  if (st->stop_at < j) return;  // an earlier step ended this cycle
  const int32_t ncol = j + 1;
  const bool sub = m > 0, norm = m == ncol;
  const int64_t pa = sub ? (2 * m - 2) % ncol : 0, pb = sub ? (2 * m - 1) % ncol : 0;
  const int64_t qa = norm ? 0 : (2 * m) % ncol, qb = norm ? 0 : (2 * m + 1) % ncol;
  // pass 0 subtracts nothing: with J its first projection stream is inv_diag
  const float *ua = (J && !sub) ? inv_diag : V + pa * ld;
  const float *ub = V + pb * ld;
  const float *va = V + qa * ld;
  const float *vb = V + qb * ld;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kSolverThreads;
  const int64_t base0 = static_cast<int64_t>(blockIdx.x) * kSolverThreads + threadIdx.x;
  double pv_in[kSlots] = {0.0, 0.0, 0.0, 0.0};
  if (sub) load_partials(part_in, nparts, pv_in);
  float w0[kUnroll], a0[kUnroll], b0[kUnroll], x0[kUnroll], y0[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base0 + u * stride < n ? base0 + u * stride : (base0 < n ? base0 : 0);
    w0[u] = w[i];
    a0[u] = (sub || J) ? ua[i] : 0.0f;
    b0[u] = sub ? ub[i] : 0.0f;
    x0[u] = norm ? 0.0f : va[i];
    y0[u] = norm ? 0.0f : vb[i];
  }
  float ca = 0.0f, cb = 0.0f;
  if (sub) {
    double t[kSlots];
    reduce_partials(pv_in, nparts, t);
    ca = static_cast<float>(t[0]);
    cb = static_cast<float>(t[1] - static_cast<double>(ca) * t[2]);
    if (lead()) {
      h[pa * k + j] += ca;
      h[pb * k + j] += cb;
    }
  }
  double acc0 = 0.0, acc1 = 0.0, acc2 = 0.0;
  auto one = [&](int64_t i, float wv, float av, float bv, float xv, float yv) {
    if (sub) {
      const float ta = ca * av;
      wv = wv - ta;
      const float tb = cb * bv;
      wv = wv - tb;
      w[i] = wv;
    } else if (J) {
      wv = wv * av;
      w[i] = wv;
    }
    if (norm) {
      acc0 += static_cast<double>(wv) * static_cast<double>(wv);
    } else {
      const float pa_ = xv * wv, pb_ = yv * wv, g = xv * yv;
      acc0 += static_cast<double>(pa_);
      acc1 += static_cast<double>(pb_);
      acc2 += static_cast<double>(g);
    }
  };
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    if (base0 + u * stride < n) one(base0 + u * stride, w0[u], a0[u], b0[u], x0[u], y0[u]);
  for (int64_t base = base0 + kUnroll * stride; base < n; base += kUnroll * stride) {
    float wv[kUnroll], av[kUnroll], bv[kUnroll], xv[kUnroll], yv[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * stride < n ? base + u * stride : base;
      wv[u] = w[i];
      av[u] = (sub || J) ? ua[i] : 0.0f;
      bv[u] = sub ? ub[i] : 0.0f;
      xv[u] = norm ? 0.0f : va[i];
      yv[u] = norm ? 0.0f : vb[i];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (base + u * stride < n) one(base + u * stride, wv[u], av[u], bv[u], xv[u], yv[u]);
  }
  double v[kSlots] = {acc0, acc1, acc2, 0.0};
  write_partials(v, part_out);
}

// h[j+1][j] = ||w|| (norm_float); the next basis vector w / ||w||, or the
// end of the cycle's steps when ||w|| <= eps.  J: a non-finite ||w|| ends
// the cycle with no steps (gmres.cpp:437-440 there).
template <bool J>
__global__ void __launch_bounds__(kSolverThreads)
    gm_norm(const float *__restrict__ w, float *__restrict__ next, int64_t n, int32_t j,
            const double *part, int nparts, float *__restrict__ h, int64_t k, GmState *st) {
  if (st->stop_at < j) return;  // stop_at is only ever set to this step's j below
  double t[kSlots];
  read_totals(part, nparts, t);
  const float ww = static_cast<float>(t[0]);
  const float h_next = sqrtf(max0(ww));
  const bool lost = J && !fin(h_next);
  if (lead()) {
    h[static_cast<int64_t>(j + 1) * k + j] = h_next;
    st->used = lost ? 0 : j + 1;
    if (lost || h_next <= kEpsF) st->stop_at = j;
  }
  if (lost || h_next <= kEpsF) return;
  MSX_SOLVER_LOOP({ next[i] = w[i] / h_next; })
}

// x_out = x_in + V y: each row's update sum_c V_c[i] y[c] in double, column
// order; a row whose update or new value is not finite is recorded (2 row
// for the update, 2 row + 1 for the value) and keeps x_in when the update
// itself is not finite, as the reference stops before that row's add.
__global__ void __launch_bounds__(kSolverThreads)
    gm_update(const float *__restrict__ V, int64_t ld, int32_t used, const double *__restrict__ y,
              const float *__restrict__ x_in, float *__restrict__ x_out, int64_t n, GmState *st) {
  unsigned long long bad = ~0ull;
  MSX_SOLVER_LOOP({
    double u = 0.0;
    for (int32_t c = 0; c < used; ++c)
      u += static_cast<double>(V[static_cast<int64_t>(c) * ld + i]) * y[c];
    const float xi = x_in[i];
    float xo = xi;
    if (!isfinite(u)) {
      bad = std::min(bad, 2ull * static_cast<unsigned long long>(i));
    } else {
      xo = xi + static_cast<float>(u);
      if (!fin(xo)) bad = std::min(bad, 2ull * static_cast<unsigned long long>(i) + 1ull);
    }
    x_out[i] = xo;
  })
  if (bad != ~0ull) atomicMin(&st->bad, bad);
}

// After a non-finite update at row `first` (2 row + kind): the rows after it
// keep x_in, as the reference's loop stopped there.
__global__ void __launch_bounds__(kSolverThreads)
    gm_fix(const float *__restrict__ x_in, float *__restrict__ x_out, int64_t n, int64_t first) {
  MSX_SOLVER_LOOP({
    if (i > first) x_out[i] = x_in[i];
  })
}

__global__ void __launch_bounds__(kSolverThreads)
    gm_copy(const float *__restrict__ src, float *__restrict__ dst, int64_t n) {
  MSX_SOLVER_LOOP({ dst[i] = src[i]; })
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

// Device scratch (stream-ordered): the basis (kcap + 1 vectors), w, A x,
// r, two x buffers, h, y, the state, totals and three partial arrays.
struct Scratch {
  char *base = nullptr;
  hipStream_t stream = nullptr;
  ~Scratch() {
    if (base) (void)hipFreeAsync(base, stream);
  }
};

float norm_of(double total) {
  const float f = static_cast<float>(total);
  return std::sqrt(f < 0.0f ? 0.0f : f);
}

// J: the Jacobi loop, inv_diag non-null (z = M r in one more vector).
template <bool J>
msx_status gmres(const System &s, const float *b, const float *x0, const float *inv_diag,
                 float *x, float rtol, float atol, int64_t restart, int64_t maxiter,
                 msx_solver_result *result) {
  const int64_t n = s.n;
  const int64_t kcap = std::max<int64_t>(1, std::min({restart, maxiter, n}));
  const size_t vec = (static_cast<size_t>(n) * sizeof(float) + 255) / 256 * 256;
  const int64_t ld = static_cast<int64_t>(vec / sizeof(float));
  const size_t hbytes = (static_cast<size_t>((kcap + 1) * kcap) * sizeof(float) + 255) / 256 * 256;
  const size_t ybytes = (static_cast<size_t>(kcap) * sizeof(double) + 255) / 256 * 256;
  const size_t part_bytes = sizeof(double) * kSlots * kSolverMaxBlocks;
  const size_t nvec = static_cast<size_t>(kcap + 1) + (J ? 6 : 5);
  Scratch sc;
  sc.stream = s.stream;
  MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&sc.base),
                             nvec * vec + hbytes + ybytes + 256 + 256 + 3 * part_bytes, s.stream));
  char *p = sc.base;
  float *V = reinterpret_cast<float *>(p);
  p += static_cast<size_t>(kcap + 1) * vec;
  float *w = reinterpret_cast<float *>(p);
  float *ax = reinterpret_cast<float *>(p + vec);
  float *r = reinterpret_cast<float *>(p + 2 * vec);
  float *xa = reinterpret_cast<float *>(p + 3 * vec);
  float *xb = reinterpret_cast<float *>(p + 4 * vec);
  float *z = J ? reinterpret_cast<float *>(p + 5 * vec) : r;
  p += (J ? 6 : 5) * vec;
  float *h = reinterpret_cast<float *>(p);
  p += hbytes;
  double *y_dev = reinterpret_cast<double *>(p);
  p += ybytes;
  auto *st = reinterpret_cast<GmState *>(p);
  double *tot = reinterpret_cast<double *>(p + 256);
  p += 512;
  double *part[3] = {reinterpret_cast<double *>(p), reinterpret_cast<double *>(p + part_bytes),
                     reinterpret_cast<double *>(p + 2 * part_bytes)};
  const int np = s.nparts;
  msx_status e;
  auto spmv = [&](const float *in, float *out) {
    return launch_spmv(MSX_F32, s.it, n, n, s.nnz, s.data, s.indices, s.indptr, in, out, s.plan,
                       s.stream);
  };
  struct Host {
    double tot[kSlots];
    GmState st;
  } host{};
  // r = b - A x and its totals (plus the state) on the host
  auto residual = [&](const float *xv) -> msx_status {
    msx_status es = spmv(xv, ax);
    if (es != MSX_OK) return es;
    hipLaunchKernelGGL(gm_resid<J>, s.grid, s.block, 0, s.stream, b, xv, ax, inv_diag, r, z, n,
                       part[2]);
    hipLaunchKernelGGL(gm_totals, dim3(1), s.block, 0, s.stream, part[2], np, tot);
    MSX_HIP_TRY(hipGetLastError());
    MSX_HIP_TRY(hipMemcpyAsync(host.tot, tot, sizeof(host.tot), hipMemcpyDeviceToHost, s.stream));
    MSX_HIP_TRY(hipMemcpyAsync(&host.st, st, sizeof(GmState), hipMemcpyDeviceToHost, s.stream));
    MSX_HIP_TRY(hipStreamSynchronize(s.stream));
    return MSX_OK;
  };

  hipLaunchKernelGGL(gm_copy, s.grid, s.block, 0, s.stream, x0, xa, n);
  MSX_HIP_TRY(hipGetLastError());
  double bb = 0.0;  // J: ||b||^2 from its own pass (gm_resid's slot 2 holds z.z)
  if (J) {
    hipLaunchKernelGGL(gm_sumsq, s.grid, s.block, 0, s.stream, b, n, part[1]);
    hipLaunchKernelGGL(gm_totals, dim3(1), s.block, 0, s.stream, part[1], np, tot);
    MSX_HIP_TRY(hipGetLastError());
    MSX_HIP_TRY(hipMemcpyAsync(&bb, tot, sizeof(double), hipMemcpyDeviceToHost, s.stream));
  }
  if ((e = residual(xa)) != MSX_OK) return e;
  const float b_norm = norm_of(J ? bb : host.tot[2]);
  const float scaled = rtol * b_norm;
  const float tol = atol > scaled ? atol : scaled;
  int64_t iters = 0;
  int32_t status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
  float res = std::numeric_limits<float>::infinity();
  const auto finish = [&]() -> msx_status {
    hipLaunchKernelGGL(gm_copy, s.grid, s.block, 0, s.stream, xa, x, n);
    MSX_HIP_TRY(hipGetLastError());
    MSX_HIP_TRY(hipStreamSynchronize(s.stream));
    *result = {status, static_cast<int32_t>(iters), res, 0};
    return MSX_OK;
  };
  if (host.tot[3] != 0.0 || !std::isfinite(b_norm) || !std::isfinite(tol)) {
    status = -3;
    return finish();
  }
  std::vector<float> hh(static_cast<size_t>((kcap + 1) * kcap));
  std::vector<double> y;
  // host.tot holds the residual of the current x (xa) at the top of the loop
  while (iters < maxiter) {
    float beta = norm_of(host.tot[0]);
    res = beta;
    if (host.tot[1] != 0.0 || !std::isfinite(res) || (J && !std::isfinite(host.tot[2]))) {
      status = -3;
      break;
    }
    if (res <= tol) {
      status = 0;
      break;
    }
    if (J) {  // the cycle starts from z = M r (gmres.cpp:632-637 there)
      beta = norm_of(host.tot[2]);
      if (!std::isfinite(beta) || beta <= kEpsF) {
        status = -1;
        break;
      }
    }
    const int64_t steps = std::min({restart, maxiter - iters, n});
    hipLaunchKernelGGL(gm_v0norm, s.grid, s.block, 0, s.stream, z, beta, n, part[2]);
    hipLaunchKernelGGL(gm_start<J>, s.grid, s.block, 0, s.stream, z, beta, part[2], np, V, n, h,
                       (steps + 1) * steps, st);
    MSX_HIP_TRY(hipGetLastError());
    for (int64_t j = 0; j < steps; ++j) {
      if ((e = spmv(V + j * ld, w)) != MSX_OK) return e;
      const auto jj = static_cast<int32_t>(j);
      int cur = 0;
      for (int32_t pass = 0; pass <= jj + 1; ++pass) {
        hipLaunchKernelGGL(gm_pair<J>, s.grid, s.block, 0, s.stream, V, ld, w, inv_diag, n, jj,
                           pass, part[cur ^ 1], np, part[cur], h, steps, st);
        cur ^= 1;
      }
      hipLaunchKernelGGL(gm_norm<J>, s.grid, s.block, 0, s.stream, w, V + (j + 1) * ld, n, jj,
                         part[cur ^ 1], np, h, steps, st);
      MSX_HIP_TRY(hipGetLastError());
    }
    MSX_HIP_TRY(hipMemcpyAsync(hh.data(), h, sizeof(float) * static_cast<size_t>((steps + 1) * steps),
                               hipMemcpyDeviceToHost, s.stream));
    MSX_HIP_TRY(hipMemcpyAsync(&host.st, st, sizeof(GmState), hipMemcpyDeviceToHost, s.stream));
    MSX_HIP_TRY(hipStreamSynchronize(s.stream));
    const int64_t used = host.st.used;
    if (used == 0) {
      status = -1;
      break;
    }
    std::vector<double> hu(static_cast<size_t>((used + 1) * used));
    bool bad = false;
    for (int64_t row = 0; row <= used; ++row)
      for (int64_t col = 0; col < used; ++col) {
        hu[row * used + col] = static_cast<double>(hh[row * steps + col]);
        bad = bad || !std::isfinite(hu[row * used + col]);
      }
    if (bad) {
      status = -3;
      break;
    }
    std::vector<double> e1(static_cast<size_t>(used + 1), 0.0);
    e1[0] = static_cast<double>(beta);
    if (!hessenberg_least_squares(std::move(hu), std::move(e1), used, y)) {
      status = -1;
      break;
    }
    if (!J)  // the Jacobi loop tests only each row's update (gmres.cpp:693-707 there)
      for (double v : y) bad = bad || !std::isfinite(v);
    if (bad) {
      status = -3;
      break;
    }
    MSX_HIP_TRY(hipMemcpyAsync(y_dev, y.data(), sizeof(double) * static_cast<size_t>(used),
                               hipMemcpyHostToDevice, s.stream));
    hipLaunchKernelGGL(gm_update, s.grid, s.block, 0, s.stream, V, ld,
                       static_cast<int32_t>(used), y_dev, xa, xb, n, st);
    MSX_HIP_TRY(hipGetLastError());
    // the next cycle's residual (or the final one) on the new x; the same
    // read reports a non-finite update
    if ((e = residual(xb)) != MSX_OK) return e;
    if (host.st.bad != ~0ull) {
      hipLaunchKernelGGL(gm_fix, s.grid, s.block, 0, s.stream, xa, xb, n,
                         static_cast<int64_t>(host.st.bad / 2));
      MSX_HIP_TRY(hipGetLastError());
      std::swap(xa, xb);
      status = -3;
      break;
    }
    std::swap(xa, xb);
    iters += used;
    if (iters >= maxiter) {
      res = norm_of(host.tot[0]);
      if (host.tot[1] != 0.0 || !std::isfinite(res)) status = -3;
      else if (res <= tol) status = 0;
      break;
    }
  }
  if (maxiter == 0 && status > 0) {
    res = norm_of(host.tot[0]);
    if (host.tot[1] != 0.0 || !std::isfinite(res)) status = -3;
    else if (res <= tol) status = 0;
  }
  return finish();
}

}  // namespace
}  // namespace msx

using namespace msx;

extern "C" msx_status msx_csr_gmres(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                    const void *indices, const void *indptr, const float *b,
                                    const float *x0, float *x, float rtol, float atol,
                                    int64_t restart, int64_t maxiter, const msx_csr_plan *plan,
                                    msx_solver_result *result, void *stream) {
  clear_error();
  if (!valid_itype(it)) return fail(MSX_ETYPE, "csr_gmres requires int32 or int64 indices.");
  if (n <= 0 || n >= 2147483647) return fail(MSX_EINVAL, "csr_gmres requires a non-empty square matrix.");
  if (restart <= 0 || maxiter < 0)
    return fail(MSX_EINVAL, "csr_gmres requires restart > 0 and maxiter >= 0.");
  if (maxiter > 2147483647) return fail(MSX_EINVAL, "csr_gmres maxiter must fit in int32.");
  if (nnz < 0 || nnz >= 2147483647)
    return fail(MSX_EINVAL, "csr_gmres supports at most 2^31 - 2 stored values.");
  if (indptr == nullptr || b == nullptr || x0 == nullptr || x == nullptr || result == nullptr ||
      (nnz > 0 && (data == nullptr || indices == nullptr)))
    return fail(MSX_EINVAL, "csr_gmres buffers must be non-NULL.");
  const msx_status st = check_plan("csr_gmres", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const uint32_t blocks = blocks_for(n);
  const System s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                 dim3(blocks), dim3(kSolverThreads), static_cast<int>(blocks)};
  return gmres<false>(s, b, x0, nullptr, x, rtol, atol, restart, maxiter, result);
}

extern "C" msx_status msx_csr_gmres_jacobi(msx_itype it, int64_t n, int64_t nnz,
                                           const float *data, const void *indices,
                                           const void *indptr, const float *b, const float *x0,
                                           const float *inv_diag, float *x, float rtol,
                                           float atol, int64_t restart, int64_t maxiter,
                                           const msx_csr_plan *plan, msx_solver_result *result,
                                           void *stream) {
  clear_error();
  if (!valid_itype(it)) return fail(MSX_ETYPE, "csr_gmres_jacobi requires int32 or int64 indices.");
  if (n <= 0 || n >= 2147483647)
    return fail(MSX_EINVAL, "csr_gmres_jacobi requires a non-empty square matrix.");
  if (restart <= 0 || maxiter < 0)
    return fail(MSX_EINVAL, "csr_gmres_jacobi requires restart > 0 and maxiter >= 0.");
  if (maxiter > 2147483647) return fail(MSX_EINVAL, "csr_gmres_jacobi maxiter must fit in int32.");
  if (nnz < 0 || nnz >= 2147483647)
    return fail(MSX_EINVAL, "csr_gmres_jacobi supports at most 2^31 - 2 stored values.");
  if (indptr == nullptr || b == nullptr || x0 == nullptr || x == nullptr || result == nullptr ||
      inv_diag == nullptr || (nnz > 0 && (data == nullptr || indices == nullptr)))
    return fail(MSX_EINVAL, "csr_gmres_jacobi buffers must be non-NULL.");
  const msx_status st =
      check_plan("csr_gmres_jacobi", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const uint32_t blocks = blocks_for(n);
  const System s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                 dim3(blocks), dim3(kSolverThreads), static_cast<int>(blocks)};
  return gmres<true>(s, b, x0, inv_diag, x, rtol, atol, restart, maxiter, result);
}
