// csr_cg.hip - conjugate gradients (plain and Jacobi-preconditioned) on a
// square float32 CSR matrix, with the loop resident on the device.
//
// The reference runs its GPU solvers in one 256-thread threadgroup
// (reference: src/linalg/cg/cg.metal, kSolverThreads in
// src/linalg/common/common.h:33).  Here every step is device-wide:
//
//   ap = A p              the path's SpMV with the matrix's plan (panels,
//                         slices or row blocks; no plan: the row-group kernel)
//   cg_alpha / pcg_alpha  p.ap, p.p, ap.ap and non-finite counts in one pass
//   cg_update / pcg_update  alpha or the breakdown status from those sums,
//                         then x += alpha p, r -= alpha ap (z = inv_diag r)
//                         and r.r (r.z) in one pass
//   cg_direction          convergence and beta from those sums, then
//                         p = r + beta p (z + beta p)
//
// Scalars live in a device state block; kernels return at once when the
// solve has stopped, so the host enqueues iterations in batches and reads the
// state between batches only.  Sums: each workgroup reduces its grid-stride
// share in double and writes it out; every workgroup of the NEXT pass adds
// those partials in workgroup order and takes the same scalar decision, so
// no workgroup waits on another inside a kernel (a device-scope fence costs
// an L2 write-back and invalidate on this multi-XCD part) and a solve is
// reproducible run to run.  The scalar
// rules (tolerance, breakdown tests, status codes) follow the reference's CPU
// loops: src/linalg/cg/cg.cpp:75-246 (csr_cg_cpu_impl) and
// src/preconditioners/pcg/pcg.cpp:71-236 (csr_pcg_jacobi_cpu_impl).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cfloat>
#include <string>

#include "msx_device.h"
#include "msx_internal.h"
#include "msx_solver.h"
#include "msx_sparse.h"

namespace msx {
namespace {

using namespace solver;  // slot 3 of every pass counts non-finite values

struct CgState {
  double rr;       // CG: r.r of the current residual; PCG: rho = r.z (a float)
  double rr_next;  // value of rr for the next iteration, committed by the next alpha pass
  double true_rr;  // PCG: float r.r of the current residual
  float tol;
  int32_t status;     // reference status: 0, maxiter, -1, -2, -3
  int32_t completed;  // completed iterations
  int32_t running;    // 1 while iterating
};

__device__ inline void stop(CgState *st, int32_t status, int32_t completed) {
  st->status = status;
  st->completed = completed;
  st->running = 0;
}

// ---------------------------------------------------------------------------
// Plain CG (cg.cpp:75-246).  Passes: start -> [SpMV, alpha, update,
// direction] x it -> finish.  alpha consumes the previous direction pass,
// update the alpha pass, direction the update pass.

__global__ void __launch_bounds__(kSolverThreads)
    cg_start(const float *__restrict__ b, const float *__restrict__ x, const float *__restrict__ ap,
             float *__restrict__ r, float *__restrict__ p, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const float ri = b[i] - ap[i];
    r[i] = ri;
    p[i] = ri;
    v[0] += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    v[1] += static_cast<double>(ri) * static_cast<double>(ri);
    if (!(fin(ri) && fin(ap[i]) && fin(b[i]) && fin(x[i]))) v[3] += 1.0;
  })
  write_partials(v, part);
}

// One workgroup: the start decision (cg.cpp:122-145).
__global__ void __launch_bounds__(kSolverThreads)
    cg_decide_start(const double *part, int nparts, float rtol, float atol, int64_t maxiter,
                    CgState *st) {
  double t[kSlots];
  read_totals(part, nparts, t);
  if (threadIdx.x != 0) return;
  const double rr = t[1];
  const float residual_norm = static_cast<float>(sqrt(max0(rr)));
  const float b_norm = static_cast<float>(sqrt(max0(t[0])));
  const float scaled = rtol * b_norm;
  st->tol = atol > scaled ? atol : scaled;
  st->rr = rr;
  st->rr_next = rr;
  st->true_rr = 0.0;
  if (t[3] != 0.0 || !fin(rr) || !fin(residual_norm) || !fin(b_norm)) {
    stop(st, -3, 0);
  } else if (residual_norm <= st->tol) {
    stop(st, 0, 0);
  } else {
    st->status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
    st->completed = 0;
    st->running = maxiter > 0 ? 1 : 0;
  }
}

// p.ap, p.p, ap.ap, non-finite p/ap.  From the second iteration on, first
// checks the previous direction pass (any non-finite p stops with -3) and
// commits the residual norm it left.
__global__ void __launch_bounds__(kSolverThreads)
    cg_alpha(const float *__restrict__ p, const float *__restrict__ ap, int64_t n, int32_t it,
             const double *dir_part, double *part, int nparts, CgState *st) {
  if (!st->running) return;
  double pin[kSlots] = {0.0, 0.0, 0.0, 0.0};
  if (it > 1) load_partials(dir_part, nparts, pin);
  const float *const vec[2] = {p, ap};
  Round<2> first;
  load_round<2>(vec, first_base(), n, first);
  if (it > 1) {
    double t[kSlots];
    reduce_partials(pin, nparts, t);
    if (t[3] != 0.0) {
      if (blockIdx.x == 0 && threadIdx.x == 0) stop(st, -3, it - 1);
      return;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) st->rr = st->rr_next;
  }
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<2>(vec, n, first, [&](int64_t, const float(&e)[2]) {
    const double pd = e[0], ad = e[1];
    v[0] += pd * ad;
    v[1] += pd * pd;
    v[2] += ad * ad;
    if (!(fin(e[0]) && fin(e[1]))) v[3] += 1.0;
  });
  write_partials(v, part);
}

// alpha from the alpha pass (cg.cpp:158-199), then x += alpha p and
// r -= alpha ap in double, rounded once; r.r and non-finite counts.
__global__ void __launch_bounds__(kSolverThreads)
    cg_update(float *__restrict__ x, float *__restrict__ r, const float *__restrict__ p,
              const float *__restrict__ ap, int64_t n, int32_t it, const double *alpha_part,
              double *part, int nparts, CgState *st) {
  if (!st->running) return;
  double pin[kSlots];
  load_partials(alpha_part, nparts, pin);
  const float *const vec[4] = {x, r, p, ap};
  Round<4> first;
  load_round<4>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  const double denom = t[0];
  const double eps = static_cast<double>(FLT_EPSILON);
  int32_t verdict = 1;  // 1: go on
  if (t[3] != 0.0 || !fin(denom)) {
    verdict = -3;
  } else if (fabs(denom) <= eps) {
    const double scale = sqrt(max0(t[1] * t[2]));
    const double dtol = fmin(eps, eps * eps * fmax(1.0, scale));
    if (!fin(scale)) verdict = -3;
    else if (fabs(denom) <= dtol) verdict = -1;
  }
  const double alpha = st->rr / denom;
  if (verdict == 1 && !fin(alpha)) verdict = -3;
  if (verdict != 1) {
    if (lead) stop(st, verdict, it - 1);
    return;
  }
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  // All loads of a round first, then the arithmetic and the stores: written
  // as one loop body, the compiler waited for each element's loads in turn.
  for_rounds<4>(vec, n, first, [&](int64_t i, const float(&e)[4]) {
    const double xc = static_cast<double>(e[0]) + alpha * static_cast<double>(e[2]);
    const double rc = static_cast<double>(e[1]) - alpha * static_cast<double>(e[3]);
    const float xf = static_cast<float>(xc), rf = static_cast<float>(rc);
    if (!fin(xc) || !fin(rc) || !fin(xf) || !fin(rf)) {
      v[3] += 1.0;
    } else {
      x[i] = xf;
      r[i] = rf;
      v[0] += static_cast<double>(rf) * static_cast<double>(rf);
    }
  });
  write_partials(v, part);
}

// Convergence and beta from the update pass (cg.cpp:200-238), then
// p = r + beta p; non-finite p values are counted for the next alpha pass.
__global__ void __launch_bounds__(kSolverThreads)
    cg_direction(const float *__restrict__ r, float *__restrict__ p, int64_t n, int32_t it,
                 const double *upd_part, double *part, int nparts, CgState *st) {
  if (!st->running) return;
  double pin[kSlots];
  load_partials(upd_part, nparts, pin);
  const float *const vec[2] = {r, p};
  Round<2> first;
  load_round<2>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  const double rr_new = t[0];
  const float r_norm = static_cast<float>(sqrt(max0(rr_new)));
  if (t[3] != 0.0 || !fin(rr_new) || !fin(r_norm)) {
    if (lead) stop(st, -3, it);
    return;
  }
  if (r_norm <= st->tol) {
    if (lead) {
      st->rr = rr_new;
      stop(st, 0, it);
    }
    return;
  }
  const double beta = rr_new / st->rr;
  if (!fin(beta)) {
    if (lead) stop(st, -3, it);
    return;
  }
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<2>(vec, n, first, [&](int64_t i, const float(&e)[2]) {
    const double pc = static_cast<double>(e[0]) + beta * static_cast<double>(e[1]);
    const float pf = static_cast<float>(pc);
    if (!fin(pc) || !fin(pf)) v[3] += 1.0;
    else p[i] = pf;
  });
  write_partials(v, part);
  if (lead) {
    st->completed = it;
    st->rr_next = rr_new;
  }
}

// One workgroup, after the last launched iteration: settles the check the
// final direction pass left open.
__global__ void __launch_bounds__(kSolverThreads)
    cg_finish(const double *dir_part, int nparts, CgState *st) {
  if (!st->running) return;
  double t[kSlots];
  read_totals(dir_part, nparts, t);
  if (threadIdx.x != 0) return;
  if (t[3] != 0.0) {
    stop(st, -3, st->completed);
  } else {
    st->rr = st->rr_next;
    st->running = 0;
  }
}

// ---------------------------------------------------------------------------
// Jacobi-preconditioned CG (pcg.cpp:71-236): float scalars from double sums,
// float vector updates.

__device__ inline float to_f(double v) { return static_cast<float>(v); }

__global__ void __launch_bounds__(kSolverThreads)
    pcg_start(const float *__restrict__ b, const float *__restrict__ ap,
              const float *__restrict__ inv_diag, float *__restrict__ r, float *__restrict__ z,
              float *__restrict__ p, int64_t n, double *part) {
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const float ri = b[i] - ap[i];
    const float zi = inv_diag[i] * ri;
    r[i] = ri;
    z[i] = zi;
    p[i] = zi;
    v[0] += static_cast<double>(b[i]) * static_cast<double>(b[i]);
    v[1] += static_cast<double>(ri) * static_cast<double>(ri);
    v[2] += static_cast<double>(ri) * static_cast<double>(zi);
    if (!(fin(ri) && fin(zi) && fin(inv_diag[i]))) v[3] += 1.0;
  })
  write_partials(v, part);
}

__global__ void __launch_bounds__(kSolverThreads)
    pcg_decide_start(const double *part, int nparts, float rtol, float atol, int64_t maxiter,
                     CgState *st) {
  double t[kSlots];
  read_totals(part, nparts, t);
  if (threadIdx.x != 0) return;
  const float true_rr = to_f(t[1]), rho = to_f(t[2]);
  const float b_norm = static_cast<float>(sqrt(max0(t[0])));
  const float scaled = rtol * b_norm;
  st->tol = atol > scaled ? atol : scaled;
  st->true_rr = true_rr;
  st->rr = rho;
  st->rr_next = rho;
  const float true_residual = sqrtf(max0(true_rr));
  if (t[3] != 0.0 || !fin(true_rr) || !fin(rho)) {
    stop(st, -3, 0);
  } else if (true_residual <= st->tol) {
    stop(st, 0, 0);
  } else if (rho <= 0.0f) {
    stop(st, -2, 0);
  } else {
    st->status = maxiter > 0 ? static_cast<int32_t>(maxiter) : 1;
    st->completed = 0;
    st->running = maxiter > 0 ? 1 : 0;
  }
}

__global__ void __launch_bounds__(kSolverThreads)
    pcg_alpha(const float *__restrict__ p, const float *__restrict__ ap, int64_t n, int32_t it,
              double *part, CgState *st) {
  if (!st->running) return;
  if (it > 1 && blockIdx.x == 0 && threadIdx.x == 0) st->rr = st->rr_next;
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  MSX_SOLVER_LOOP({
    const double pd = p[i], ad = ap[i];
    v[0] += pd * ad;
    v[1] += pd * pd;
    v[2] += ad * ad;
  })
  write_partials(v, part);
}

// alpha (pcg.cpp:165-184), then x += alpha p; r -= alpha ap; z = inv_diag r;
// r.r and r.z.
__global__ void __launch_bounds__(kSolverThreads)
    pcg_update(float *__restrict__ x, float *__restrict__ r, float *__restrict__ z,
               const float *__restrict__ p, const float *__restrict__ ap,
               const float *__restrict__ inv_diag, int64_t n, int32_t it,
               const double *alpha_part, double *part, int nparts, CgState *st) {
  if (!st->running) return;
  double pin[kSlots];
  load_partials(alpha_part, nparts, pin);
  const float *const vec[5] = {x, p, r, ap, inv_diag};
  Round<5> first;
  load_round<5>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  const float eps = FLT_EPSILON;
  const float denom = to_f(t[0]), p2 = to_f(t[1]), ap2 = to_f(t[2]);
  const float scale = sqrtf(max0(p2 * ap2));
  const float dtol = eps * fmaxf(1.0f, scale);
  if (!fin(denom) || !fin(scale) || fabsf(denom) <= dtol) {
    if (lead) stop(st, -1, it - 1);
    return;
  }
  const float alpha = static_cast<float>(st->rr) / denom;
  if (!fin(alpha)) {
    if (lead) stop(st, -3, it - 1);
    return;
  }
  double v[kSlots] = {0.0, 0.0, 0.0, 0.0};
  for_rounds<5>(vec, n, first, [&](int64_t i, const float(&e)[5]) {
    const float xi = e[0] + alpha * e[1];
    const float ri = e[2] - alpha * e[3];
    const float zi = e[4] * ri;
    x[i] = xi;
    r[i] = ri;
    z[i] = zi;
    v[0] += static_cast<double>(ri) * static_cast<double>(ri);
    v[1] += static_cast<double>(ri) * static_cast<double>(zi);
    if (!(fin(xi) && fin(ri) && fin(zi))) v[3] += 1.0;
  });
  write_partials(v, part);
}

// Convergence, rho and beta (pcg.cpp:186-232), then p = z + beta p.
__global__ void __launch_bounds__(kSolverThreads)
    pcg_direction(const float *__restrict__ z, float *__restrict__ p, int64_t n, int32_t it,
                  const double *upd_part, int nparts, CgState *st) {
  if (!st->running) return;
  double pin[kSlots];
  load_partials(upd_part, nparts, pin);
  const float *const vec[2] = {z, p};
  Round<2> first;
  load_round<2>(vec, first_base(), n, first);
  double t[kSlots];
  reduce_partials(pin, nparts, t);
  const bool lead = blockIdx.x == 0 && threadIdx.x == 0;
  const float true_rr = to_f(t[0]);
  const float r_norm = sqrtf(max0(true_rr));
  int32_t verdict = 1;
  if (t[3] != 0.0 || !fin(true_rr) || !fin(r_norm)) verdict = -3;
  else if (r_norm <= st->tol) verdict = 0;
  const float rho_new = to_f(t[1]);
  if (verdict == 1 && (!fin(rho_new) || rho_new <= 0.0f)) verdict = -2;
  const float beta = rho_new / static_cast<float>(st->rr);
  if (verdict == 1 && !fin(beta)) verdict = -3;
  if (lead) {
    st->true_rr = true_rr;
    st->completed = it;
  }
  if (verdict != 1) {
    if (lead) stop(st, verdict, it);
    return;
  }
  for_rounds<2>(vec, n, first, [&](int64_t i, const float(&e)[2]) { p[i] = e[0] + beta * e[1]; });
  if (lead) st->rr_next = rho_new;
}

__global__ void pcg_finish(CgState *st) {
  if (threadIdx.x == 0 && st->running) st->running = 0;
}


__global__ void copy_vec(const float *__restrict__ src, float *__restrict__ dst, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kSolverThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kSolverThreads)
    dst[i] = src[i];
}

struct Solve {
  int64_t n, nnz;
  msx_itype it;
  const float *data;
  const void *indices, *indptr;
  const msx_csr_plan *plan;
  hipStream_t stream;
  uint32_t blocks;
};

msx_status spmv(const Solve &s, const float *x, float *y) {
  return launch_spmv(MSX_F32, s.it, s.n, s.n, s.nnz, s.data, s.indices, s.indptr, x, y, s.plan,
                     s.stream);
}

// Host loop: enqueue iterations in batches between reads of the state
// (BatchSchedule), stop when the device says so or maxiter is reached.
// The residual of the schedule: sqrt(r.r) (CG) or of the true r.r (PCG).
template <class Step>
msx_status drive(const Solve &s, int64_t maxiter, CgState *st_dev, CgState *st_host, bool pcg,
                 Step step) {
  auto residual = [&]() {
    const double rr = pcg ? st_host->true_rr : st_host->rr;
    return std::sqrt(std::max(rr, 0.0));
  };
  int64_t done = 0;
  BatchSchedule schedule;
  int64_t batch = schedule.next(0, residual(), st_host->tol);  // the start's state
  while (done < maxiter) {
    const int64_t todo = std::min(batch, maxiter - done);
    for (int64_t k = 0; k < todo; ++k) {
      msx_status e = step(static_cast<int32_t>(done + k + 1));
      if (e != MSX_OK) return e;
    }
    done += todo;
    MSX_HIP_TRY(hipMemcpyAsync(st_host, st_dev, sizeof(CgState), hipMemcpyDeviceToHost, s.stream));
    MSX_HIP_TRY(hipStreamSynchronize(s.stream));
    if (!st_host->running) return MSX_OK;
    // still running: every enqueued iteration has completed
    batch = schedule.next(done, residual(), st_host->tol);
  }
  return MSX_OK;
}

struct Scratch {
  char *base = nullptr;
  hipStream_t stream = nullptr;
  ~Scratch() {
    if (base) (void)hipFreeAsync(base, stream);
  }
};

msx_status finish(const Solve &s, CgState *st_dev, CgState *st_host, bool pcg,
                  msx_solver_result *result) {
  MSX_HIP_TRY(hipMemcpyAsync(st_host, st_dev, sizeof(CgState), hipMemcpyDeviceToHost, s.stream));
  MSX_HIP_TRY(hipStreamSynchronize(s.stream));
  result->info = st_host->status;
  result->iterations = st_host->completed;
  result->residual = pcg ? sqrtf(std::max(static_cast<float>(st_host->true_rr), 0.0f))
                         : static_cast<float>(std::sqrt(std::max(st_host->rr, 0.0)));
  result->reserved = 0;
  return MSX_OK;
}

msx_status solve(const Solve &s, const float *b, const float *x0, const float *inv_diag, float *x,
                 float rtol, float atol, int64_t maxiter, msx_solver_result *result) {
  const bool pcg = inv_diag != nullptr;
  const int64_t n = s.n;
  const size_t vec = (static_cast<size_t>(n) * sizeof(float) + 255) / 256 * 256;
  const size_t state_bytes = 256;
  const size_t part_bytes = sizeof(double) * kSlots * kSolverMaxBlocks;
  const int nvec = pcg ? 4 : 3;  // r, p, ap (+ z)
  Scratch sc;
  sc.stream = s.stream;
  MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&sc.base),
                             nvec * vec + state_bytes + 3 * part_bytes, s.stream));
  float *r = reinterpret_cast<float *>(sc.base);
  float *p = reinterpret_cast<float *>(sc.base + vec);
  float *ap = reinterpret_cast<float *>(sc.base + 2 * vec);
  float *z = pcg ? reinterpret_cast<float *>(sc.base + 3 * vec) : nullptr;
  auto *st = reinterpret_cast<CgState *>(sc.base + nvec * vec);
  // per-pass partial sums: alpha (also the start pass), update, direction
  auto *alpha_part = reinterpret_cast<double *>(sc.base + nvec * vec + state_bytes);
  auto *upd_part = reinterpret_cast<double *>(sc.base + nvec * vec + state_bytes + part_bytes);
  auto *dir_part = reinterpret_cast<double *>(sc.base + nvec * vec + state_bytes + 2 * part_bytes);
  const int nparts = static_cast<int>(s.blocks);
  CgState host{};
  const dim3 grid(s.blocks), block(kSolverThreads);

  hipLaunchKernelGGL(copy_vec, grid, block, 0, s.stream, x0, x, n);
  MSX_HIP_TRY(hipGetLastError());
  msx_status e = spmv(s, x, ap);
  if (e != MSX_OK) return e;
  if (pcg) {
    hipLaunchKernelGGL(pcg_start, grid, block, 0, s.stream, b, ap, inv_diag, r, z, p, n, alpha_part);
    hipLaunchKernelGGL(pcg_decide_start, dim3(1), block, 0, s.stream, alpha_part, nparts, rtol,
                       atol, maxiter, st);
  } else {
    hipLaunchKernelGGL(cg_start, grid, block, 0, s.stream, b, x, ap, r, p, n, alpha_part);
    hipLaunchKernelGGL(cg_decide_start, dim3(1), block, 0, s.stream, alpha_part, nparts, rtol,
                       atol, maxiter, st);
  }
  MSX_HIP_TRY(hipGetLastError());
  MSX_HIP_TRY(hipMemcpyAsync(&host, st, sizeof(CgState), hipMemcpyDeviceToHost, s.stream));
  MSX_HIP_TRY(hipStreamSynchronize(s.stream));
  if (host.running) {
    auto step = [&](int32_t k) -> msx_status {
      msx_status es = spmv(s, p, ap);
      if (es != MSX_OK) return es;
      if (pcg) {
        hipLaunchKernelGGL(pcg_alpha, grid, block, 0, s.stream, p, ap, n, k, alpha_part, st);
        hipLaunchKernelGGL(pcg_update, grid, block, 0, s.stream, x, r, z, p, ap, inv_diag, n, k,
                           alpha_part, upd_part, nparts, st);
        hipLaunchKernelGGL(pcg_direction, grid, block, 0, s.stream, z, p, n, k, upd_part, nparts,
                           st);
      } else {
        hipLaunchKernelGGL(cg_alpha, grid, block, 0, s.stream, p, ap, n, k, dir_part, alpha_part,
                           nparts, st);
        hipLaunchKernelGGL(cg_update, grid, block, 0, s.stream, x, r, p, ap, n, k, alpha_part,
                           upd_part, nparts, st);
        hipLaunchKernelGGL(cg_direction, grid, block, 0, s.stream, r, p, n, k, upd_part, dir_part,
                           nparts, st);
      }
      MSX_HIP_TRY(hipGetLastError());
      return MSX_OK;
    };
    e = drive(s, maxiter, st, &host, pcg, step);
    if (e != MSX_OK) return e;
    if (pcg)
      hipLaunchKernelGGL(pcg_finish, dim3(1), dim3(kWave), 0, s.stream, st);
    else
      hipLaunchKernelGGL(cg_finish, dim3(1), block, 0, s.stream, dir_part, nparts, st);
    MSX_HIP_TRY(hipGetLastError());
  }
  return finish(s, st, &host, pcg, result);
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

extern "C" msx_status msx_csr_cg(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                 const void *indices, const void *indptr, const float *b,
                                 const float *x0, float *x, float rtol, float atol,
                                 int64_t maxiter, const msx_csr_plan *plan,
                                 msx_solver_result *result, void *stream) {
  clear_error();
  msx_status st = check("csr_cg", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  st = check_plan("csr_cg", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const Solve s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                blocks_for(n)};
  return solve(s, b, x0, nullptr, x, rtol, atol, maxiter, result);
}

extern "C" msx_status msx_csr_pcg_jacobi(msx_itype it, int64_t n, int64_t nnz, const float *data,
                                         const void *indices, const void *indptr, const float *b,
                                         const float *x0, const float *inv_diag, float *x,
                                         float rtol, float atol, int64_t maxiter,
                                         const msx_csr_plan *plan, msx_solver_result *result,
                                         void *stream) {
  clear_error();
  msx_status st =
      check("csr_pcg_jacobi", it, n, nnz, data, indices, indptr, b, x0, x, maxiter, result);
  if (st != MSX_OK) return st;
  if (inv_diag == nullptr) return fail(MSX_EINVAL, "csr_pcg_jacobi inverse diagonal is NULL.");
  st = check_plan("csr_pcg_jacobi", plan, MSX_F32, it, n, n, nnz, data, indices, indptr);
  if (st != MSX_OK) return st;
  const Solve s{n, nnz, it, data, indices, indptr, plan, static_cast<hipStream_t>(stream),
                blocks_for(n)};
  return solve(s, b, x0, inv_diag, x, rtol, atol, maxiter, result);
}
