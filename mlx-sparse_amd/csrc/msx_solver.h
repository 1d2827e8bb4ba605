// msx_solver.h - device-side building blocks of the Krylov solver loops
// (csr_cg.hip, csr_krylov.hip): workgroup sizes, the reproducible
// partial-sum protocol and the grid-stride loop with loads in flight.
//
// Sums: each workgroup reduces its grid-stride share in double and writes
// one partial per slot; every workgroup of the NEXT pass adds those
// partials in workgroup order, so all workgroups see the same bits and
// take the same scalar decisions, and no workgroup waits on another inside
// a kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

#include "msx_device.h"

namespace msx {
namespace solver {

constexpr int kSolverThreads = 512;
constexpr int kSolverMaxBlocks = 512;  // two workgroups per CU at most (partials re-read by each)
constexpr int kSlots = 4;              // partial sums per pass
constexpr int kUnroll = 4;             // independent loads in flight per thread

__device__ inline bool fin(float v) { return isfinite(v); }
__device__ inline bool fin(double v) { return isfinite(v); }

// std::max(v, 0) of the reference loops: a NaN stays NaN (fmax would drop it).
__device__ inline double max0(double v) { return v < 0.0 ? 0.0 : v; }
__device__ inline float max0(float v) { return v < 0.0f ? 0.0f : v; }

__device__ inline double wave_sum(double v) {
  // butterfly: every lane ends with the same value (each level adds a
  // commutative pair)
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Workgroup sums of v[] -> part[k * kSolverMaxBlocks + blockIdx.x].
__device__ inline void write_partials(double (&v)[kSlots], double *part) {
  __shared__ double sh[kSlots][kSolverThreads / kWave];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (int k = 0; k < kSlots; ++k) {
    const double w = wave_sum(v[k]);
    if (lane == 0) sh[k][wave] = w;
  }
  __syncthreads();
  if (threadIdx.x < kSlots) {
    double s = 0.0;
    for (int w = 0; w < kSolverThreads / kWave; ++w) s += sh[threadIdx.x][w];
    part[threadIdx.x * kSolverMaxBlocks + blockIdx.x] = s;
  }
}

// Totals of the previous pass's `nparts` partials, the same bits in every
// workgroup (fixed order, written by an earlier kernel).  In two steps, so
// that a kernel can issue its own element loads between them: loads are
// waited on in issue order, so partials loaded after the elements would wait
// for the elements too.
__device__ inline void load_partials(const double *part, int nparts, double (&v)[kSlots]) {
  // all kSlots loads at once (clamped index, no branch)
  const int idx = static_cast<int>(threadIdx.x) < nparts ? static_cast<int>(threadIdx.x) : 0;
#pragma unroll
  for (int k = 0; k < kSlots; ++k) v[k] = part[k * kSolverMaxBlocks + idx];
}

__device__ inline void reduce_partials(const double (&v)[kSlots], int nparts, double (&t)[kSlots]) {
  __shared__ double sh[kSlots][kSolverThreads / kWave];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const bool mine = static_cast<int>(threadIdx.x) < nparts;
#pragma unroll
  for (int k = 0; k < kSlots; ++k) {
    const double w = wave_sum(mine ? v[k] : 0.0);
    if (lane == 0) sh[k][wave] = w;
  }
  __syncthreads();
  for (int k = 0; k < kSlots; ++k) {
    double s = 0.0;
    for (int w = 0; w < kSolverThreads / kWave; ++w) s += sh[k][w];
    t[k] = s;
  }
  __syncthreads();
}

__device__ inline void read_totals(const double *part, int nparts, double (&t)[kSlots]) {
  double v[kSlots];
  load_partials(part, nparts, v);
  reduce_partials(v, nparts, t);
}

// Grid-stride over [0, n) with kUnroll coalesced elements per round.
// A thread whose kUnroll elements all lie below n runs them without a
// per-element test, so the compiler issues all of their loads before the
// first use (a test per element made it wait for each load in turn); the
// last, partial group tests each element.
#define MSX_SOLVER_LOOP(...)                                                                    \
  {                                                                                          \
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kSolverThreads;                     \
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kSolverThreads + threadIdx.x; base < n; \
         base += kUnroll * stride) {                                                         \
      if (base + (kUnroll - 1) * stride < n) {                                               \
        _Pragma("unroll") for (int u = 0; u < kUnroll; ++u) {                                \
          const int64_t i = base + u * stride;                                               \
          __VA_ARGS__                                                                        \
        }                                                                                    \
      } else {                                                                               \
        _Pragma("unroll") for (int u = 0; u < kUnroll; ++u) {                                \
          const int64_t i = base + u * stride;                                               \
          if (i < n) { __VA_ARGS__ }                                                         \
        }                                                                                    \
      }                                                                                      \
    }                                                                                        \
  }

// A pass whose arithmetic needs the previous pass's totals issues, in this
// order, that pass's partial loads (load_partials), the loads of its own
// first round of elements (load_round: kUnroll grid-stride elements of each
// of NV vectors; an index past n reads the thread's first element, or
// element 0), then reduces the partials (reduce_partials) and runs
// for_rounds: op(i, e) for every element i of the thread in grid-stride
// order, e holding its NV values - the first round from those registers,
// each later round loaded whole before its first use.  The reduction's
// wave sums and barriers then overlap the element loads.
template <int NV>
struct Round {
  float e[kUnroll][NV];
};

template <int NV>
__device__ inline void load_round(const float *const (&vec)[NV], int64_t base, int64_t n,
                                  Round<NV> &r) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kSolverThreads;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t j = base + u * stride < n ? base + u * stride : (base < n ? base : 0);
#pragma unroll
    for (int k = 0; k < NV; ++k) r.e[u][k] = vec[k][j];
  }
}

__device__ inline int64_t first_base() {
  return static_cast<int64_t>(blockIdx.x) * kSolverThreads + threadIdx.x;
}

template <int NV, class Op>
__device__ inline void for_rounds(const float *const (&vec)[NV], int64_t n, const Round<NV> &first,
                                  Op op) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kSolverThreads;
  const int64_t base0 = first_base();
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
    if (base0 + u * stride < n) op(base0 + u * stride, first.e[u]);
  for (int64_t base = base0 + kUnroll * stride; base < n; base += kUnroll * stride) {
    Round<NV> r;
    load_round<NV>(vec, base, n, r);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (base + u * stride < n) op(base + u * stride, r.e[u]);
  }
}

// Host side: iterations to enqueue before the next read of the solver
// state.  An iteration enqueued past the solve's stop still runs its SpMVs
// in full (only the vector passes return early), while a read costs a round
// trip to the host; so the batch doubles (1, 2, 4, ... kMaxBatch) until two
// reads give a rate of residual decrease, and from then on covers the
// iterations that rate needs to reach the tolerance (at most kMaxBatch).
// The device alone decides where the solve stops, so results do not depend
// on the batches.
class BatchSchedule {
 public:
  static constexpr int64_t kMaxBatch = 32;
  // `completed` iterations done, their residual norm, the solve's tolerance.
  int64_t next(int64_t completed, double residual, double tol) {
    int64_t b = doubling_;
    if (k_ >= 0 && completed > k_ && residual > tol && tol > 0.0 && residual < res_) {
      const double rate = std::log(residual / res_) / static_cast<double>(completed - k_);
      const double need = std::ceil(std::log(tol / residual) / rate);
      b = need >= static_cast<double>(kMaxBatch) ? kMaxBatch : (need < 1.0 ? 1 : static_cast<int64_t>(need));
    }
    doubling_ = doubling_ * 2 < kMaxBatch ? doubling_ * 2 : kMaxBatch;
    k_ = completed;
    res_ = residual;
    return b;
  }

 private:
  int64_t doubling_ = 1;
  int64_t k_ = -1;
  double res_ = 0.0;
};

// Workgroups of a solver pass over n elements (kUnroll per thread and round).
inline uint32_t blocks_for(int64_t n) {
  const int64_t per_block = static_cast<int64_t>(kUnroll) * kSolverThreads;
  const int64_t blocks = (n + per_block - 1) / per_block;
  return static_cast<uint32_t>(blocks < 1 ? 1 : (blocks > kSolverMaxBlocks ? kSolverMaxBlocks : blocks));
}

}  // namespace solver
}  // namespace msx
