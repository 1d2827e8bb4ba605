// csr_spmm.hip - CSR SpMM with a dense row-major right-hand side, gfx950.
//
//   Y[i, c] = sum_{p in [indptr[i], indptr[i+1])} data[p] * X[indices[p], c]
//
// The reference launches one Metal thread per output element (or 128 lanes
// per element), so each row's indices/data are re-read k times (reference:
// src/sparse/csr_matmul/csr_matmul.metal:17-39,86-120).  Here one group of LR
// lanes owns a whole row of Y: each lane holds CW consecutive columns in
// registers (CW * sizeof(value) = 16 bytes when the layout allows, else 1
// column), walks the row's stored values once in order, and reads the
// matching X row as one 16-byte load per lane, so the LR lanes together read
// a contiguous X row segment.  A row's indices and data are read once per
// column tile of 64 * CW columns instead of once per column.  Each column is
// summed from zero in stored order - the reference's CPU order
// (src/sparse/csr_matmul/csr_matmul.cpp:83-133) - so float32 results match
// its CPU kernel bit for bit.  A row's values are taken in chunks of 8: one
// load per lane fetches the chunk's columns and values (lane l holds value
// l, shared with the group by shuffles; groups narrower than 8 lanes load the
// whole chunk per lane), then all of the chunk's X loads are issued before
// the first use.  A 7-value stencil row thus costs three dependent round
// trips (bounds, chunk, X rows) instead of one per value: on the 3D Poisson
// matrix at k = 64 this took the SpMM from 467 to about 380 us.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "msx_device.h"
#include "msx_internal.h"

namespace msx {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kMaxGrid = 1u << 20;
constexpr int64_t kMaxBatchGrid = 65535;  // batches per launch (grid y extent)

template <class S, int CW>
struct Vec {
  S v[CW];
};

template <class S, int CW>
__device__ inline Vec<S, CW> load_vec(const S *p) {
  if constexpr (CW * sizeof(S) == 16) {
    const uint4 raw = *reinterpret_cast<const uint4 *>(p);
    return __builtin_bit_cast(Vec<S, CW>, raw);
  } else {
    Vec<S, CW> r;
#pragma unroll
    for (int c = 0; c < CW; ++c) r.v[c] = p[c];
    return r;
  }
}

// Y is written once and not read back by the kernel: 16-byte stores are
// non-temporal (measured at k = 8 / 64 / 256 on the 3D Poisson matrix: 63 ->
// 52, 362 -> 351, 1,694 -> 1,650 us), unless the caller reads Y again right
// away (the batched SpMV's transposed intermediate: NT false).  NT is a
// template parameter: a runtime choice between the two stores is merged by
// the compiler into one ordinary store.
template <class S, int CW, bool NT = true>
__device__ inline void store_vec(S *p, const Vec<S, CW> &v) {
  if constexpr (CW * sizeof(S) == 16) {
    using W = uint32_t __attribute__((ext_vector_type(4)));
    const W w = __builtin_bit_cast(W, v);
    if constexpr (NT) __builtin_nontemporal_store(w, reinterpret_cast<W *>(p));
    else *reinterpret_cast<W *>(p) = w;
  } else {
#pragma unroll
    for (int c = 0; c < CW; ++c) p[c] = v.v[c];
  }
}

__device__ inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

constexpr int kChunk = 8;         // values per chunk of a row (shuffle path)
constexpr int kUnrollDirect = 4;  // values per step when each lane loads them itself

__device__ inline float shfl_idx(float v, int src, int width) { return __shfl(v, src, width); }
__device__ inline c64 shfl_idx(c64 v, int src, int width) {
  return c64{__shfl(v.re, src, width), __shfl(v.im, src, width)};
}

// Y-row segment of row [s, e): sum from zero in stored order; fetch(c)
// returns the lane's CW values of X row c.  The row's group is LR lanes wide
// (lane l of it); every lane of the group calls this with the same s and e.  SHUF: LR >= kChunk, a chunk of kChunk
// values is loaded one value per lane and shared by shuffles; otherwise every
// lane loads the values itself, kUnrollDirect per step (narrow groups, small
// k: measured faster there than whole chunks).  Columns outside [0, n_cols)
// add nothing.
template <class V, class I, int CW, bool SHUF, class Fetch>
__device__ inline void row_segment(const typename V::Storage *__restrict__ data,
                                   const I *__restrict__ indices, Fetch fetch, int64_t n_cols,
                                   int64_t s, int64_t e, int l, int LR,
                                   typename V::Acc (&acc)[CW]) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  // Positions stay 64-bit: 32-bit ones measured 15 % slower here (the
  // address arithmetic of the index and value loads).
#pragma unroll
  for (int c = 0; c < CW; ++c) acc[c] = vzero<A>();
  if constexpr (!SHUF) {
    // Narrow groups: four values per step, loads issued before use.
    int64_t p = s;
    for (; p + kUnrollDirect <= e; p += kUnrollDirect) {
      int cu[kUnrollDirect];
      A au[kUnrollDirect];
      Vec<S, CW> xv[kUnrollDirect];
#pragma unroll
      for (int u = 0; u < kUnrollDirect; ++u) {
        const I c = indices[p + u];
        cu[u] = static_cast<uint64_t>(static_cast<int64_t>(c)) < static_cast<uint64_t>(n_cols) ? static_cast<int>(c) : -1;
        au[u] = V::widen(data[p + u]);
      }
#pragma unroll
      for (int u = 0; u < kUnrollDirect; ++u)
        if (cu[u] >= 0) xv[u] = fetch(cu[u]);
#pragma unroll
      for (int u = 0; u < kUnrollDirect; ++u)
        if (cu[u] >= 0) {
#pragma unroll
          for (int c = 0; c < CW; ++c) acc[c] = vmadd<V>(acc[c], au[u], xv[u].v[c]);
        }
    }
    for (; p < e; ++p) {
      const I c = indices[p];
      if (static_cast<uint64_t>(static_cast<int64_t>(c)) < static_cast<uint64_t>(n_cols)) {
        const A a = V::widen(data[p]);
        const Vec<S, CW> xv = fetch(static_cast<int>(c));
#pragma unroll
        for (int q = 0; q < CW; ++q) acc[q] = vmadd<V>(acc[q], a, xv.v[q]);
      }
    }
    return;
  }
  auto chunk = [&](int64_t b) {
    int cu[kChunk];
    A au[kChunk];
    int ci = -1;
    A av = vzero<A>();
    if (l < kChunk && b + l < e) {
      const I c = indices[b + l];
      ci = static_cast<uint64_t>(static_cast<int64_t>(c)) < static_cast<uint64_t>(n_cols) ? static_cast<int>(c) : -1;
      av = V::widen(data[b + l]);
    }
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      cu[u] = __shfl(ci, u, LR);
      au[u] = shfl_idx(av, u, LR);
    }
    Vec<S, CW> xv[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      if (cu[u] >= 0) xv[u] = fetch(cu[u]);
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      if (cu[u] >= 0) {
#pragma unroll
        for (int c = 0; c < CW; ++c) acc[c] = vmadd<V>(acc[c], au[u], xv[u].v[c]);
      }
  };
  // The first chunk outside the loop: rows of up to 8 values (stencils)
  // then run straight-line code.
  chunk(s);
  for (int64_t b = s + kChunk; b < e; b += kChunk) chunk(b);
}

// LRT: the group width LR as a compile-time constant (a runtime width in
// every shuffle and index measured 6 % slower at k = 256); 0 takes LR_rt.
// Float32 rows of 16-byte chunks are held to 72 registers, 7 waves per SIMD
// (k = 256 on the 3D Poisson matrix: 1,641 -> 1,607 us; at 64 registers the
// spills cost 30 %).
template <class V, class I, int CW, bool SHUF, int LRT = 0, bool NTY = true>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(std::is_same_v<V, F32> && CW == 4 ? 7 : 1, 8)))
    spmm_rows(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
              const I *__restrict__ indptr, const typename V::Storage *__restrict__ X,
              int64_t ldx, typename V::Storage *__restrict__ Y, int64_t ldy, int64_t n_rows,
              int64_t nnz, int64_t n_cols, int64_t k, int LR_rt, int64_t n_col_tiles, int64_t x_batch,
              int64_t y_batch) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int LR = LRT > 0 ? LRT : LR_rt;
  X += blockIdx.y * x_batch;  // batch blockIdx.y (one for a plain SpMM)
  Y += blockIdx.y * y_batch;
  const int rows_per_group = kThreads / LR;
  const int g = threadIdx.x / LR;
  const int l = threadIdx.x % LR;
  const int64_t tile_cols = static_cast<int64_t>(LR) * CW;
  const int64_t n_row_tiles = (n_rows + rows_per_group - 1) / rows_per_group;
  const int64_t n_tiles = n_row_tiles * n_col_tiles;
  for (int64_t t = xcd_remap(blockIdx.x, gridDim.x); t < n_tiles; t += gridDim.x) {
    // one column tile (k <= 64 * CW) is the common case: no 64-bit division
    // (measured 1,767 -> 1,627 us at k = 256 on the 3D Poisson matrix)
    const int64_t rt = n_col_tiles == 1 ? t : t / n_col_tiles;
    const int64_t ct = t - rt * n_col_tiles;
    const int64_t row = rt * rows_per_group + g;
    const int64_t col = ct * tile_cols + static_cast<int64_t>(l) * CW;
    if (row >= n_rows) continue;
    const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    A acc[CW];
    // Lanes past k still take part in the shuffles; they read column 0.
    const S *Xc = X + (col < k ? col : 0);
    row_segment<V, I, CW, SHUF>(
        data, indices, [&](int c) { return load_vec<S, CW>(Xc + static_cast<int64_t>(c) * ldx); },
        n_cols, s, e, l, LR, acc);
    if (col >= k) continue;
    Vec<S, CW> out;
#pragma unroll
    for (int c = 0; c < CW; ++c) out.v[c] = V::narrow(acc[c]);
    store_vec<S, CW, NTY>(Y + row * ldy + col, out);
  }
}

// Batched SpMV from the transposed vectors: Xt is n_cols x kpad (row c
// holds x_b[c] of every vector b, padded to whole 16-byte vectors), and
// each row's sums go straight to the vectors of Y (Y[b * ldy + row], b <
// batch) - the same sums as spmm_rows over Xt, without an n_rows x kpad
// intermediate and its transpose.  A wave's stores for one vector are
// consecutive rows.
template <class V, class I, int CW, int LR>
__global__ void __launch_bounds__(kThreads)
    spmv_batch_rows(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                    const I *__restrict__ indptr, const typename V::Storage *__restrict__ Xt,
                    int64_t kpad, typename V::Storage *__restrict__ Y, int64_t ldy, int64_t batch,
                    int64_t n_rows, int64_t nnz, int64_t n_cols) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  constexpr int kRowsPerGroup = kThreads / LR;
  const int g = threadIdx.x / LR;
  const int l = threadIdx.x % LR;
  const int64_t n_tiles = (n_rows + kRowsPerGroup - 1) / kRowsPerGroup;
  for (int64_t t = xcd_remap(blockIdx.x, gridDim.x); t < n_tiles; t += gridDim.x) {
    const int64_t row = t * kRowsPerGroup + g;
    if (row >= n_rows) continue;
    const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    A acc[CW];
    const S *Xc = Xt + static_cast<int64_t>(l) * CW;
    row_segment<V, I, CW, (LR >= kChunk)>(
        data, indices, [&](int c) { return load_vec<S, CW>(Xc + static_cast<int64_t>(c) * kpad); },
        n_cols, s, e, l, LR, acc);
#pragma unroll
    for (int c = 0; c < CW; ++c) {
      const int64_t b = static_cast<int64_t>(l) * CW + c;
      if (b >= batch) continue;
      // float32: non-temporal (each wave writes whole lines, read by no one here)
      if constexpr (std::is_same_v<V, F32>)
        __builtin_nontemporal_store(V::narrow(acc[c]), Y + b * ldy + row);
      else
        Y[b * ldy + row] = V::narrow(acc[c]);
    }
  }
}

// Line-tiled SpMM for X rows of G whole 128-byte cache lines.  XCD x
// (workgroup g runs on XCD g % 8) owns column tile x % G (one line) and a
// contiguous G/8 share of the rows.  Each XCD then keeps only its own line of
// every X row in its L2, halving (G = 2) the X window that a stencil's far
// neighbours need, at the cost of reading each row's indices/data G times.
// Sums per column are in stored order, as in spmm_rows.
template <class V, class I, int CW, bool NTY = true>
__global__ void __launch_bounds__(kThreads)
    spmm_linetile(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                  const I *__restrict__ indptr, const typename V::Storage *__restrict__ X,
                  int64_t ldx, typename V::Storage *__restrict__ Y, int64_t ldy, int64_t n_rows,
                  int64_t nnz, int64_t n_cols, int G, int64_t x_batch, int64_t y_batch) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  X += blockIdx.y * x_batch;
  Y += blockIdx.y * y_batch;
  constexpr int LR = 128 / (CW * static_cast<int>(sizeof(S)));  // lanes per row (one line)
  constexpr int kRowsPerGroup = kThreads / LR;
  const int xcd = static_cast<int>(blockIdx.x % kNumXcd);
  const int64_t slot = blockIdx.x / kNumXcd;
  const int64_t slots = gridDim.x / kNumXcd;
  const int ct = xcd % G;
  const int gi = xcd / G;
  const int n_groups = kNumXcd / G;
  const int64_t n_rt = (n_rows + kRowsPerGroup - 1) / kRowsPerGroup;
  const int64_t rt_begin = n_rt * gi / n_groups;
  const int64_t rt_end = n_rt * (gi + 1) / n_groups;
  const int g = threadIdx.x / LR;
  const int l = threadIdx.x % LR;
  const int64_t col = static_cast<int64_t>(ct) * LR * CW + static_cast<int64_t>(l) * CW;
  for (int64_t rt = rt_begin + slot; rt < rt_end; rt += slots) {
    const int64_t row = rt * kRowsPerGroup + g;
    if (row >= n_rows) continue;
    const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    A acc[CW];
    const S *Xc = X + col;
    row_segment<V, I, CW, true>(
        data, indices, [&](int c) { return load_vec<S, CW>(Xc + static_cast<int64_t>(c) * ldx); },
        n_cols, s, e, l, LR, acc);
    Vec<S, CW> out;
#pragma unroll
    for (int c = 0; c < CW; ++c) out.v[c] = V::narrow(acc[c]);
    store_vec<S, CW, NTY>(Y + row * ldy + col, out);
  }
}

// ---------------------------------------------------------------------------
// Column windows.  A bound plan records, for each tile of kWinRows
// consecutive rows, the lowest and highest valid column of its values.  On a
// banded matrix (half-bandwidth 32) a tile's values touch about 100 rows of
// X, yet each row gathers one X row per value (about 43): staging the
// window once per workgroup with coalesced loads and gathering from LDS
// reads X from L2 about three times per tile instead of once per value.
constexpr int kWinRows = 32;
constexpr int64_t kWinLdsBytes = 65536;  // LDS of one workgroup's window

// A tile with more values than this can never be staged (4-byte columns
// alone would fill the 64 KB), so its window is not scanned: it is recorded
// empty and its value count disables the window kernel for the matrix.
constexpr int64_t kWinScanMax = 16384;

template <class I>
__global__ void __launch_bounds__(kThreads)
    window_bounds(const I *__restrict__ indices, const I *__restrict__ indptr, int64_t n_rows,
                  int64_t nnz, int64_t n_cols, int64_t n_win, int32_t *__restrict__ win,
                  unsigned long long *__restrict__ widest) {
  // widest[0]: window rows, widest[1]: values of a tile; one atomic per
  // workgroup (a wave per tile would serialise tens of thousands on them)
  __shared__ unsigned long long wg_max[2][kThreads / kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  unsigned long long w_rows = 0, w_vals = 0;
  for (int64_t t = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + wave; t < n_win;
       t += static_cast<int64_t>(gridDim.x) * (kThreads / kWave)) {
    const int64_t r0 = t * kWinRows;
    const int64_t r1 = std::min<int64_t>(r0 + kWinRows, n_rows);
    const int64_t p0 = clamp64(static_cast<int64_t>(indptr[r0]), 0, nnz);
    const int64_t p1 = clamp64(static_cast<int64_t>(indptr[r1]), p0, nnz);
    const int64_t cnt = p1 - p0;
    w_vals = std::max<unsigned long long>(w_vals, static_cast<unsigned long long>(cnt));
    int64_t lo = INT64_MAX, hi = -1;
    if (cnt <= kWinScanMax) {
      // four unconditional loads per lane and step (past the tile: zero, masked)
      const auto rr = make_rsrc(indices + p0, static_cast<uint64_t>(cnt) * sizeof(I));
      for (int64_t b = 0; b < cnt; b += 4 * kWave) {
        I c[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          c[u] = buffer_index<I>(rr, static_cast<uint32_t>(b + lane + u * kWave) * sizeof(I));
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t v = static_cast<int64_t>(c[u]);
          if (b + lane + u * kWave < cnt && static_cast<uint64_t>(v) < static_cast<uint64_t>(n_cols)) {
            lo = v < lo ? v : lo;
            hi = v > hi ? v : hi;
          }
        }
      }
#pragma unroll
      for (int d = kWave / 2; d >= 1; d >>= 1) {
        const int64_t ol = __shfl_xor(lo, d, kWave);
        const int64_t oh = __shfl_xor(hi, d, kWave);
        lo = ol < lo ? ol : lo;
        hi = oh > hi ? oh : hi;
      }
    }
    const bool any = hi >= lo;
    if (lane == 0) {
      win[2 * t] = any ? static_cast<int32_t>(lo) : 1;
      win[2 * t + 1] = any ? static_cast<int32_t>(hi) : 0;
    }
    if (any) w_rows = std::max<unsigned long long>(w_rows, static_cast<unsigned long long>(hi - lo + 1));
  }
  if (lane == 0) {
    wg_max[0][wave] = w_rows;
    wg_max[1][wave] = w_vals;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long a = 0, b = 0;
    for (int w = 0; w < kThreads / kWave; ++w) {
      a = std::max(a, wg_max[0][w]);
      b = std::max(b, wg_max[1][w]);
    }
    if (a > 0) atomicMax(widest, a);
    if (b > 0) atomicMax(widest + 1, b);
  }
}

// One workgroup per row tile.  Staged in LDS with loads all issued at once:
// X rows [lo, hi] of the tile's window (LR lanes of 16 bytes, the whole k),
// the tile's columns and widened values (its positions [p0, p1)), and its
// row pointers.  Each row is then summed from zero in stored order, as in
// spmm_rows, from LDS only.  A column outside the window (the indices
// changed after the plan was built) is read from X directly, and a row
// outside [p0, p1) (non-monotone indptr) or a tile with more values than
// staged takes the global path, so the result never depends on the plan.
template <class V, class I, int CW>
__global__ void __launch_bounds__(kThreads)
    spmm_window(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                const I *__restrict__ indptr, const typename V::Storage *__restrict__ X,
                int64_t ldx, typename V::Storage *__restrict__ Y, int64_t ldy, int64_t n_rows,
                int64_t nnz, int64_t n_cols, int64_t k, int LR, const int32_t *__restrict__ win,
                int64_t n_win, int64_t win_rows_cap, int64_t tile_nnz_cap) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  static_assert(CW * sizeof(S) == 16, "window rows are staged in 16-byte lanes");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  // Layout (the launcher sizes it alike): X window, row pointers, columns
  // and values in their storage type (counts rounded to a multiple of 4, so
  // every array stays aligned).
  const int64_t cap4 = (tile_nnz_cap + 3) & ~int64_t{3};
  uint4 *xs = reinterpret_cast<uint4 *>(lds_raw);                  // win_rows_cap * LR
  int64_t *rptr = reinterpret_cast<int64_t *>(xs + win_rows_cap * LR);  // kWinRows + 1 (+1)
  int32_t *cols = reinterpret_cast<int32_t *>(rptr + kWinRows + 2);     // cap4
  S *vals = reinterpret_cast<S *>(cols + cap4);                         // cap4
  const int g = threadIdx.x / LR;
  const int l = threadIdx.x % LR;
  const int lg = __builtin_ctz(static_cast<unsigned>(LR));  // LR is a power of two
  const int rows_per_pass = kThreads / LR;
  const int64_t col = static_cast<int64_t>(l) * CW;
  const S *Xc = X + (col < k ? col : 0);
  for (int64_t t = xcd_remap(blockIdx.x, gridDim.x); t < n_win; t += gridDim.x) {
    const int64_t lo = win[2 * t];
    const int64_t nw = std::min<int64_t>(
        win_rows_cap, std::max<int64_t>(0, static_cast<int64_t>(win[2 * t + 1]) - lo + 1));
    const int64_t r0 = t * kWinRows;
    const int64_t r1 = std::min<int64_t>(r0 + kWinRows, n_rows);
    const int64_t p0 = clamp64(static_cast<int64_t>(indptr[r0]), 0, nnz);
    const int64_t p1 = clamp64(static_cast<int64_t>(indptr[r1]), p0, nnz);
    const bool staged = p1 - p0 <= tile_nnz_cap;
    for (int64_t q = threadIdx.x; q < nw * LR; q += kThreads) {
      const int64_t wr = q / LR;
      const int64_t wc = (q - wr * LR) * CW;
      if (wc < k) xs[q] = *reinterpret_cast<const uint4 *>(X + (lo + wr) * ldx + wc);
    }
    // cols[q]: the value's row in the window (>= 0); -1 for a column
    // outside [0, n_cols) (adds nothing); -2 - c for a valid column c
    // outside the window (read from X).
    if (staged) {
      for (int64_t q = threadIdx.x; q < p1 - p0; q += kThreads) {
        const int64_t c = static_cast<int64_t>(indices[p0 + q]);
        const int64_t w = c - lo;
        int32_t code = -1;
        if (static_cast<uint64_t>(c) < static_cast<uint64_t>(n_cols))
          code = static_cast<uint64_t>(w) < static_cast<uint64_t>(nw) ? static_cast<int32_t>(w)
                                                                       : static_cast<int32_t>(-2 - c);
        cols[q] = code;
        vals[q] = data[p0 + q];
      }
    }
    for (int64_t q = threadIdx.x; q <= r1 - r0; q += kThreads)
      rptr[q] = static_cast<int64_t>(indptr[r0 + q]);
    __syncthreads();
    auto fetch = [&](int c) {
      const int64_t w = static_cast<int64_t>(c) - lo;
      if (static_cast<uint64_t>(w) < static_cast<uint64_t>(nw))
        return __builtin_bit_cast(Vec<S, CW>, xs[w * LR + l]);
      return load_vec<S, CW>(Xc + static_cast<int64_t>(c) * ldx);
    };
    for (int64_t row = r0 + g; row < r1; row += rows_per_pass) {
      const int64_t s = clamp64(rptr[row - r0], 0, nnz);
      const int64_t e = clamp64(rptr[row - r0 + 1], s, nnz);
      A acc[CW];
#pragma unroll
      for (int c = 0; c < CW; ++c) acc[c] = vzero<A>();
      if (staged && s >= p0 && e <= p1) {
        // Window reads for four values at a time, no branch on the common
        // path; the rare out-of-window column is read from X afterwards.
        auto step = [&](int code, A a, const Vec<S, CW> &lv) {
          if (code == -1) return;  // column outside [0, n_cols)
          Vec<S, CW> xv = lv;
          if (code < -1) xv = load_vec<S, CW>(Xc + static_cast<int64_t>(-2 - code) * ldx);
#pragma unroll
          for (int c = 0; c < CW; ++c) acc[c] = vmadd<V>(acc[c], a, xv.v[c]);
        };
        int64_t q = s - p0;
        const int64_t qe = e - p0;
        for (; q + 4 <= qe; q += 4) {
          int code[4];
          A au[4];
          Vec<S, CW> lv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            code[u] = cols[q + u];
            au[u] = V::widen(vals[q + u]);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u)
            lv[u] = __builtin_bit_cast(Vec<S, CW>, xs[((code[u] > 0 ? code[u] : 0) << lg) + l]);
#pragma unroll
          for (int u = 0; u < 4; ++u) step(code[u], au[u], lv[u]);
        }
        for (; q < qe; ++q) {
          const int code = cols[q];
          step(code, V::widen(vals[q]),
               __builtin_bit_cast(Vec<S, CW>, xs[((code > 0 ? code : 0) << lg) + l]));
        }
      } else {
        for (int64_t p = s; p < e; ++p) {
          const int64_t c = static_cast<int64_t>(indices[p]);
          if (static_cast<uint64_t>(c) < static_cast<uint64_t>(n_cols)) {
            const A a = V::widen(data[p]);
            const Vec<S, CW> xv = fetch(static_cast<int>(c));
#pragma unroll
            for (int cc = 0; cc < CW; ++cc) acc[cc] = vmadd<V>(acc[cc], a, xv.v[cc]);
          }
        }
      }
      if (col < k) {
        Vec<S, CW> out;
#pragma unroll
        for (int c = 0; c < CW; ++c) out.v[c] = V::narrow(acc[c]);
        store_vec<S, CW>(Y + row * ldy + col, out);
      }
    }
    __syncthreads();  // the next tile overwrites the staged data
  }
}

// ---------------------------------------------------------------------------
// Column windows on the matrix cores (float16 / bfloat16, k a multiple of
// 16).  One 256-thread workgroup per 32-row tile: the tile's values are
// scattered into a dense 32 x Kp block of its window in LDS (Kp: the
// plan's widest window rounded up to 32 columns), the window's X rows are
// staged row-major by buffer-to-LDS loads (no registers), each lane's MFMA
// operand of X comes from two transposing LDS reads (ds_read_b64_tr_b16:
// within 16 lanes, lane j's 4 values are element j % 4 of the addresses of
// lanes 4 t + j / 4, t = 0..3 - checked on gfx950), and v_mfma_f32_16x16x32 forms
// the 32 x k tile of Y with float32 accumulation (lane layout, checked on
// gfx950: A lane l holds row l % 16, k = 8 (l / 16) + 0..7; B lane l holds
// column l % 16, the same k; D lane l holds column l % 16, rows
// 4 (l / 16) + 0..3).  A product of two 16-bit values is exact in float32;
// the sums run in the matrix core's order, within the float16 / bfloat16
// tolerance of the reference's stored-order sum.  A tile with a repeated
// (row, column) pair, a column outside its window, row pointers outside
// the tile's range or a non-finite X value in its window takes the
// stored-order path from global memory instead (its result then equals the
// reference's).
typedef float MfmaAcc __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

template <class V>
struct Mfma16;
template <>
struct Mfma16<F16> {
  typedef _Float16 Vec8 __attribute__((ext_vector_type(8)));
  static constexpr uint16_t kInfBits = 0x7C00;  // magnitude bits >= this: inf or NaN
  __device__ static inline MfmaAcc mma(uint4 a, uint4 b, MfmaAcc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(Vec8, a),
                                                  __builtin_bit_cast(Vec8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma16<BF16> {
  typedef __bf16 Vec8 __attribute__((ext_vector_type(8)));
  static constexpr uint16_t kInfBits = 0x7F80;
  __device__ static inline MfmaAcc mma(uint4 a, uint4 b, MfmaAcc c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(Vec8, a),
                                                   __builtin_bit_cast(Vec8, b), c, 0, 0, 0);
  }
};

// Halves of padding per LDS row of the dense block and of the output: with
// Kp (or k) a multiple of 32 such a row is an odd number of 16-byte units
// long, so 8 consecutive rows start in 8 different groups of 4 banks (of
// 32) and stay 16-byte aligned for the operand reads.
constexpr int kMfmaPad = 8;
// Entries of one tile read through 32-bit descriptor offsets.
constexpr int64_t kMfmaTileEntries = int64_t{1} << 26;

// DPP moves within rows of 16 lanes (pure VALU): lane i takes lane i - 1
// (row_shr:1), or lane (i - 9) mod 16 (row_ror:9: lanes 0 and 8 take lanes 7
// and 15, the last lane of their group of 8).
template <int CTRL>
__device__ inline int64_t dpp_move(int64_t v) {
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), CTRL, 0xF, 0xF, false);
  return static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                              static_cast<uint32_t>(lo));
}
template <int CTRL>
__device__ inline int32_t dpp_move(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppShr1 = 0x111, kDppRor9 = 0x129;
// The X window in LDS: Kp rows of k halves, row-major, each row's 16-byte
// chunks permuted by a swizzle of the row (below).  The area afterwards holds
// the tile's output (kWinRows rows of k + kMfmaPad halves).
__host__ __device__ inline int64_t mfma_xt_halves(int64_t Kp, int64_t k) {
  const int64_t a = k * Kp, b = kWinRows * (k + kMfmaPad);
  return a > b ? a : b;
}

// Chunk c of window row r sits at chunk slot c ^ 2 x(r) of its row.  A
// transposing operand read takes 32 bytes (two chunks, an even pair) from
// each of 4 consecutive rows; x(r) in 0..3 moves those pairs into 4
// different 32-byte bank groups (of 128 bytes).  With P = CH / 2 pairs per
// row, rows already start in different groups for P < 4.
template <int CH>
__device__ inline int mfma_swizzle(int r) {
  constexpr int P = CH / 2;
  constexpr int S = P >= 4 ? 0 : (P == 2 ? 1 : 2);
  return 2 * ((r & 3) >> S);
}

typedef short MfmaHalf4 __attribute__((ext_vector_type(4)));

// LDS bytes of spmm_window_mfma for a padded window Kp and k columns.
__host__ __device__ inline int64_t mfma_window_lds(int64_t Kp, int64_t k) {
  return 2 * (kWinRows * (Kp + kMfmaPad) + mfma_xt_halves(Kp, k)) + 8 * (kWinRows + 2) +
         4 * kWinRows * (Kp / 32) + 16;
}

// k in {16, 32, 64, 128, 256}: LG = log2(k / 8), the 16-byte chunks of a row.
// Up to k = 64 the LDS admits 7 workgroups per CU; the register budget is
// held to match.
template <class V, class I, int LG>
__global__ void __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(LG <= 3 ? 7 : 1, 8)))
    spmm_window_mfma(const uint16_t *__restrict__ data, const I *__restrict__ indices,
                     const I *__restrict__ indptr, const uint16_t *__restrict__ X, int64_t ldx,
                     uint16_t *__restrict__ Y, int64_t ldy, int64_t n_rows, int64_t nnz,
                     int64_t n_cols, const int32_t *__restrict__ win, int64_t n_win, int Kp) {
  using A = typename V::Acc;
  constexpr int CH = 1 << LG;  // 16-byte chunks per X / Y row
  constexpr int K = 8 * CH;    // columns
  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int stride = Kp + kMfmaPad;    // dense block rows
  uint16_t *ad = reinterpret_cast<uint16_t *>(lds_raw);              // kWinRows x stride
  uint16_t *xt = ad + kWinRows * stride;                              // Kp x K, swizzled
  int64_t *rptr = reinterpret_cast<int64_t *>(xt + mfma_xt_halves(Kp, K));  // kWinRows + 1
  uint32_t *seen = reinterpret_cast<uint32_t *>(rptr + kWinRows + 2);  // kWinRows x Kp / 32
  int *flag = reinterpret_cast<int *>(seen + kWinRows * (Kp / 32));
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int words = Kp / 32;
  // staging: one buffer-to-LDS load per lane and step writes 16 bytes at
  // 16 * lane of its wave's destination, so a wave step covers 64 / CH rows
  // (lane: row lane / CH, chunk slot lane % CH)
  constexpr int kRowsPerLoad = kWave / CH;
  const int ld_row = lane / CH, ld_slot = lane % CH;
  for (int64_t t = xcd_remap(blockIdx.x, gridDim.x); t < n_win; t += gridDim.x) {
    const int64_t lo = win[2 * t];
    const int nw = static_cast<int>(std::min<int64_t>(
        Kp, std::max<int64_t>(0, static_cast<int64_t>(win[2 * t + 1]) - lo + 1)));
    const int64_t r0 = t * kWinRows;
    const int nr = static_cast<int>(std::min<int64_t>(kWinRows, n_rows - r0));
    // Loads through descriptors: whatever lies past a descriptor reads as
    // zero, so no load needs a branch and every load of this part is issued
    // before the first wait.  The tile's row pointers:
    const auto r_ptr = make_rsrc(indptr + r0, sizeof(I) * static_cast<uint64_t>(nr + 1));
    const I rp = buffer_index<I>(r_ptr, static_cast<uint32_t>(tid * sizeof(I)));
    // the window's X rows inside x (nv of them; rows past them read zero,
    // so the padded part of K adds nothing), two row pairs per thread and
    // step:
    const int64_t nv = std::max<int64_t>(0, std::min<int64_t>(nw, n_cols - lo));
    const auto r_x = make_rsrc(X + (nv > 0 ? lo : 0) * ldx, 2 * static_cast<uint64_t>(nv * ldx));
    const uint32_t row_bytes = static_cast<uint32_t>(2 * ldx);
    for (int i = tid; i < kWinRows * stride / 8; i += kThreads)
      reinterpret_cast<uint4 *>(ad)[i] = uint4{0, 0, 0, 0};
    if (tid == 0) {
      flag[0] = 0;  // the tile keeps the stored-order sum
      flag[1] = 0;  // some row's columns do not increase
    }
    // X window rows into LDS by buffer-to-LDS loads (no registers; rows past
    // the window's nv rows read zero, so the padded part of K adds nothing).
    for (int r0 = wave * kRowsPerLoad; r0 < Kp; r0 += (kThreads / kWave) * kRowsPerLoad) {
      const int r = r0 + ld_row;
      const uint32_t voff = static_cast<uint32_t>(r) * row_bytes +
                            16u * static_cast<uint32_t>(ld_slot ^ mfma_swizzle<CH>(r));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r_x, (__attribute__((address_space(3))) void *)(xt + r0 * K), 16, voff, 0, 0, 0);
    }
    if (tid <= nr) rptr[tid] = clamp64(static_cast<int64_t>(rp), 0, nnz);
    __builtin_amdgcn_s_waitcnt(0);  // the buffer-to-LDS loads have landed
    __syncthreads();
    {
      // A non-finite X value in the window would reach every row of the tile
      // through a zero of the dense block (0 x inf), so such a tile keeps the
      // stored-order sum: the largest magnitude bits of the window.
      u16x2 big = {0, 0};
      for (int i = tid; i < Kp * CH; i += kThreads) {
        const uint4 v = reinterpret_cast<const uint4 *>(xt)[i];
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          big = __builtin_elementwise_max(big, __builtin_bit_cast(u16x2, w4[j] & 0x7FFF7FFFu));
      }
      if ((big.x > big.y ? big.x : big.y) >= Mfma16<V>::kInfBits) flag[0] = 1;
    }
    // Values into the dense block, in stored order: 8 threads per row (lanes
    // 8 g .. 8 g + 7 of a wave), each taking kU entries (8 apart) per step,
    // all loaded before the first is placed (one memory round trip per
    // step).  Each entry's column is compared with the entry before it
    // (moved across lanes by DPP): when every row's columns increase, no
    // (row, column) pair repeats and the entries go straight to the block.
    const int ri = tid >> 3, j8 = tid & 7;
    int64_t rs = 0, re = 0;
    if (ri < nr) {
      rs = rptr[ri];
      re = std::max<int64_t>(rptr[ri + 1], rs);
    }
    // The tile's entries [q0, q1) through descriptors (offsets relative to
    // q0, so at most kMfmaTileEntries of them; a tile with more holds
    // repeated pairs and keeps the stored-order sum).
    const int64_t q0 = rptr[0], q1 = std::max<int64_t>(rptr[nr], q0);
    if (q1 - q0 > kMfmaTileEntries) {
      if (tid == 0) flag[0] = 1;
    } else if (ri < nr) {
      const auto r_ind = make_rsrc(indices + q0, sizeof(I) * static_cast<uint64_t>(q1 - q0));
      const auto r_dat = make_rsrc(data + q0, 2 * static_cast<uint64_t>(q1 - q0));
      constexpr int kU = 4;
      I cu[kU];
      uint16_t du[kU];
      bool unsorted = false;
      I carry = I{0};  // the previous step's last column of the lane
      auto load_entries = [&](int64_t qb) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int64_t q = qb + 8 * u;
          // rows out of [q0, q1) (decreasing row pointers) read zero and
          // are caught below
          const uint32_t e = static_cast<uint32_t>(q - q0);
          const I c = buffer_index<I>(r_ind, e * static_cast<uint32_t>(sizeof(I)));
          const uint16_t v = static_cast<uint16_t>(__builtin_amdgcn_raw_buffer_load_b16(r_dat, 2 * e, 0, 0));
          cu[u] = q < re ? c : I{-1};
          du[u] = v;
        }
      };
      auto place = [&](int64_t qb) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int64_t q = qb + 8 * u;
          // the entry before q: lane j8 - 1's, or for j8 = 0 lane 7's of the
          // step before.  Both moves run on every lane (a lane reads only
          // lanes that run the move with it).
          const I from_left = dpp_move<kDppShr1>(cu[u]);
          const I from_last = dpp_move<kDppRor9>(u > 0 ? cu[u > 0 ? u - 1 : 0] : carry);
          const I before = j8 > 0 ? from_left : from_last;
          if (q < re && q > rs && static_cast<int64_t>(cu[u]) <= static_cast<int64_t>(before))
            unsorted = true;
          const int64_t c = static_cast<int64_t>(cu[u]);
          // past the row, or out of range: adds nothing
          if (static_cast<uint64_t>(c) >= static_cast<uint64_t>(n_cols)) continue;
          const int64_t w = c - lo;
          if (static_cast<uint64_t>(w) >= static_cast<uint64_t>(nw)) {
            flag[0] = 1;
            continue;
          }
          ad[ri * stride + static_cast<int>(w)] = du[u];
        }
        carry = cu[kU - 1];
      };
      // the same number of steps on the row's 8 lanes (the moves read them)
      for (int64_t qb = rs + j8; qb - j8 < re; qb += 8 * kU) {
        load_entries(qb);
        place(qb);
      }
      if (unsorted) flag[1] = 1;
      // row pointers that decrease or leave the tile's range: stored order
      if (j8 == 0 && (rs < rptr[0] || rptr[ri + 1] < rs)) flag[0] = 1;
    }
    __syncthreads();
    if (flag[1] && !flag[0]) {
      // Some row's columns do not increase: look for a repeated (row,
      // column) pair with a bitmap of the dense block.
      for (int i = tid; i < kWinRows * words; i += kThreads) seen[i] = 0;
      __syncthreads();
      if (ri < nr) {
        for (int64_t q = rs + j8; q < re; q += 8) {
          const int64_t c = static_cast<int64_t>(indices[q]);
          const int64_t w = c - lo;
          if (static_cast<uint64_t>(c) >= static_cast<uint64_t>(n_cols) ||
              static_cast<uint64_t>(w) >= static_cast<uint64_t>(nw))
            continue;
          const uint32_t bit = 1u << (w & 31);
          if (atomicOr(&seen[ri * words + static_cast<int>(w >> 5)], bit) & bit) flag[0] = 1;
        }
      }
    }
    __syncthreads();
    if (flag[0]) {
      // Stored order from global memory, 8 columns per thread.
      for (int q = tid; q < nr * CH; q += kThreads) {
        const int i = q >> LG;
        const int cc = (q & (CH - 1)) * 8;
        const int64_t s = rptr[i];
        const int64_t e = std::max<int64_t>(rptr[i + 1], s);
        A acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = vzero<A>();
        for (int64_t p = s; p < e; ++p) {
          const int64_t c = static_cast<int64_t>(indices[p]);
          if (static_cast<uint64_t>(c) >= static_cast<uint64_t>(n_cols)) continue;
          const A a = V::widen(data[p]);
          const uint4 v = *reinterpret_cast<const uint4 *>(X + c * ldx + cc);
          const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int j = 0; j < 8; ++j)
            acc[j] = vmadd<V>(acc[j], a, static_cast<uint16_t>(w4[j / 2] >> (16 * (j & 1))));
        }
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = static_cast<uint32_t>(V::narrow(acc[2 * j])) |
                 (static_cast<uint32_t>(V::narrow(acc[2 * j + 1])) << 16);
        *reinterpret_cast<uint4 *>(Y + (r0 + i) * ldy + cc) = uint4{o[0], o[1], o[2], o[3]};
      }
      __syncthreads();
      continue;
    }
    // Matrix cores: 2 x (K / 16) output blocks of 16 x 16 over the waves,
    // each wave keeping its blocks' accumulators (a lane holds four rows of
    // one column); the tile then goes through LDS (the transposed-X area,
    // free once every wave is done) and out as 16-byte row segments.
    constexpr int kBlocks = 2 * (K / 16);
    constexpr int kWaves = kThreads / kWave;
    constexpr int kPerWave = (kBlocks + kWaves - 1) / kWaves;
    const int lr = lane % 16, lk = 8 * (lane / 16);
    // B operand of lane (k-group gq = lane / 16, column n = lane % 16): two
    // transposing reads of 4 rows each; the lane's address is row
    // kk + 8 gq + 4 h + n / 4, columns 16 cb + 4 (n % 4) .. + 3, and the read
    // hands it rows kk + 8 gq + 4 h + 0..3 of column 16 cb + n.
    const int b_row = 8 * (lane / 16) + (lr >> 2);
    const int b_col = 4 * (lr & 3);
    auto b_read = [&](int row, int col) {
      const int c = col >> 3;
      const int off = row * (2 * K) + 16 * (c ^ mfma_swizzle<CH>(row)) + 2 * (col & 7);
      return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) MfmaHalf4 *)(reinterpret_cast<unsigned char *>(xt) + off));
    };
    MfmaAcc accs[kPerWave];
#pragma unroll
    for (int b = 0; b < kPerWave; ++b) {
      const int blk = wave + kWaves * b;
      accs[b] = MfmaAcc{0.f, 0.f, 0.f, 0.f};
      if (blk < kBlocks) {
        const int rb = blk & 1, cb = blk >> 1;
        const uint16_t *arow = ad + (rb * 16 + lr) * stride + lk;
        for (int kk = 0; kk < Kp; kk += 32) {
          const MfmaHalf4 lo4 = b_read(kk + b_row, 16 * cb + b_col);
          const MfmaHalf4 hi4 = b_read(kk + b_row + 4, 16 * cb + b_col);
          const uint2 l2 = __builtin_bit_cast(uint2, lo4), h2 = __builtin_bit_cast(uint2, hi4);
          const uint4 bv{l2.x, l2.y, h2.x, h2.y};
          accs[b] = Mfma16<V>::mma(*reinterpret_cast<const uint4 *>(arow + kk), bv, accs[b]);
        }
      }
    }
    __syncthreads();
    constexpr int KY = K + kMfmaPad;  // output row stride (staggers the banks)
    uint16_t *yb = xt;                // kWinRows x KY
#pragma unroll
    for (int b = 0; b < kPerWave; ++b) {
      const int blk = wave + kWaves * b;
      if (blk < kBlocks) {
        const int rb = blk & 1, cb = blk >> 1;
#pragma unroll
        for (int v = 0; v < 4; ++v)
          yb[(rb * 16 + 4 * (lane / 16) + v) * KY + cb * 16 + lr] = V::narrow(accs[b][v]);
      }
    }
    __syncthreads();
    for (int q = tid; q < nr * CH; q += kThreads) {
      const int i = q >> LG;
      const int cc = (q & (CH - 1)) * 8;
      *reinterpret_cast<uint4 *>(Y + (r0 + i) * ldy + cc) =
          *reinterpret_cast<const uint4 *>(yb + i * KY + cc);
    }
    __syncthreads();  // the next tile overwrites the staged data
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }



template <class V, class I>
msx_status spmm_typed(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data_v,
                      const void *indices_v, const void *indptr_v, int64_t batch, int64_t k,
                      const void *X_v, int64_t x_batch, int64_t ldx, void *Y_v, int64_t y_batch,
                      int64_t ldy, const msx_csr_plan *plan, bool y_nt, hipStream_t stream) {
  using S = typename V::Storage;
  constexpr int CWV = static_cast<int>(16 / sizeof(S));
  const auto *data = static_cast<const S *>(data_v);
  const auto *indices = static_cast<const I *>(indices_v);
  const auto *indptr = static_cast<const I *>(indptr_v);
  const auto *X = static_cast<const S *>(X_v);
  auto *Y = static_cast<S *>(Y_v);
  const bool vec = (k % CWV) == 0 && (ldx % CWV) == 0 && (ldy % CWV) == 0 &&
                   (x_batch % CWV) == 0 && (y_batch % CWV) == 0 && aligned16(X) && aligned16(Y);
  // X rows of exactly two cache lines (k = 64 float32, 128 float16/bfloat16,
  // 32 complex64): one line per group of four XCDs.  Measured on the 3D
  // Poisson matrix at k = 64: 468 us against 493 us for spmm_rows; at four or
  // eight lines per row the extra reads of the matrix cancel the gain.
  const int64_t row_bytes = k * static_cast<int64_t>(sizeof(S));
  // Column windows of a bound plan: every tile's window of X, its values
  // and row pointers in LDS.
  if constexpr (std::is_same_v<V, F16> || std::is_same_v<V, BF16>) {
    // 16-bit values, k = 16 .. 256 a power of two: the matrix-core window
    // kernel.
    const int lg = k == 16 ? 1 : k == 32 ? 2 : k == 64 ? 3 : k == 128 ? 4 : k == 256 ? 5 : 0;
    if (vec && batch == 1 && plan != nullptr && plan->win_rows_max > 0 &&
        plan->n_win == (n_rows + kWinRows - 1) / kWinRows && lg > 0) {
      const int64_t Kp = (plan->win_rows_max + 31) / 32 * 32;
      const int64_t lds = mfma_window_lds(Kp, k);
      // the kernel reads a window of Kp rows of X through one descriptor
      if (lds <= kWinLdsBytes && static_cast<uint64_t>(Kp + 1) * 2 * ldx <= kGatherMaxBytes) {
        const uint32_t grid = static_cast<uint32_t>(std::min<int64_t>(plan->n_win, kMaxGrid));
        auto go = [&](auto kern) {
          hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), static_cast<size_t>(lds), stream,
                             data, indices, indptr, X, ldx, Y, ldy, n_rows, nnz, n_cols,
                             plan->win, plan->n_win, static_cast<int>(Kp));
        };
        switch (lg) {
        case 1: go(spmm_window_mfma<V, I, 1>); break;
        case 2: go(spmm_window_mfma<V, I, 2>); break;
        case 3: go(spmm_window_mfma<V, I, 3>); break;
        case 4: go(spmm_window_mfma<V, I, 4>); break;
        default: go(spmm_window_mfma<V, I, 5>); break;
        }
        MSX_HIP_TRY(hipGetLastError());
        return MSX_OK;
      }
    }
  }
  if (vec && batch == 1 && plan != nullptr && plan->win_rows_max > 0 &&
      plan->n_win == (n_rows + kWinRows - 1) / kWinRows && k <= int64_t{kWave} * CWV) {
    int LR = 1;
    while (LR * CWV < k) LR <<= 1;
    const int64_t tile_cap = plan->win_nnz_max;
    const int64_t cap4 = (tile_cap + 3) & ~int64_t{3};
    const int64_t lds = plan->win_rows_max * LR * 16 + (kWinRows + 2) * 8 +
                        cap4 * static_cast<int64_t>(sizeof(typename V::Storage) + 4);
    if (lds <= kWinLdsBytes) {
      const uint32_t grid = static_cast<uint32_t>(std::min<int64_t>(plan->n_win, kMaxGrid));
      hipLaunchKernelGGL((spmm_window<V, I, CWV>), dim3(grid), dim3(kThreads),
                         static_cast<size_t>(lds), stream, data, indices, indptr, X, ldx, Y, ldy,
                         n_rows, nnz, n_cols, k, LR, plan->win, plan->n_win, plan->win_rows_max,
                         tile_cap);
      MSX_HIP_TRY(hipGetLastError());
      return MSX_OK;
    }
  }
  const int G = static_cast<int>(row_bytes / 128);
  if (vec && row_bytes == 256) {
    constexpr int LRT = 128 / 16;
    const int64_t n_rt = (n_rows + kThreads / LRT - 1) / (kThreads / LRT);
    const int64_t per_group = (n_rt + (kNumXcd / G) - 1) / (kNumXcd / G);
    const int64_t slots = std::max<int64_t>(1, std::min<int64_t>(per_group, kMaxGrid / kNumXcd));
    // The grid's x extent is a multiple of 8, so workgroup (x, b) still runs
    // on XCD x % 8 when batches are stacked along y.
    for (int64_t b0 = 0; b0 < batch; b0 += kMaxBatchGrid) {
      const uint32_t nb = static_cast<uint32_t>(std::min<int64_t>(batch - b0, kMaxBatchGrid));
      auto kern = y_nt ? spmm_linetile<V, I, CWV, true> : spmm_linetile<V, I, CWV, false>;
      hipLaunchKernelGGL(kern, dim3(static_cast<uint32_t>(slots * kNumXcd), nb),
                         dim3(kThreads), 0, stream, data, indices, indptr, X + b0 * x_batch, ldx,
                         Y + b0 * y_batch, ldy, n_rows, nnz, n_cols, G, x_batch, y_batch);
      MSX_HIP_TRY(hipGetLastError());
    }
    return MSX_OK;
  }
  const int CW = vec ? CWV : 1;
  const int64_t lanes = (k + CW - 1) / CW;
  int LR = 1;
  while (LR < lanes && LR < 64) LR <<= 1;
  const int64_t n_col_tiles = (k + static_cast<int64_t>(LR) * CW - 1) / (static_cast<int64_t>(LR) * CW);
  const int64_t rows_per_group = kThreads / LR;
  const int64_t tiles = ((n_rows + rows_per_group - 1) / rows_per_group) * n_col_tiles;
  const uint32_t grid = static_cast<uint32_t>(std::max<int64_t>(1, std::min<int64_t>(tiles, kMaxGrid)));
  for (int64_t b0 = 0; b0 < batch; b0 += kMaxBatchGrid) {
    const uint32_t nb = static_cast<uint32_t>(std::min<int64_t>(batch - b0, kMaxBatchGrid));
    const S *Xb = X + b0 * x_batch;
    S *Yb = Y + b0 * y_batch;
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(grid, nb), dim3(kThreads), 0, stream, data, indices, indptr, Xb,
                         ldx, Yb, ldy, n_rows, nnz, n_cols, k, LR, n_col_tiles, x_batch, y_batch);
    };
    if (vec) {
      auto go = [&](auto nt) {
        constexpr bool NT = decltype(nt)::value;
        switch (LR) {
        case 1: launch(spmm_rows<V, I, CWV, false, 1, NT>); break;
        case 2: launch(spmm_rows<V, I, CWV, false, 2, NT>); break;
        case 4: launch(spmm_rows<V, I, CWV, false, 4, NT>); break;
        case 8: launch(spmm_rows<V, I, CWV, true, 8, NT>); break;
        case 16: launch(spmm_rows<V, I, CWV, true, 16, NT>); break;
        case 32: launch(spmm_rows<V, I, CWV, true, 32, NT>); break;
        default: launch(spmm_rows<V, I, CWV, true, 64, NT>); break;
        }
      };
      if (y_nt) go(std::true_type{});
      else go(std::false_type{});
    } else {
      if (LR >= kChunk) launch(spmm_rows<V, I, 1, true>);
      else launch(spmm_rows<V, I, 1, false>);
    }
    MSX_HIP_TRY(hipGetLastError());
  }
  return MSX_OK;
}

template <class V>
msx_status spmm_vt(msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                   const void *indices, const void *indptr, int64_t batch, int64_t k, const void *X,
                   int64_t x_batch, int64_t ldx, void *Y, int64_t y_batch, int64_t ldy,
                   const msx_csr_plan *plan, bool y_nt, hipStream_t stream) {
  if (it == MSX_I32)
    return spmm_typed<V, int32_t>(n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch,
                                  ldx, Y, y_batch, ldy, plan, y_nt, stream);
  return spmm_typed<V, int64_t>(n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch,
                                ldx, Y, y_batch, ldy, plan, y_nt, stream);
}

template <class I>
msx_status windows_typed(msx_csr_plan *p, const void *indices, const void *indptr,
                         hipStream_t stream) {
  const int64_t n_win = (p->n_rows + kWinRows - 1) / kWinRows;
  if (n_win == 0 || p->nnz == 0) return MSX_OK;
  const size_t b_win = (static_cast<size_t>(2 * n_win) * sizeof(int32_t) + 255) / 256 * 256;
  char *base = nullptr;
  if (hipMalloc(&base, b_win + 256) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MSX_ENOMEM, "msx_csr_plan_create_bound: device allocation of the column windows failed.");
  }
  p->win = reinterpret_cast<int32_t *>(base);
  p->win_bytes = b_win + 256;
  auto *widest = reinterpret_cast<unsigned long long *>(base + b_win);
  MSX_HIP_TRY(hipMemsetAsync(widest, 0, 2 * sizeof(*widest), stream));
  const int64_t groups =
      std::min<int64_t>((n_win + kThreads / kWave - 1) / (kThreads / kWave), 2048);
  hipLaunchKernelGGL((window_bounds<I>), dim3(static_cast<uint32_t>(groups)), dim3(kThreads), 0,
                     stream, static_cast<const I *>(indices), static_cast<const I *>(indptr),
                     p->n_rows, p->nnz, p->n_cols, n_win, p->win, widest);
  MSX_HIP_TRY(hipGetLastError());
  unsigned long long w[2] = {0, 0};
  MSX_HIP_TRY(hipMemcpyAsync(w, widest, sizeof(w), hipMemcpyDeviceToHost, stream));
  MSX_HIP_TRY(hipStreamSynchronize(stream));
  p->n_win = n_win;
  p->win_rows_max = static_cast<int64_t>(w[0]);
  p->win_nnz_max = static_cast<int64_t>(w[1]);
  return MSX_OK;
}

}  // namespace

namespace {
msx_status spmm_dispatch(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz,
                         const void *data, const void *indices, const void *indptr, int64_t batch,
                         int64_t k, const void *X, int64_t x_batch, int64_t ldx, void *Y,
                         int64_t y_batch, int64_t ldy, const msx_csr_plan *plan, bool y_nt,
                         hipStream_t stream) {
  if (batch <= 0 || n_rows <= 0 || k <= 0) return MSX_OK;
  switch (vt) {
  case MSX_F32:
    return spmm_vt<F32>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                        Y, y_batch, ldy, plan, y_nt, stream);
  case MSX_F16:
    return spmm_vt<F16>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                        Y, y_batch, ldy, plan, y_nt, stream);
  case MSX_BF16:
    return spmm_vt<BF16>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                         Y, y_batch, ldy, plan, y_nt, stream);
  case MSX_C64:
    return spmm_vt<C64>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                        Y, y_batch, ldy, plan, y_nt, stream);
  }
  return fail(MSX_ETYPE, "csr_matmul unsupported value dtype.");
}
}  // namespace

msx_status launch_spmm_batched(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                               int64_t nnz, const void *data, const void *indices,
                               const void *indptr, int64_t batch, int64_t k, const void *X,
                               int64_t x_batch, int64_t ldx, void *Y, int64_t y_batch, int64_t ldy,
                               bool y_nt, hipStream_t stream) {
  return spmm_dispatch(vt, it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch,
                       ldx, Y, y_batch, ldy, nullptr, y_nt, stream);
}

template <class V, class I>
bool batch_rows_typed(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                      const void *indices, const void *indptr, const void *Xt, int64_t kpad,
                      void *Y, int64_t ldy, int64_t batch, hipStream_t stream) {
  using S = typename V::Storage;
  constexpr int CW = static_cast<int>(16 / sizeof(S));
  if (kpad % CW != 0 || (reinterpret_cast<uintptr_t>(Xt) & 15u) != 0) return false;
  const int64_t LR = kpad / CW;
  if (LR != 1 && LR != 2 && LR != 4 && LR != 8) return false;
  const int64_t rows_per_group = kThreads / LR;
  const int64_t tiles = (n_rows + rows_per_group - 1) / rows_per_group;
  const uint32_t grid = static_cast<uint32_t>(std::max<int64_t>(1, std::min<int64_t>(tiles, kMaxGrid)));
  const auto *d = static_cast<const S *>(data);
  const auto *ix = static_cast<const I *>(indices);
  const auto *ip = static_cast<const I *>(indptr);
  const auto *x = static_cast<const S *>(Xt);
  auto *y = static_cast<S *>(Y);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), 0, stream, d, ix, ip, x, kpad, y, ldy,
                       batch, n_rows, nnz, n_cols);
  };
  switch (LR) {
  case 1: go(spmv_batch_rows<V, I, CW, 1>); break;
  case 2: go(spmv_batch_rows<V, I, CW, 2>); break;
  case 4: go(spmv_batch_rows<V, I, CW, 4>); break;
  default: go(spmv_batch_rows<V, I, CW, 8>); break;
  }
  return true;
}

template <class V>
bool batch_rows_vt(msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                   const void *indices, const void *indptr, const void *Xt, int64_t kpad, void *Y,
                   int64_t ldy, int64_t batch, hipStream_t stream) {
  return it == MSX_I32 ? batch_rows_typed<V, int32_t>(n_rows, n_cols, nnz, data, indices, indptr,
                                                       Xt, kpad, Y, ldy, batch, stream)
                       : batch_rows_typed<V, int64_t>(n_rows, n_cols, nnz, data, indices, indptr,
                                                       Xt, kpad, Y, ldy, batch, stream);
}

msx_status launch_spmv_batch_rows(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                                  int64_t nnz, const void *data, const void *indices,
                                  const void *indptr, const void *Xt, int64_t kpad, void *Y,
                                  int64_t ldy, int64_t batch, hipStream_t stream, bool *done) {
  bool ok = false;
  switch (vt) {
  case MSX_F32: ok = batch_rows_vt<F32>(it, n_rows, n_cols, nnz, data, indices, indptr, Xt, kpad, Y, ldy, batch, stream); break;
  case MSX_F16: ok = batch_rows_vt<F16>(it, n_rows, n_cols, nnz, data, indices, indptr, Xt, kpad, Y, ldy, batch, stream); break;
  case MSX_BF16: ok = batch_rows_vt<BF16>(it, n_rows, n_cols, nnz, data, indices, indptr, Xt, kpad, Y, ldy, batch, stream); break;
  case MSX_C64: ok = batch_rows_vt<C64>(it, n_rows, n_cols, nnz, data, indices, indptr, Xt, kpad, Y, ldy, batch, stream); break;
  }
  *done = ok;
  if (ok) MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

msx_status build_windows(msx_csr_plan *p, const void *indices, const void *indptr,
                         hipStream_t stream) {
  return p->itype == MSX_I32 ? windows_typed<int32_t>(p, indices, indptr, stream)
                             : windows_typed<int64_t>(p, indices, indptr, stream);
}

msx_status launch_spmm(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz,
                       const void *data, const void *indices, const void *indptr, int64_t k,
                       const void *X, int64_t ldx, void *Y, int64_t ldy, const msx_csr_plan *plan,
                       hipStream_t stream) {
  return spmm_dispatch(vt, it, n_rows, n_cols, nnz, data, indices, indptr, 1, k, X, 0, ldx, Y, 0,
                       ldy, plan, true, stream);
}

}  // namespace msx
