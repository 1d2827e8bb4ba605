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

template <class S, int CW>
__device__ inline void store_vec(S *p, const Vec<S, CW> &v) {
  if constexpr (CW * sizeof(S) == 16) {
    *reinterpret_cast<uint4 *>(p) = __builtin_bit_cast(uint4, v);
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

// Y-row segment [col, col + CW) of row [s, e): sum from zero in stored order.
// The row's group is LR lanes wide (lane l of it); every lane of the group
// calls this with the same s and e.  SHUF: LR >= kChunk, a chunk of kChunk
// values is loaded one value per lane and shared by shuffles; otherwise every
// lane loads the values itself, kUnrollDirect per step (narrow groups, small
// k: measured faster there than whole chunks).  Columns outside [0, n_cols)
// add nothing.
template <class V, class I, int CW, bool SHUF>
__device__ inline void row_segment(const typename V::Storage *__restrict__ data,
                                   const I *__restrict__ indices, const typename V::Storage *__restrict__ X,
                                   int64_t ldx, int64_t n_cols, int64_t s, int64_t e, int64_t col, int l,
                                   int LR, typename V::Acc (&acc)[CW]) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  // Positions stay 64-bit: 32-bit ones measured 15 % slower here (the
  // address arithmetic of the index and value loads).
  const auto *Xc = X + col;
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
        if (cu[u] >= 0) xv[u] = load_vec<S, CW>(Xc + static_cast<int64_t>(cu[u]) * ldx);
#pragma unroll
      for (int u = 0; u < kUnrollDirect; ++u)
        if (cu[u] >= 0) {
#pragma unroll
          for (int c = 0; c < CW; ++c) acc[c] = vadd(acc[c], vmul_acc<V>(au[u], xv[u].v[c]));
        }
    }
    for (; p < e; ++p) {
      const I c = indices[p];
      if (static_cast<uint64_t>(static_cast<int64_t>(c)) < static_cast<uint64_t>(n_cols)) {
        const A a = V::widen(data[p]);
        const Vec<S, CW> xv = load_vec<S, CW>(Xc + static_cast<int64_t>(c) * ldx);
#pragma unroll
        for (int q = 0; q < CW; ++q) acc[q] = vadd(acc[q], vmul_acc<V>(a, xv.v[q]));
      }
    }
    return;
  }
  for (int64_t b = s; b < e; b += kChunk) {
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
      if (cu[u] >= 0) xv[u] = load_vec<S, CW>(Xc + static_cast<int64_t>(cu[u]) * ldx);
#pragma unroll
    for (int u = 0; u < kChunk; ++u)
      if (cu[u] >= 0) {
#pragma unroll
        for (int c = 0; c < CW; ++c) acc[c] = vadd(acc[c], vmul_acc<V>(au[u], xv[u].v[c]));
      }
  }
}

template <class V, class I, int CW, bool SHUF>
__global__ void __launch_bounds__(kThreads)
    spmm_rows(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
              const I *__restrict__ indptr, const typename V::Storage *__restrict__ X,
              int64_t ldx, typename V::Storage *__restrict__ Y, int64_t ldy, int64_t n_rows,
              int64_t nnz, int64_t n_cols, int64_t k, int LR, int64_t n_col_tiles, int64_t x_batch,
              int64_t y_batch) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  X += blockIdx.y * x_batch;  // batch blockIdx.y (one for a plain SpMM)
  Y += blockIdx.y * y_batch;
  const int rows_per_group = kThreads / LR;
  const int g = threadIdx.x / LR;
  const int l = threadIdx.x % LR;
  const int64_t tile_cols = static_cast<int64_t>(LR) * CW;
  const int64_t n_row_tiles = (n_rows + rows_per_group - 1) / rows_per_group;
  const int64_t n_tiles = n_row_tiles * n_col_tiles;
  for (int64_t t = xcd_remap(blockIdx.x, gridDim.x); t < n_tiles; t += gridDim.x) {
    const int64_t rt = t / n_col_tiles;
    const int64_t ct = t - rt * n_col_tiles;
    const int64_t row = rt * rows_per_group + g;
    const int64_t col = ct * tile_cols + static_cast<int64_t>(l) * CW;
    if (row >= n_rows) continue;
    const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    A acc[CW];
    // Lanes past k still take part in the shuffles; they read column 0.
    row_segment<V, I, CW, SHUF>(data, indices, X, ldx, n_cols, s, e, col < k ? col : 0, l, LR, acc);
    if (col >= k) continue;
    Vec<S, CW> out;
#pragma unroll
    for (int c = 0; c < CW; ++c) out.v[c] = V::narrow(acc[c]);
    store_vec<S, CW>(Y + row * ldy + col, out);
  }
}

// Line-tiled SpMM for X rows of G whole 128-byte cache lines.  XCD x
// (workgroup g runs on XCD g % 8) owns column tile x % G (one line) and a
// contiguous G/8 share of the rows.  Each XCD then keeps only its own line of
// every X row in its L2, halving (G = 2) the X window that a stencil's far
// neighbours need, at the cost of reading each row's indices/data G times.
// Sums per column are in stored order, as in spmm_rows.
template <class V, class I, int CW>
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
    row_segment<V, I, CW, true>(data, indices, X, ldx, n_cols, s, e, col, l, LR, acc);
    Vec<S, CW> out;
#pragma unroll
    for (int c = 0; c < CW; ++c) out.v[c] = V::narrow(acc[c]);
    store_vec<S, CW>(Y + row * ldy + col, out);
  }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }



template <class V, class I>
msx_status spmm_typed(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data_v,
                      const void *indices_v, const void *indptr_v, int64_t batch, int64_t k,
                      const void *X_v, int64_t x_batch, int64_t ldx, void *Y_v, int64_t y_batch,
                      int64_t ldy, hipStream_t stream) {
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
      hipLaunchKernelGGL((spmm_linetile<V, I, CWV>), dim3(static_cast<uint32_t>(slots * kNumXcd), nb),
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
      if (LR >= kChunk) launch(spmm_rows<V, I, CWV, true>);
      else launch(spmm_rows<V, I, CWV, false>);
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
                   hipStream_t stream) {
  if (it == MSX_I32)
    return spmm_typed<V, int32_t>(n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch,
                                  ldx, Y, y_batch, ldy, stream);
  return spmm_typed<V, int64_t>(n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch,
                                ldx, Y, y_batch, ldy, stream);
}

}  // namespace

msx_status launch_spmm_batched(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                               int64_t nnz, const void *data, const void *indices,
                               const void *indptr, int64_t batch, int64_t k, const void *X,
                               int64_t x_batch, int64_t ldx, void *Y, int64_t y_batch, int64_t ldy,
                               hipStream_t stream) {
  if (batch <= 0 || n_rows <= 0 || k <= 0) return MSX_OK;
  switch (vt) {
  case MSX_F32:
    return spmm_vt<F32>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                        Y, y_batch, ldy, stream);
  case MSX_F16:
    return spmm_vt<F16>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                        Y, y_batch, ldy, stream);
  case MSX_BF16:
    return spmm_vt<BF16>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                         Y, y_batch, ldy, stream);
  case MSX_C64:
    return spmm_vt<C64>(it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X, x_batch, ldx,
                        Y, y_batch, ldy, stream);
  }
  return fail(MSX_ETYPE, "csr_matmul unsupported value dtype.");
}

msx_status launch_spmm(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz,
                       const void *data, const void *indices, const void *indptr, int64_t k,
                       const void *X, int64_t ldx, void *Y, int64_t ldy, hipStream_t stream) {
  return launch_spmm_batched(vt, it, n_rows, n_cols, nnz, data, indices, indptr, 1, k, X, 0, ldx, Y,
                             0, ldy, stream);
}

}  // namespace msx
