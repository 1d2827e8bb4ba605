// csr_batched.hip - CSR products with a batch of right-hand sides.
//
//   batched SpMV:  Y[b, i] = sum_p data[p] * X[b, indices[p]]       (X: batch x n_cols)
//   batched SpMM:  Y[b][i, c] = sum_p data[p] * X[b][indices[p], c]  (X[b]: n_cols x k)
//
// Each output element is summed from zero in stored order, as the
// reference's batched CPU kernels sum it (reference:
// src/sparse/csr_batched_matvec/csr_batched_matvec.cpp, csr_batched_matvec_cpu_impl;
// src/sparse/csr_batched_matmul/csr_batched_matmul.cpp, the generic and
// small-k CPU impls) - the rule of the SpMM kernels, so float32 results equal
// the reference bit for bit.
//
// Batched SpMM stacks the batches along the grid's y extent of the SpMM
// kernels.  Batched SpMV transposes the vectors into the columns of one
// n_cols x B matrix (padded to a 16-byte row), runs one SpMM - the matrix is
// read once and each gather fetches all B values of a column together - and
// transposes the n_rows x B result back.  The two scratch matrices come from
// the stream-ordered allocator of `stream`.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "msx_device.h"
#include "msx_internal.h"
#include "msx_sparse.h"

namespace msx {
namespace {

constexpr int kTile = 32;
constexpr int kThreads = 256;
constexpr int64_t kIntMax = 2147483647;
constexpr int64_t kMaxGrid = int64_t{1} << 20;

// out[c * ldo + r] = in[r * ldi + c] for r < rows, c < cols, and zero for
// rows <= r < rows_pad.  32 x 32 tiles through LDS (one padding column
// against bank conflicts), tiles visited by a grid-stride loop.
template <class T>
__global__ void __launch_bounds__(kThreads)
    transpose_tiles(const T *__restrict__ in, int64_t rows, int64_t rows_pad, int64_t cols,
                    int64_t ldi, T *__restrict__ out, int64_t ldo) {
  __shared__ T tile[kTile][kTile + 1];
  const int tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
  const int64_t tiles_c = (cols + kTile - 1) / kTile;
  const int64_t tiles_r = (rows_pad + kTile - 1) / kTile;
  for (int64_t t = blockIdx.x; t < tiles_c * tiles_r; t += gridDim.x) {
    const int64_t r0 = (t / tiles_c) * kTile, c0 = (t % tiles_c) * kTile;
    for (int j = ty; j < kTile; j += kThreads / kTile) {
      const int64_t r = r0 + j, c = c0 + tx;
      tile[j][tx] = (r < rows && c < cols) ? in[r * ldi + c] : T{};
    }
    __syncthreads();
    for (int j = ty; j < kTile; j += kThreads / kTile) {
      const int64_t c = c0 + j, r = r0 + tx;
      if (c < cols && r < rows_pad) out[c * ldo + r] = tile[tx][j];
    }
    __syncthreads();
  }
}

// Narrow transposes for batches of at most kNarrow vectors (padded width
// kpad, a multiple of the 16-byte vector): one thread per column of the
// batch, 16-byte accesses on the transposed side, one coalesced access per
// vector on the other - no LDS, every load and store fully used.
constexpr int kNarrow = 32;

template <class T>
union Vec16 {
  uint4 u;
  T e[16 / sizeof(T)];
};

// Xt[c * kpad + b] = X[b * ldx + c] (b < batch), 0 for batch <= b < kpad.
template <class T>
__global__ void __launch_bounds__(kThreads)
    gather_columns(const T *__restrict__ X, int64_t batch, int64_t kpad, int64_t n, int64_t ldx,
                   T *__restrict__ Xt) {
  constexpr int E = 16 / sizeof(T);
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; c < n;
       c += static_cast<int64_t>(gridDim.x) * kThreads) {
    uint4 *out = reinterpret_cast<uint4 *>(Xt + c * kpad);
    for (int64_t q = 0; q < kpad / E; ++q) {
      Vec16<T> v;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int64_t b = q * E + e;
        v.e[e] = b < batch ? X[b * ldx + c] : T{};
      }
      out[q] = v.u;
    }
  }
}

// Y[b * ldy + r] = Yt[r * kpad + b] for b < batch.
template <class T>
__global__ void __launch_bounds__(kThreads)
    scatter_rows(const T *__restrict__ Yt, int64_t batch, int64_t kpad, int64_t n, int64_t ldy,
                 T *__restrict__ Y) {
  constexpr int E = 16 / sizeof(T);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r < n;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint4 *in = reinterpret_cast<const uint4 *>(Yt + r * kpad);
    for (int64_t q = 0; q < kpad / E; ++q) {
      Vec16<T> v;
      v.u = in[q];
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int64_t b = q * E + e;
        if (b < batch) Y[b * ldy + r] = v.e[e];
      }
    }
  }
}

// The same transposes with the number of 16-byte vectors per column, Q, a
// constant: every load of a thread is issued before its first store (with
// a runtime Q the compiler waited for each vector's loads in turn).  A lane
// past `batch` loads element batch - 1 and stores zero.
template <class T, int Q>
__global__ void __launch_bounds__(kThreads)
    gather_columns_q(const T *__restrict__ X, int64_t batch, int64_t n, int64_t ldx,
                     T *__restrict__ Xt) {
  constexpr int E = 16 / sizeof(T);
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; c < n;
       c += static_cast<int64_t>(gridDim.x) * kThreads) {
    Vec16<T> v[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int64_t b = q * E + e;
        const T t = X[(b < batch ? b : batch - 1) * ldx + c];
        v[q].e[e] = b < batch ? t : T{};
      }
    uint4 *out = reinterpret_cast<uint4 *>(Xt + c * (Q * E));
#pragma unroll
    for (int q = 0; q < Q; ++q) out[q] = v[q].u;
  }
}

template <class T, int Q>
__global__ void __launch_bounds__(kThreads)
    scatter_rows_q(const T *__restrict__ Yt, int64_t batch, int64_t n, int64_t ldy,
                   T *__restrict__ Y) {
  constexpr int E = 16 / sizeof(T);
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r < n;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint4 *in = reinterpret_cast<const uint4 *>(Yt + r * (Q * E));
    Vec16<T> v[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) v[q].u = in[q];
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int64_t b = q * E + e;
        if (b < batch) Y[b * ldy + r] = v[q].e[e];
      }
  }
}

template <class T, int Q>
void narrow_q(bool to_columns, const void *in, int64_t batch, int64_t n, int64_t ld, void *out,
              uint32_t grid, hipStream_t stream) {
  if (to_columns)
    hipLaunchKernelGGL((gather_columns_q<T, Q>), dim3(grid), dim3(kThreads), 0, stream,
                       static_cast<const T *>(in), batch, n, ld, static_cast<T *>(out));
  else
    hipLaunchKernelGGL((scatter_rows_q<T, Q>), dim3(grid), dim3(kThreads), 0, stream,
                       static_cast<const T *>(in), batch, n, ld, static_cast<T *>(out));
}

template <class T>
msx_status narrow_t(bool to_columns, const void *in, int64_t batch, int64_t kpad, int64_t n,
                    int64_t ld, void *out, hipStream_t stream) {
  if (n == 0 || batch <= 0) return MSX_OK;
  const uint32_t grid = static_cast<uint32_t>(std::min((n + kThreads - 1) / kThreads, kMaxGrid));
  constexpr int64_t E = 16 / sizeof(T);
  bool done = true;
  switch (kpad / E) {
  case 1: narrow_q<T, 1>(to_columns, in, batch, n, ld, out, grid, stream); break;
  case 2: narrow_q<T, 2>(to_columns, in, batch, n, ld, out, grid, stream); break;
  case 4: narrow_q<T, 4>(to_columns, in, batch, n, ld, out, grid, stream); break;
  case 8: narrow_q<T, 8>(to_columns, in, batch, n, ld, out, grid, stream); break;
  default: done = false; break;  // other widths: the kernels with a runtime width
  }
  if (done) {
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  }
  if (to_columns)
    hipLaunchKernelGGL((gather_columns<T>), dim3(grid), dim3(kThreads), 0, stream,
                       static_cast<const T *>(in), batch, kpad, n, ld, static_cast<T *>(out));
  else
    hipLaunchKernelGGL((scatter_rows<T>), dim3(grid), dim3(kThreads), 0, stream,
                       static_cast<const T *>(in), batch, kpad, n, ld, static_cast<T *>(out));
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

msx_status narrow(msx_vtype vt, bool to_columns, const void *in, int64_t batch, int64_t kpad,
                  int64_t n, int64_t ld, void *out, hipStream_t stream) {
  switch (value_bytes(vt)) {
  case 2: return narrow_t<uint16_t>(to_columns, in, batch, kpad, n, ld, out, stream);
  case 4: return narrow_t<uint32_t>(to_columns, in, batch, kpad, n, ld, out, stream);
  default: return narrow_t<uint64_t>(to_columns, in, batch, kpad, n, ld, out, stream);
  }
}

template <class T>
msx_status transpose_t(const void *in, int64_t rows, int64_t rows_pad, int64_t cols, int64_t ldi,
                       void *out, int64_t ldo, hipStream_t stream) {
  const int64_t tiles = ((cols + kTile - 1) / kTile) * ((rows_pad + kTile - 1) / kTile);
  if (tiles == 0) return MSX_OK;
  hipLaunchKernelGGL((transpose_tiles<T>), dim3(static_cast<uint32_t>(std::min(tiles, kMaxGrid))),
                     dim3(kThreads), 0, stream, static_cast<const T *>(in), rows, rows_pad, cols,
                     ldi, static_cast<T *>(out), ldo);
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

msx_status transpose(msx_vtype vt, const void *in, int64_t rows, int64_t rows_pad, int64_t cols,
                     int64_t ldi, void *out, int64_t ldo, hipStream_t stream) {
  switch (value_bytes(vt)) {
  case 2: return transpose_t<uint16_t>(in, rows, rows_pad, cols, ldi, out, ldo, stream);
  case 4: return transpose_t<uint32_t>(in, rows, rows_pad, cols, ldi, out, ldo, stream);
  default: return transpose_t<uint64_t>(in, rows, rows_pad, cols, ldi, out, ldo, stream);
  }
}

msx_status check_batched(const char *op, msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                         int64_t nnz, const void *data, const void *indices, const void *indptr,
                         int64_t batch) {
  if (!valid_itype(it)) return fail(MSX_ETYPE, std::string(op) + " requires int32 or int64 indices.");
  if (!valid_vtype(vt)) return fail(MSX_ETYPE, std::string(op) + " unsupported value dtype.");
  if (n_rows < 0 || n_cols < 0 || nnz < 0 || batch < 0)
    return fail(MSX_EINVAL, std::string(op) + " shape dimensions must be non-negative.");
  if (n_rows >= kIntMax || n_cols > kIntMax || batch > kIntMax)
    return fail(MSX_EINVAL, std::string(op) + " shape dimensions must fit in int32.");
  if (indptr == nullptr) return fail(MSX_EINVAL, std::string(op) + " indptr is NULL.");
  if (nnz > 0 && (data == nullptr || indices == nullptr))
    return fail(MSX_EINVAL, std::string(op) + " data and indices must be non-NULL when nnz > 0.");
  return MSX_OK;
}

}  // namespace
}  // namespace msx

using namespace msx;

extern "C" msx_status msx_csr_batched_spmv(msx_vtype vt, msx_itype it, int64_t n_rows,
                                           int64_t n_cols, int64_t nnz, const void *data,
                                           const void *indices, const void *indptr, int64_t batch,
                                           const void *X, int64_t ldx, void *Y, int64_t ldy,
                                           void *stream_v) {
  clear_error();
  const char *op = "csr_batched_matvec";
  msx_status st = check_batched(op, vt, it, n_rows, n_cols, nnz, data, indices, indptr, batch);
  if (st != MSX_OK) return st;
  if (ldx < n_cols || ldy < n_rows)
    return fail(MSX_EINVAL, "csr_batched_matvec row strides must be at least the vector lengths.");
  if (batch > 0 && n_rows > 0 && Y == nullptr) return fail(MSX_EINVAL, "csr_batched_matvec Y is NULL.");
  if (batch > 0 && n_cols > 0 && nnz > 0 && X == nullptr)
    return fail(MSX_EINVAL, "csr_batched_matvec X is NULL.");
  if (batch == 0 || n_rows == 0) return MSX_OK;
  auto stream = static_cast<hipStream_t>(stream_v);
  if (batch == 1)  // one vector is a one-column SpMM, no transposes
    return launch_spmm_batched(vt, it, n_rows, n_cols, nnz, data, indices, indptr, 1, 1, X, 0, 1,
                               Y, 0, 1, true, stream);
  // Columns padded so that a row of the transposed operands is a whole number
  // of 16-byte vectors (the SpMM's vector path); padding columns read zero.
  const int64_t sv = static_cast<int64_t>(value_bytes(vt));
  const int64_t per16 = 16 / sv;
  const int64_t kpad = (batch + per16 - 1) / per16 * per16;
  const size_t bx = static_cast<size_t>(std::max<int64_t>(n_cols, 1) * kpad * sv);
  const size_t by = static_cast<size_t>(n_rows * kpad * sv);
  char *scratch = nullptr;
  MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&scratch), bx + by, stream));
  void *Xt = scratch, *Yt = scratch + bx;
  const bool thin = kpad <= kNarrow;
  st = thin ? narrow(vt, true, X, batch, kpad, n_cols, ldx, Xt, stream)
            : transpose(vt, X, batch, kpad, n_cols, ldx, Xt, kpad, stream);
  // Up to 8 16-byte vectors per row of Xt the sums go straight to Y;
  // otherwise through an n_rows x kpad SpMM result and its transpose.
  bool direct = false;
  if (st == MSX_OK)
    st = launch_spmv_batch_rows(vt, it, n_rows, n_cols, nnz, data, indices, indptr, Xt, kpad, Y,
                                ldy, batch, stream, &direct);
  if (st == MSX_OK && !direct) {
    st = launch_spmm_batched(vt, it, n_rows, n_cols, nnz, data, indices, indptr, 1, kpad, Xt, 0,
                             kpad, Yt, 0, kpad, false, stream);  // Yt is read back next
    if (st == MSX_OK)
      st = thin ? narrow(vt, false, Yt, batch, kpad, n_rows, ldy, Y, stream)
                : transpose(vt, Yt, n_rows, n_rows, batch, kpad, Y, ldy, stream);
  }
  const hipError_t e = hipFreeAsync(scratch, stream);
  if (st == MSX_OK && e != hipSuccess) return hip_fail(e, "csr_batched_matvec scratch release");
  return st;
}

extern "C" msx_status msx_csr_batched_spmm(msx_vtype vt, msx_itype it, int64_t n_rows,
                                           int64_t n_cols, int64_t nnz, const void *data,
                                           const void *indices, const void *indptr, int64_t batch,
                                           int64_t k, const void *X, int64_t x_batch, int64_t ldx,
                                           void *Y, int64_t y_batch, int64_t ldy, void *stream) {
  clear_error();
  const char *op = "csr_batched_matmul";
  msx_status st = check_batched(op, vt, it, n_rows, n_cols, nnz, data, indices, indptr, batch);
  if (st != MSX_OK) return st;
  if (k < 0 || k > kIntMax)
    return fail(MSX_EINVAL, "csr_batched_matmul rhs column count must fit in int32.");
  if (ldx < k || ldy < k)
    return fail(MSX_EINVAL, "csr_batched_matmul leading dimensions must be at least the column count.");
  if (batch > 1 && (x_batch < n_cols * ldx || y_batch < n_rows * ldy))
    return fail(MSX_EINVAL, "csr_batched_matmul batch strides must cover one matrix.");
  if (batch > 0 && n_rows > 0 && k > 0 && Y == nullptr)
    return fail(MSX_EINVAL, "csr_batched_matmul Y is NULL.");
  if (batch > 0 && n_cols > 0 && k > 0 && nnz > 0 && X == nullptr)
    return fail(MSX_EINVAL, "csr_batched_matmul X is NULL.");
  return launch_spmm_batched(vt, it, n_rows, n_cols, nnz, data, indices, indptr, batch, k, X,
                             x_batch, ldx, Y, y_batch, ldy, true, static_cast<hipStream_t>(stream));
}
