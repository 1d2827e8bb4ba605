// csr_transpose.hip - the adjoint side of the path: the CSR transpose, the
// transposed products A^T x / A^T X, and the value gradients of A x / A X.
//
//   msx_csr_transpose       CSR of A^T (= CSC of A), every column's entries
//                           in row order (the reference's counting sort,
//                           reference: src/sparse/csr_transpose/csr_transpose.cpp).
//                           Built by a stable radix sort of (column,
//                           position) pairs; fully asynchronous on `stream`.
//   msx_csr_spmv_transpose  y = A^T x, and msx_csr_spmm_transpose Y = A^T X,
//                           without a transpose: each stored value adds its
//                           product to its column's output with a float
//                           atomic (the reference's Metal kernels scatter the
//                           same way, csr_matvec_transpose.metal:27-49).  The
//                           order of those additions is not fixed, so the
//                           result agrees with a sequential sum to rounding.
//                           Deterministic transposed products come from
//                           msx_csr_transpose followed by msx_csr_spmv/_spmm.
//   msx_csr_spmv_data_vjp   g[p] = cot[row(p)] * x[col(p)], one rounding
//                           (reference: csr_matvec_data_vjp.cpp,
//                           csr_matvec_data_vjp_cpu_impl).
//   msx_csr_spmm_data_vjp   g[p] = sum_c cot[row(p), c] * X[col(p), c] from
//                           zero in c order (reference: csr_matmul_data_vjp.cpp).
// Complex conjugation of an operand (the Hermitian adjoint) is the caller's.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <mutex>
#include <string>

#include "msx_device.h"
#include "msx_internal.h"
#include "msx_sparse.h"

namespace msx {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kMaxGrid = int64_t{1} << 20;
constexpr int64_t kIntMax = 2147483647;

uint32_t grid_for(int64_t n) {
  return static_cast<uint32_t>(std::max<int64_t>(1, std::min<int64_t>((n + kThreads - 1) / kThreads, kMaxGrid)));
}

// Allocation-free transposed SpMV (msx_csr_spmv_transpose_noalloc): the
// float32 accumulators of 16-bit values live in this file-scope device array
// instead of stream-ordered scratch.  Each GPU the library runs on holds its
// own copy (32 MiB) until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): it passes the address hipGetSymbolAddress gives for the current
// device (noalloc_scratch below).
constexpr int64_t kNoAllocAccMax = int64_t{1} << 23;  // float32 accumulators
static __device__ __align__(256) float scratch[kNoAllocAccMax];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up on the first
// call made with that device current and kept.
msx_status noalloc_scratch(float **out) {
  int dev = -1;
  MSX_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MSX_EINVAL, "csr_matvec_transpose_noalloc supports device ordinals below 64.");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail(MSX_EHIP, "hipGetSymbolAddress(scratch) returned NULL.");
    g_scratch_ptr[dev] = static_cast<float *>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return MSX_OK;
}

__device__ inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

__device__ inline float amul(float a, float b) { return a * b; }
__device__ inline c64 amul(c64 a, c64 b) { return vmul<C64>(a, b); }

__device__ inline void atomic_acc(float *p, float v) { unsafeAtomicAdd(p, v); }
__device__ inline void atomic_acc(c64 *p, c64 v) {
  float *f = reinterpret_cast<float *>(p);
  unsafeAtomicAdd(f, v.re);
  unsafeAtomicAdd(f + 1, v.im);
}

// out[i] = src[pos[i]] (conjugated on request) for pos[i] in [0, n_src);
// entries with another position (the dropped values past t_indptr[n_cols])
// get zero bits, as a fresh transpose writes them.
template <class S>
__global__ void __launch_bounds__(kThreads)
    gather_positions(const S *__restrict__ src, int64_t n_src, const int32_t *__restrict__ pos,
                     int64_t count, bool conjugate, S *__restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t p = pos[i];
    if (p < 0 || p >= n_src) {
      out[i] = S(0);
      continue;
    }
    S v = src[p];
    if constexpr (sizeof(S) == 8) {
      if (conjugate) {
        uint64_t bits = 0;
        __builtin_memcpy(&bits, &v, 8);
        bits ^= uint64_t{1} << 63;  // sign of the imaginary part (the high float)
        __builtin_memcpy(&v, &bits, 8);
      }
    }
    out[i] = v;
  }
}

template <class T>
__global__ void __launch_bounds__(kThreads) fill(T *__restrict__ p, int64_t n, T v) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    p[i] = v;
}

// acc[r * lda + q] = 0 for r < rows, q < k (padding columns untouched).
template <class T>
__global__ void __launch_bounds__(kThreads)
    fill_rows(T *__restrict__ acc, int64_t rows, int64_t k, int64_t lda) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < rows * k;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t r = i / k;
    acc[r * lda + (i - r * k)] = T{};
  }
}

template <class V>
__global__ void __launch_bounds__(kThreads)
    narrow_all(const typename V::Acc *__restrict__ acc, int64_t n, typename V::Storage *__restrict__ y) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    y[i] = V::narrow(acc[i]);
}

// ---------------------------------------------------------------------------
// Transpose build.

// key[p] = column of p (n_cols when out of range), row[p] = its row; G
// lanes per row.
template <class I>
__global__ void __launch_bounds__(kThreads)
    column_keys(const I *__restrict__ indices, const I *__restrict__ indptr, int64_t n_rows,
                int64_t nnz, int64_t n_cols, int G, uint32_t *__restrict__ key,
                I *__restrict__ row) {
  const int64_t rows_per_block = kThreads / G;
  const int j = threadIdx.x % G;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / G;
       r < n_rows; r += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t s = clamp64(static_cast<int64_t>(indptr[r]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[r + 1]), s, nnz);
    for (int64_t p = s + j; p < e; p += G) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      key[p] = (c >= 0 && c < n_cols) ? static_cast<uint32_t>(c) : static_cast<uint32_t>(n_cols);
      row[p] = static_cast<I>(r);
    }
  }
}

__global__ void __launch_bounds__(kThreads)
    init_keys(int64_t nnz, uint32_t drop, uint32_t *__restrict__ key, uint32_t *__restrict__ pos) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; p < nnz;
       p += static_cast<int64_t>(gridDim.x) * kThreads) {
    key[p] = drop;
    pos[p] = static_cast<uint32_t>(p);
  }
}

// t_indptr[c] = first sorted index with key >= c, c in [0, n_cols].
template <class I>
__global__ void __launch_bounds__(kThreads)
    column_starts(const uint32_t *__restrict__ sorted, int64_t nnz, int64_t n_cols,
                  I *__restrict__ t_indptr) {
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; c <= n_cols;
       c += static_cast<int64_t>(gridDim.x) * kThreads) {
    int64_t lo = 0, hi = nnz;
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (static_cast<int64_t>(sorted[mid]) < c) lo = mid + 1; else hi = mid;
    }
    t_indptr[c] = static_cast<I>(lo);
  }
}

template <class S, class I>
__global__ void __launch_bounds__(kThreads)
    transpose_gather(const S *__restrict__ data, const I *__restrict__ row,
                     const uint32_t *__restrict__ key, const uint32_t *__restrict__ pos, int64_t nnz,
                     int64_t n_cols, S *__restrict__ t_data, I *__restrict__ t_indices) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < nnz;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    if (static_cast<int64_t>(key[i]) >= n_cols) {  // dropped: past t_indptr[n_cols]
      t_data[i] = S{};
      t_indices[i] = I(0);
      continue;
    }
    const int64_t p = clamp64(pos[i], 0, nnz - 1);
    t_data[i] = data[p];
    t_indices[i] = row[p];
  }
}

// Packed path (values of at most 4 bytes): the sort carries (row << 32) |
// value bits, so the transposed arrays come out of one coalesced pass.
// key[p] = column of p (n_cols when out of range), val[p] = packed pair;
// G lanes per row.  With kPos the "value" of p is p itself (int32): the
// transpose then lists, per entry, the position of A it came from.
template <class S, class I, bool kPos = false>
__global__ void __launch_bounds__(kThreads)
    packed_keys(const S *__restrict__ data, const I *__restrict__ indices,
                const I *__restrict__ indptr, int64_t n_rows, int64_t nnz, int64_t n_cols, int G,
                uint32_t *__restrict__ key, uint64_t *__restrict__ val) {
  static_assert(sizeof(S) <= 4, "packed transpose holds values of at most 4 bytes");
  const int64_t rows_per_block = kThreads / G;
  const int j = threadIdx.x % G;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / G;
       r < n_rows; r += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t s = clamp64(static_cast<int64_t>(indptr[r]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[r + 1]), s, nnz);
    for (int64_t p = s + j; p < e; p += G) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      key[p] = (c >= 0 && c < n_cols) ? static_cast<uint32_t>(c) : static_cast<uint32_t>(n_cols);
      uint32_t bits = 0;
      if constexpr (kPos)
        bits = static_cast<uint32_t>(p);
      else
        __builtin_memcpy(&bits, &data[p], sizeof(S));
      val[p] = (static_cast<uint64_t>(r) << 32) | bits;
    }
  }
}

__global__ void __launch_bounds__(kThreads)
    drop_keys(int64_t nnz, uint32_t drop, uint32_t *__restrict__ key) {
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; p < nnz;
       p += static_cast<int64_t>(gridDim.x) * kThreads)
    key[p] = drop;
}

// Sorted pairs -> t_data, t_indices, and t_indptr[c] = first sorted index
// with key >= c, written by the index where the key crosses c.  The entries
// past t_indptr[n_cols] (dropped values) get zero bits and row 0 (position
// -1 with kPos).
template <class S, class I, bool kPos = false>
__global__ void __launch_bounds__(kThreads)
    packed_unpack(const uint32_t *__restrict__ key, const uint64_t *__restrict__ val, int64_t nnz,
                  int64_t n_cols, S *__restrict__ t_data, I *__restrict__ t_indices,
                  I *__restrict__ t_indptr) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i <= nnz;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t prev = i == 0 ? -1 : static_cast<int64_t>(key[i - 1]);
    const int64_t cur = i == nnz ? n_cols : static_cast<int64_t>(key[i]);
    for (int64_t c = prev + 1; c <= cur && c <= n_cols; ++c) t_indptr[c] = static_cast<I>(i);
    if (i < nnz && cur < n_cols) {
      const uint64_t v = val[i];
      const uint32_t bits = static_cast<uint32_t>(v);
      S d;
      __builtin_memcpy(&d, &bits, sizeof(S));
      t_data[i] = d;
      t_indices[i] = static_cast<I>(v >> 32);
    } else if (i < nnz) {  // dropped values: zero bits (position -1 with kPos), row 0
      t_data[i] = kPos ? S(-1) : S(0);
      t_indices[i] = I(0);
    }
  }
}

int lanes_for(int64_t n_rows, int64_t nnz);

template <class S, class I, bool kPos = false>
msx_status transpose_packed(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                            const void *indices, const void *indptr, void *t_data,
                            void *t_indices, void *t_indptr, int end_bit, hipStream_t stream) {
  const size_t b4 = (static_cast<size_t>(nnz) * 4 + 255) / 256 * 256;
  const size_t b8 = (static_cast<size_t>(nnz) * 8 + 255) / 256 * 256;
  size_t sort_bytes = 0;
  MSX_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint64_t *>(nullptr),
                                                 static_cast<uint64_t *>(nullptr),
                                                 static_cast<int>(nnz), 0, end_bit, stream));
  char *work = nullptr;
  MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&work), 2 * b4 + 2 * b8 + sort_bytes, stream));
  auto *key = reinterpret_cast<uint32_t *>(work);
  auto *key_out = reinterpret_cast<uint32_t *>(work + b4);
  auto *val = reinterpret_cast<uint64_t *>(work + 2 * b4);
  auto *val_out = reinterpret_cast<uint64_t *>(work + 2 * b4 + b8);
  void *sort_tmp = work + 2 * b4 + 2 * b8;
  const int G = lanes_for(n_rows, nnz);
  hipLaunchKernelGGL(drop_keys, dim3(grid_for(nnz)), dim3(kThreads), 0, stream, nnz,
                     static_cast<uint32_t>(n_cols), key);
  hipLaunchKernelGGL((packed_keys<S, I, kPos>), dim3(grid_for(n_rows * G)), dim3(kThreads), 0, stream,
                     static_cast<const S *>(data), static_cast<const I *>(indices),
                     static_cast<const I *>(indptr), n_rows, nnz, n_cols, G, key, val);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess)
    e = hipcub::DeviceRadixSort::SortPairs(sort_tmp, sort_bytes, key, key_out, val, val_out,
                                           static_cast<int>(nnz), 0, end_bit, stream);
  if (e == hipSuccess) {
    hipLaunchKernelGGL((packed_unpack<S, I, kPos>), dim3(grid_for(nnz + 1)), dim3(kThreads), 0, stream,
                       key_out, val_out, nnz, n_cols, static_cast<S *>(t_data),
                       static_cast<I *>(t_indices), static_cast<I *>(t_indptr));
    e = hipGetLastError();
  }
  msx_status st = MSX_OK;
  if (e != hipSuccess) st = hip_fail(e, "csr_transpose");
  const hipError_t ef = hipFreeAsync(work, stream);
  if (st == MSX_OK && ef != hipSuccess) st = hip_fail(ef, "csr_transpose scratch release");
  return st;
}

int bits_for(uint64_t v) {
  int b = 0;
  while (b < 64 && (v >> b) != 0) ++b;
  return std::max(1, b);
}

template <class S, class I>
msx_status transpose_typed(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                           const void *indices, const void *indptr, void *t_data, void *t_indices,
                           void *t_indptr, hipStream_t stream) {
  const auto *ip = static_cast<const I *>(indptr);
  auto *tp = static_cast<I *>(t_indptr);
  if (nnz == 0) {
    hipLaunchKernelGGL((fill<I>), dim3(grid_for(n_cols + 1)), dim3(kThreads), 0, stream, tp,
                       n_cols + 1, I{0});
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  }
  const int end_bit = bits_for(static_cast<uint64_t>(n_cols));  // keys <= n_cols
  if constexpr (sizeof(S) <= 4)
    return transpose_packed<S, I>(n_rows, n_cols, nnz, data, indices, indptr, t_data, t_indices,
                                  t_indptr, end_bit, stream);
  // Wider values: sort (column, position), then gather values and rows.
  // Scratch: 4 key/position arrays, the row of each value, the sort's temp.
  const size_t b4 = (static_cast<size_t>(nnz) * 4 + 255) / 256 * 256;
  const size_t bI = (static_cast<size_t>(nnz) * sizeof(I) + 255) / 256 * 256;
  size_t sort_bytes = 0;
  MSX_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, sort_bytes, static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint32_t *>(nullptr),
                                                 static_cast<int>(nnz), 0, end_bit, stream));
  char *work = nullptr;
  MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&work), 4 * b4 + bI + sort_bytes, stream));
  auto *key = reinterpret_cast<uint32_t *>(work);
  auto *key_out = reinterpret_cast<uint32_t *>(work + b4);
  auto *pos = reinterpret_cast<uint32_t *>(work + 2 * b4);
  auto *pos_out = reinterpret_cast<uint32_t *>(work + 3 * b4);
  auto *row = reinterpret_cast<I *>(work + 4 * b4);
  void *sort_tmp = work + 4 * b4 + bI;
  msx_status st = MSX_OK;
  hipLaunchKernelGGL(init_keys, dim3(grid_for(nnz)), dim3(kThreads), 0, stream, nnz,
                     static_cast<uint32_t>(n_cols), key, pos);
  const int G = lanes_for(n_rows, nnz);
  hipLaunchKernelGGL((column_keys<I>), dim3(grid_for(n_rows * G)), dim3(kThreads), 0, stream,
                     static_cast<const I *>(indices), ip, n_rows, nnz, n_cols, G, key, row);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess)
    e = hipcub::DeviceRadixSort::SortPairs(sort_tmp, sort_bytes, key, key_out, pos, pos_out,
                                           static_cast<int>(nnz), 0, end_bit, stream);
  if (e == hipSuccess) {
    hipLaunchKernelGGL((column_starts<I>), dim3(grid_for(n_cols + 1)), dim3(kThreads), 0, stream,
                       key_out, nnz, n_cols, tp);
    hipLaunchKernelGGL((transpose_gather<S, I>), dim3(grid_for(nnz)), dim3(kThreads), 0, stream,
                       static_cast<const S *>(data), row, key_out, pos_out, nnz, n_cols,
                       static_cast<S *>(t_data), static_cast<I *>(t_indices));
    e = hipGetLastError();
  }
  if (e != hipSuccess) st = hip_fail(e, "csr_transpose");
  const hipError_t ef = hipFreeAsync(work, stream);
  if (st == MSX_OK && ef != hipSuccess) st = hip_fail(ef, "csr_transpose scratch release");
  return st;
}

// ---------------------------------------------------------------------------
// Transposed products by atomic scatter.  G lanes per row of A.

template <class V, class I>
__global__ void __launch_bounds__(kThreads)
    scatter_spmv(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                 const I *__restrict__ indptr, const typename V::Storage *__restrict__ x,
                 typename V::Acc *__restrict__ acc, int64_t n_rows, int64_t nnz, int64_t n_cols,
                 int G) {
  using A = typename V::Acc;
  const int64_t rows_per_block = kThreads / G;
  const int j = threadIdx.x % G;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / G;
       row < n_rows; row += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    const A xr = V::widen(x[row]);
    for (int64_t p = s + j; p < e; p += G) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      if (c >= 0 && c < n_cols) atomic_acc(acc + c, amul(V::widen(data[p]), xr));
    }
  }
}

// One wave per row of A; lanes over the k columns of X.
template <class V, class I>
__global__ void __launch_bounds__(kThreads)
    scatter_spmm(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                 const I *__restrict__ indptr, const typename V::Storage *__restrict__ X,
                 int64_t ldx, typename V::Acc *__restrict__ acc, int64_t lda, int64_t n_rows,
                 int64_t nnz, int64_t n_cols, int64_t k) {
  const int lane = threadIdx.x % kWave;
  const int64_t waves = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
       row < n_rows; row += waves) {
    const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    for (int64_t p = s; p < e; ++p) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      if (c < 0 || c >= n_cols) continue;
      const typename V::Acc a = V::widen(data[p]);
      for (int64_t q = lane; q < k; q += kWave)
        atomic_acc(acc + c * lda + q, amul(a, V::widen(X[row * ldx + q])));
    }
  }
}

template <class V>
__global__ void __launch_bounds__(kThreads)
    narrow_rows(const typename V::Acc *__restrict__ acc, int64_t rows, int64_t k, int64_t lda,
                typename V::Storage *__restrict__ Y, int64_t ldy) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < rows * k;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t r = i / k, q = i - r * k;
    Y[r * ldy + q] = V::narrow(acc[r * lda + q]);
  }
}

// ---------------------------------------------------------------------------
// Value gradients.  G lanes per row.

template <class V, class I>
__global__ void __launch_bounds__(kThreads)
    spmv_data_vjp(const I *__restrict__ indices, const I *__restrict__ indptr,
                  const typename V::Storage *__restrict__ x,
                  const typename V::Storage *__restrict__ cot, typename V::Storage *__restrict__ out,
                  int64_t n_rows, int64_t nnz, int64_t n_cols, int G) {
  using A = typename V::Acc;
  const int64_t rows_per_block = kThreads / G;
  const int j = threadIdx.x % G;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block + threadIdx.x / G;
       row < n_rows; row += static_cast<int64_t>(gridDim.x) * rows_per_block) {
    const int64_t s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
    const int64_t e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    const A g = V::widen(cot[row]);
    for (int64_t p = s + j; p < e; p += G) {
      const int64_t c = static_cast<int64_t>(indices[p]);
      out[p] = V::narrow((c >= 0 && c < n_cols) ? amul(g, V::widen(x[c])) : vzero<A>());
    }
  }
}

// One wave per block.  The wave takes 64 / G rows at a time, G lanes per row
// (lane = one stored value; long rows take several rounds).  X and cot are
// read in column tiles of kVjpTile: the wave loads each active value's X row
// segment and each row's cot segment with coalesced loads (two rows per
// instruction) into LDS, then every lane adds its tile's products in q order
// from LDS, so each value's sum runs from zero over q = 0 .. k-1 in order.
constexpr int kVjpTile = 32;

template <class V, class I>
__global__ void __launch_bounds__(kWave)
    spmm_data_vjp(const I *__restrict__ indices, const I *__restrict__ indptr,
                  const typename V::Storage *__restrict__ X, int64_t ldx,
                  const typename V::Storage *__restrict__ cot, int64_t ldc,
                  typename V::Storage *__restrict__ out, int64_t n_rows, int64_t nnz,
                  int64_t n_cols, int64_t k, int G) {
  using A = typename V::Acc;
  __shared__ A xs[kWave][kVjpTile + 1];
  __shared__ A cs[kWave][kVjpTile + 1];
  __shared__ int cl[kWave];  // column of each lane's value, -1 when none
  const int lane = threadIdx.x;
  const int R = kWave / G;
  const int g = lane / G, j = lane - g * G;
  const int half = lane >> 5, qq = lane & 31;
  for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * R; r0 < n_rows;
       r0 += static_cast<int64_t>(gridDim.x) * R) {
    const int64_t row = r0 + g;
    int64_t s = 0, e = 0;
    if (row < n_rows) {
      s = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
      e = clamp64(static_cast<int64_t>(indptr[row + 1]), s, nnz);
    }
    const int rows_here = static_cast<int>(r0 + R <= n_rows ? R : n_rows - r0);
    for (int64_t base = 0;; base += G) {
      const int64_t p = s + base + j;
      const bool act = p < e;
      const uint64_t mask = __ballot(act);
      if (mask == 0) break;  // wave-uniform
      int c = -1;
      if (act) {
        const int64_t cv = static_cast<int64_t>(indices[p]);
        c = (cv >= 0 && cv < n_cols) ? static_cast<int>(cv) : -1;
      }
      cl[lane] = c;
      __syncthreads();
      A acc = vzero<A>();
      for (int64_t q0 = 0; q0 < k; q0 += kVjpTile) {
        const int qn = static_cast<int>(k - q0 < kVjpTile ? k - q0 : kVjpTile);
        // X row segments of the active values (two per instruction) and the
        // cot segments of the group's rows: every load is issued before the
        // first LDS store, so a wave keeps them all in flight.
        // Slots a lane does not read (no value, dropped column, q >= qn)
        // hold zeros.
        using S = typename V::Storage;
        S xv[kWave / 2], cv[kWave / 2];
#pragma unroll
        for (int t = 0; t < kWave / 2; ++t) {
          const int cc = cl[2 * t + half];
          xv[t] = (cc >= 0 && qq < qn) ? X[static_cast<int64_t>(cc) * ldx + q0 + qq] : S{};
          const int gi = 2 * t + half;
          cv[t] = (gi < rows_here && qq < qn) ? cot[(r0 + gi) * ldc + q0 + qq] : S{};
        }
#pragma unroll
        for (int t = 0; t < kWave / 2; ++t) {
          xs[2 * t + half][qq] = V::widen(xv[t]);
          cs[2 * t + half][qq] = V::widen(cv[t]);
        }
        __syncthreads();
        if (c >= 0)
          for (int q = 0; q < qn; ++q) acc = vadd(acc, amul(cs[g][q], xs[lane][q]));
        __syncthreads();
      }
      if (act) out[p] = V::narrow(acc);
      __syncthreads();  // cl is rewritten by the next round
    }
  }
}

int lanes_for(int64_t n_rows, int64_t nnz) {
  const int64_t avg = n_rows > 0 ? nnz / n_rows : 0;
  int G = 1;
  while (G < kWave && 2 * G <= avg) G <<= 1;
  return G;
}

// Dispatch on value and index types.
template <template <class, class> class Fn, class... Args>
msx_status dispatch(msx_vtype vt, msx_itype it, Args... args) {
  const bool i64 = it == MSX_I64;
  switch (vt) {
  case MSX_F32: return i64 ? Fn<F32, int64_t>::run(args...) : Fn<F32, int32_t>::run(args...);
  case MSX_F16: return i64 ? Fn<F16, int64_t>::run(args...) : Fn<F16, int32_t>::run(args...);
  case MSX_BF16: return i64 ? Fn<BF16, int64_t>::run(args...) : Fn<BF16, int32_t>::run(args...);
  case MSX_C64: return i64 ? Fn<C64, int64_t>::run(args...) : Fn<C64, int32_t>::run(args...);
  }
  return fail(MSX_ETYPE, "unsupported value dtype.");
}

template <class V, class I>
struct TransposeOp {
  static msx_status run(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                        const void *indices, const void *indptr, void *t_data, void *t_indices,
                        void *t_indptr, hipStream_t stream) {
    return transpose_typed<typename V::Storage, I>(n_rows, n_cols, nnz, data, indices, indptr,
                                                   t_data, t_indices, t_indptr, stream);
  }
};

// Accumulators: the output itself when it holds the accumulator type
// (float32, complex64), else float32 scratch narrowed at the end: `fixed`
// (n_cols floats the caller provides) when non-NULL, else stream-ordered
// scratch.
template <class V, class I>
struct SpmvTransposeOp {
  static msx_status run(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                        const void *indices, const void *indptr, const void *x, void *y,
                        float *fixed, hipStream_t stream) {
    using S = typename V::Storage;
    using A = typename V::Acc;
    constexpr bool direct = sizeof(S) == sizeof(A);
    const bool owned = !direct && fixed == nullptr;
    A *acc = nullptr;
    if (direct) {
      acc = static_cast<A *>(y);
    } else if (fixed != nullptr) {
      acc = reinterpret_cast<A *>(fixed);
    } else {
      MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&acc), sizeof(A) * std::max<int64_t>(n_cols, 1), stream));
    }
    hipLaunchKernelGGL((fill<A>), dim3(grid_for(n_cols)), dim3(kThreads), 0, stream, acc, n_cols, A{});
    const int G = lanes_for(n_rows, nnz);
    hipLaunchKernelGGL((scatter_spmv<V, I>), dim3(grid_for(n_rows * G)), dim3(kThreads), 0, stream,
                       static_cast<const S *>(data), static_cast<const I *>(indices),
                       static_cast<const I *>(indptr), static_cast<const S *>(x), acc, n_rows, nnz,
                       n_cols, G);
    if (!direct)
      hipLaunchKernelGGL((narrow_all<V>), dim3(grid_for(n_cols)), dim3(kThreads), 0, stream, acc,
                         n_cols, static_cast<S *>(y));
    hipError_t e = hipGetLastError();
    if (owned) {
      const hipError_t ef = hipFreeAsync(acc, stream);
      if (e == hipSuccess) e = ef;
    }
    if (e != hipSuccess) return hip_fail(e, "csr_matvec_transpose");
    return MSX_OK;
  }
};

template <class V, class I>
struct SpmmTransposeOp {
  static msx_status run(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                        const void *indices, const void *indptr, int64_t k, const void *X,
                        int64_t ldx, void *Y, int64_t ldy, hipStream_t stream) {
    using S = typename V::Storage;
    using A = typename V::Acc;
    constexpr bool direct = sizeof(S) == sizeof(A);
    A *acc = nullptr;
    int64_t lda = ldy;
    if (direct) {
      acc = static_cast<A *>(Y);
    } else {
      lda = k;
      MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&acc),
                                 sizeof(A) * std::max<int64_t>(n_cols * k, 1), stream));
    }
    hipLaunchKernelGGL((fill_rows<A>), dim3(grid_for(n_cols * k)), dim3(kThreads), 0, stream, acc,
                       n_cols, k, lda);
    hipLaunchKernelGGL((scatter_spmm<V, I>), dim3(grid_for(n_rows * kWave)), dim3(kThreads), 0,
                       stream, static_cast<const S *>(data), static_cast<const I *>(indices),
                       static_cast<const I *>(indptr), static_cast<const S *>(X), ldx, acc, lda,
                       n_rows, nnz, n_cols, k);
    if (!direct)
      hipLaunchKernelGGL((narrow_rows<V>), dim3(grid_for(n_cols * k)), dim3(kThreads), 0, stream,
                         acc, n_cols, k, lda, static_cast<S *>(Y), ldy);
    hipError_t e = hipGetLastError();
    if (!direct) {
      const hipError_t ef = hipFreeAsync(acc, stream);
      if (e == hipSuccess) e = ef;
    }
    if (e != hipSuccess) return hip_fail(e, "csr_matmul_transpose");
    return MSX_OK;
  }
};

template <class V, class I>
struct SpmvDataVjpOp {
  static msx_status run(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *indices,
                        const void *indptr, const void *x, const void *cot, void *out,
                        hipStream_t stream) {
    using S = typename V::Storage;
    const int G = lanes_for(n_rows, nnz);
    hipLaunchKernelGGL((spmv_data_vjp<V, I>), dim3(grid_for(n_rows * G)), dim3(kThreads), 0, stream,
                       static_cast<const I *>(indices), static_cast<const I *>(indptr),
                       static_cast<const S *>(x), static_cast<const S *>(cot), static_cast<S *>(out),
                       n_rows, nnz, n_cols, G);
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  }
};

template <class V, class I>
struct SpmmDataVjpOp {
  static msx_status run(int64_t n_rows, int64_t n_cols, int64_t nnz, const void *indices,
                        const void *indptr, int64_t k, const void *X, int64_t ldx, const void *cot,
                        int64_t ldc, void *out, hipStream_t stream) {
    using S = typename V::Storage;
    const int G = lanes_for(n_rows, nnz);
    const int64_t groups = (n_rows + kWave / G - 1) / (kWave / G);
    const uint32_t grid = static_cast<uint32_t>(std::min<int64_t>(std::max<int64_t>(groups, 1), kMaxGrid));
    hipLaunchKernelGGL((spmm_data_vjp<V, I>), dim3(grid), dim3(kWave), 0, stream,
                       static_cast<const I *>(indices), static_cast<const I *>(indptr),
                       static_cast<const S *>(X), ldx, static_cast<const S *>(cot), ldc,
                       static_cast<S *>(out), n_rows, nnz, n_cols, k, G);
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  }
};

// ---------------------------------------------------------------------------
// Regather of a cached transpose's values in two streaming passes.
//
// t_data[i] = data[t_pos[i]] is a random gather (one 4-byte read per value
// from a 268 MB array on the headline matrix: 1.28 ms).  With the
// permutation fixed, it splits into two passes that each stream:
//
//   pass 1 (one workgroup per source tile of D1 values): the tile's values
//           are placed in LDS at slot1[p], their order sorted by destination
//           bucket, and written back in place to the scratch array S1
//           (coalesced in and out);
//   pass 2 (one workgroup per destination bucket of D2 entries): the
//           bucket's entries are read from S1 at src1[s] - per tile, one
//           contiguous run of D1 * D2 / nnz values - placed in LDS at
//           slot2[s] (their offset in the bucket) and written out in order.
//
// The layout (slot1, src1, slot2) comes from two stable radix sorts of the
// positions, once.  Sizes by value width: D1 * width = 128 KB of LDS at
// most (64 KB for 16-bit values), D2 * width = 64 KB; D1 <= 32768, so a
// slot fits 16 bits and 0xFFFF marks a source no entry takes.
template <int VB>
struct PermSizes {
  static constexpr int D1 = VB == 8 ? 16384 : 32768;
  static constexpr int D2 = VB == 8 ? 8192 : (VB == 4 ? 16384 : 32768);
};
constexpr int kPermThreads = 1024;
constexpr int kPermUnroll = 4;
constexpr uint16_t kNoSlot = 0xFFFF;
constexpr uint32_t kNoSource = 0xFFFFFFFFu;

template <class S>
__device__ inline S conj_bits(S v, bool conjugate) {
  if constexpr (sizeof(S) == 8) {
    if (conjugate) v ^= uint64_t{1} << 63;  // sign of the imaginary part (the high float)
  }
  return v;
}

template <class S>
__global__ void __launch_bounds__(kPermThreads)
    perm_tiles(const S *__restrict__ data, const uint16_t *__restrict__ slot1, int64_t nnz,
               bool conjugate, S *__restrict__ s1) {
  constexpr int D1 = PermSizes<sizeof(S)>::D1;
  extern __shared__ unsigned char perm_lds[];
  S *lds = reinterpret_cast<S *>(perm_lds);
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * D1;
  const int len = static_cast<int>(std::min<int64_t>(D1, nnz - p0));
  for (int j0 = threadIdx.x; j0 < len; j0 += kPermUnroll * kPermThreads) {
    S v[kPermUnroll];
    uint16_t sl[kPermUnroll];
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {  // clamped index: every load issued before any use
      const int j = j0 + u * kPermThreads < len ? j0 + u * kPermThreads : j0;
      v[u] = __builtin_nontemporal_load(data + p0 + j);
      sl[u] = __builtin_nontemporal_load(slot1 + p0 + j);
    }
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u)
      if (j0 + u * kPermThreads < len && sl[u] < D1) lds[sl[u]] = conj_bits(v[u], conjugate);
  }
  __syncthreads();
  for (int j = threadIdx.x; j < len; j += kPermThreads) s1[p0 + j] = lds[j];
}

template <class S>
__global__ void __launch_bounds__(kPermThreads)
    perm_buckets(const S *__restrict__ s1, const uint32_t *__restrict__ src1,
                 const uint16_t *__restrict__ slot2, int64_t nnz, S *__restrict__ out) {
  constexpr int D2 = PermSizes<sizeof(S)>::D2;
  extern __shared__ unsigned char perm_lds[];
  S *lds = reinterpret_cast<S *>(perm_lds);
  // each XCD takes a contiguous range of buckets: neighbouring buckets read
  // neighbouring runs of every tile, which then share L2 lines
  const int64_t b0 = static_cast<int64_t>(xcd_remap(blockIdx.x, gridDim.x)) * D2;
  const int len = static_cast<int>(std::min<int64_t>(D2, nnz - b0));
  for (int s0 = threadIdx.x; s0 < len; s0 += kPermUnroll * kPermThreads) {
    uint32_t a[kPermUnroll];
    uint16_t sl[kPermUnroll];
    S v[kPermUnroll];
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) {
      const int s = s0 + u * kPermThreads < len ? s0 + u * kPermThreads : s0;
      a[u] = __builtin_nontemporal_load(src1 + b0 + s);
      sl[u] = __builtin_nontemporal_load(slot2 + b0 + s);
    }
    // an address past the array (kNoSource: a dropped entry) reads element 0
    // and is replaced by zero, so every load is issued before any is used
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u) v[u] = s1[static_cast<int64_t>(a[u]) < nnz ? a[u] : 0u];
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u)
      if (static_cast<int64_t>(a[u]) >= nnz) v[u] = S(0);
#pragma unroll
    for (int u = 0; u < kPermUnroll; ++u)
      if (s0 + u * kPermThreads < len && sl[u] < D2) lds[sl[u]] = v[u];
  }
  __syncthreads();
  for (int j = threadIdx.x; j < len; j += kPermThreads) out[b0 + j] = lds[j];
}

// The same two passes with every stream read and written in quads of 4
// elements (16-byte loads of 4-byte values), each thread's whole share of
// its tile or bucket loaded before any is used - all of a thread's index
// quads, then all of its gathers - so that a workgroup waits on memory
// once per stage, not once per 4 elements.  Used when every buffer is
// aligned to its quad; the elements past the last whole quad of a tile or
// bucket go one per thread.
template <class S>
__global__ void __launch_bounds__(kPermThreads)
    perm_tiles_q(const S *__restrict__ data, const uint16_t *__restrict__ slot1, int64_t nnz,
                 bool conjugate, S *__restrict__ s1) {
  using V4 = S __attribute__((ext_vector_type(4)));
  using H4 = uint16_t __attribute__((ext_vector_type(4)));
  constexpr int D1 = PermSizes<sizeof(S)>::D1;
  constexpr int NQ = D1 / 4 / kPermThreads;  // quads per thread
  extern __shared__ unsigned char perm_lds[];
  S *lds = reinterpret_cast<S *>(perm_lds);
  const int64_t p0 = static_cast<int64_t>(blockIdx.x) * D1;
  const int len = static_cast<int>(std::min<int64_t>(D1, nnz - p0));
  const int nq = len / 4;
  const auto *dq = reinterpret_cast<const V4 *>(data + p0);
  const auto *sq = reinterpret_cast<const H4 *>(slot1 + p0);
  V4 v[NQ];
  H4 sl[NQ];
  if (nq > 0) {  // clamped indices: every load issued before any use
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int qi = static_cast<int>(threadIdx.x) + u * kPermThreads;
      const int qc = qi < nq ? qi : 0;
      v[u] = __builtin_nontemporal_load(dq + qc);
      sl[u] = __builtin_nontemporal_load(sq + qc);
    }
  }
  const int te = 4 * nq + static_cast<int>(threadIdx.x);  // the tail, one element per thread
  S tv{};
  uint16_t ts = kNoSlot;
  if (te < len) {
    tv = data[p0 + te];
    ts = slot1[p0 + te];
  }
  if (nq > 0) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int qi = static_cast<int>(threadIdx.x) + u * kPermThreads;
      if (qi < nq) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (sl[u][e] < D1) lds[sl[u][e]] = conj_bits(static_cast<S>(v[u][e]), conjugate);
      }
    }
  }
  if (te < len && ts < D1) lds[ts] = conj_bits(tv, conjugate);
  __syncthreads();
  const auto *lq = reinterpret_cast<const V4 *>(lds);
  auto *oq = reinterpret_cast<V4 *>(s1 + p0);
  for (int qi = threadIdx.x; qi < nq; qi += kPermThreads) oq[qi] = lq[qi];
  if (te < len) s1[p0 + te] = lds[te];
}

template <class S>
__global__ void __launch_bounds__(kPermThreads)
    perm_buckets_q(const S *__restrict__ s1, const uint32_t *__restrict__ src1,
                   const uint16_t *__restrict__ slot2, int64_t nnz, S *__restrict__ out) {
  using V4 = S __attribute__((ext_vector_type(4)));
  using H4 = uint16_t __attribute__((ext_vector_type(4)));
  using W4 = uint32_t __attribute__((ext_vector_type(4)));
  constexpr int D2 = PermSizes<sizeof(S)>::D2;
  constexpr int NQ = D2 / 4 / kPermThreads;
  extern __shared__ unsigned char perm_lds[];
  S *lds = reinterpret_cast<S *>(perm_lds);
  // each XCD takes a contiguous range of buckets (as in perm_buckets)
  const int64_t b0 = static_cast<int64_t>(xcd_remap(blockIdx.x, gridDim.x)) * D2;
  const int len = static_cast<int>(std::min<int64_t>(D2, nnz - b0));
  const int nq = len / 4;
  const auto *aq = reinterpret_cast<const W4 *>(src1 + b0);
  const auto *sq = reinterpret_cast<const H4 *>(slot2 + b0);
  W4 a[NQ];
  H4 sl[NQ];
  if (nq > 0) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int qi = static_cast<int>(threadIdx.x) + u * kPermThreads;
      const int qc = qi < nq ? qi : 0;
      a[u] = __builtin_nontemporal_load(aq + qc);
      sl[u] = __builtin_nontemporal_load(sq + qc);
    }
  }
  const int te = 4 * nq + static_cast<int>(threadIdx.x);
  uint32_t ta = kNoSource;
  uint16_t ts = kNoSlot;
  if (te < len) {
    ta = src1[b0 + te];
    ts = slot2[b0 + te];
  }
  // the gathers: an address past the array (kNoSource: a dropped entry)
  // reads element 0 and is replaced by zero
  S v[NQ][4];
  if (nq > 0) {
#pragma unroll
    for (int u = 0; u < NQ; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t ai = a[u][e];
        v[u][e] = s1[static_cast<int64_t>(ai) < nnz ? ai : 0u];
      }
  }
  S tv = s1[static_cast<int64_t>(ta) < nnz ? ta : 0u];
  if (static_cast<int64_t>(ta) >= nnz) tv = S(0);
  if (nq > 0) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int qi = static_cast<int>(threadIdx.x) + u * kPermThreads;
      if (qi < nq) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const S x = static_cast<int64_t>(a[u][e]) < nnz ? v[u][e] : S(0);
          if (sl[u][e] < D2) lds[sl[u][e]] = x;
        }
      }
    }
  }
  if (te < len && ts < D2) lds[ts] = tv;
  __syncthreads();
  const auto *lq = reinterpret_cast<const V4 *>(lds);
  auto *oq = reinterpret_cast<V4 *>(out + b0);
  for (int qi = threadIdx.x; qi < nq; qi += kPermThreads) oq[qi] = lq[qi];
  if (te < len) out[b0 + te] = lds[te];
}

// Layout build.  key[i] = (bucket of i, source of i) - the source nnz for
// a dropped entry, so it sorts last in its bucket; val[i] = i.
__global__ void __launch_bounds__(kThreads)
    layout_keys(const int32_t *__restrict__ t_pos, int64_t nnz, int D2, int pbits,
                uint64_t *__restrict__ key, uint32_t *__restrict__ val) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < nnz;
       i += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t p = t_pos[i];
    const uint64_t pv = (p >= 0 && p < nnz) ? static_cast<uint64_t>(p) : static_cast<uint64_t>(nnz);
    key[i] = (static_cast<uint64_t>(i / D2) << pbits) | pv;
    val[i] = static_cast<uint32_t>(i);
  }
}

// Sorted by (bucket, source): position s of the S order.  slot2[s] = the
// entry's offset in its bucket; then key (tile of the source; ntile for a
// dropped entry) and value (s << 32 | source) for the stable sort by tile.
__global__ void __launch_bounds__(kThreads)
    layout_buckets(const uint64_t *__restrict__ key_s, const uint32_t *__restrict__ val_s,
                   int64_t nnz, int D1, int D2, uint64_t pmask, uint32_t ntile,
                   uint16_t *__restrict__ slot2, uint32_t *__restrict__ tkey,
                   uint64_t *__restrict__ tval) {
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; s < nnz;
       s += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t b0 = s / D2 * D2;
    slot2[s] = static_cast<uint16_t>(static_cast<int64_t>(val_s[s]) - b0);
    const uint64_t pv = key_s[s] & pmask;
    tkey[s] = pv < static_cast<uint64_t>(nnz) ? static_cast<uint32_t>(pv / D1) : ntile;
    tval[s] = (static_cast<uint64_t>(s) << 32) | pv;
  }
}

// tstart[t] = first index of the tile-sorted keys with key >= t, t <= ntile.
__global__ void __launch_bounds__(kThreads)
    layout_tile_starts(const uint32_t *__restrict__ tkey_s, int64_t nnz, uint32_t ntile,
                       int64_t *__restrict__ tstart) {
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; g <= nnz;
       g += static_cast<int64_t>(gridDim.x) * kThreads) {
    const int64_t prev = g == 0 ? -1 : static_cast<int64_t>(tkey_s[g - 1]);
    const int64_t cur = g == nnz ? ntile : std::min<int64_t>(tkey_s[g], ntile);
    for (int64_t t = prev + 1; t <= cur; ++t) tstart[t] = g;
  }
}

// In tile order: the k-th entry of tile t (in S order) takes slot k of the
// tile: src1[s] = t * D1 + k, slot1[source] = k.  Dropped entries get
// kNoSource.
__global__ void __launch_bounds__(kThreads)
    layout_tiles(const uint32_t *__restrict__ tkey_s, const uint64_t *__restrict__ tval_s,
                 const int64_t *__restrict__ tstart, int64_t nnz, int D1, uint32_t ntile,
                 uint32_t *__restrict__ src1, uint16_t *__restrict__ slot1) {
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; g < nnz;
       g += static_cast<int64_t>(gridDim.x) * kThreads) {
    const uint32_t t = tkey_s[g];
    const uint64_t v = tval_s[g];
    const int64_t s = static_cast<int64_t>(v >> 32);
    const int64_t p = static_cast<int64_t>(v & 0xFFFFFFFFu);
    if (s >= nnz) continue;
    if (t >= ntile || p >= nnz) {
      src1[s] = kNoSource;
      continue;
    }
    const int64_t k = g - tstart[t];
    src1[s] = static_cast<uint32_t>(static_cast<int64_t>(t) * D1 + k);
    slot1[p] = k < D1 ? static_cast<uint16_t>(k) : kNoSlot;
  }
}

template <int VB>
msx_status transpose_layout_sized(int64_t nnz, const int32_t *t_pos, uint16_t *slot1,
                                  uint32_t *src1, uint16_t *slot2, hipStream_t stream) {
  constexpr int D1 = PermSizes<VB>::D1, D2 = PermSizes<VB>::D2;
  const int pbits = bits_for(static_cast<uint64_t>(nnz));
  const int64_t nb = (nnz + D2 - 1) / D2;
  const uint32_t ntile = static_cast<uint32_t>((nnz + D1 - 1) / D1);
  const int key_bits = pbits + bits_for(static_cast<uint64_t>(nb));
  const int tile_bits = bits_for(ntile);
  const size_t n = static_cast<size_t>(nnz);
  auto round = [](size_t b) { return (b + 255) / 256 * 256; };
  size_t t1 = 0, t2 = 0;
  MSX_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, t1, static_cast<uint64_t *>(nullptr),
                                                 static_cast<uint64_t *>(nullptr),
                                                 static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint32_t *>(nullptr),
                                                 static_cast<int>(nnz), 0, key_bits, stream));
  MSX_HIP_TRY(hipcub::DeviceRadixSort::SortPairs(nullptr, t2, static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint32_t *>(nullptr),
                                                 static_cast<uint64_t *>(nullptr),
                                                 static_cast<uint64_t *>(nullptr),
                                                 static_cast<int>(nnz), 0, tile_bits, stream));
  // A, B: 8 bytes per entry; C, D: 4 bytes; then tile starts and sort temp.
  const size_t bA = round(n * 8), bC = round(n * 4), bT = round((size_t{ntile} + 1) * 8);
  char *work = nullptr;
  MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&work), 2 * bA + 2 * bC + bT + std::max(t1, t2),
                             stream));
  char *A = work, *B = work + bA, *C = work + 2 * bA, *D = work + 2 * bA + bC;
  auto *tstart = reinterpret_cast<int64_t *>(work + 2 * bA + 2 * bC);
  void *tmp = work + 2 * bA + 2 * bC + bT;
  size_t tb1 = t1, tb2 = t2;
  hipError_t e = hipSuccess;
  hipLaunchKernelGGL(layout_keys, dim3(grid_for(nnz)), dim3(kThreads), 0, stream, t_pos, nnz, D2,
                     pbits, reinterpret_cast<uint64_t *>(A), reinterpret_cast<uint32_t *>(C));
  e = hipGetLastError();
  if (e == hipSuccess)
    e = hipcub::DeviceRadixSort::SortPairs(tmp, tb1, reinterpret_cast<uint64_t *>(A),
                                           reinterpret_cast<uint64_t *>(B),
                                           reinterpret_cast<uint32_t *>(C),
                                           reinterpret_cast<uint32_t *>(D), static_cast<int>(nnz), 0,
                                           key_bits, stream);
  if (e == hipSuccess) {
    // sorted (B, D) -> slot2, tile keys in C, tile values in A
    hipLaunchKernelGGL(layout_buckets, dim3(grid_for(nnz)), dim3(kThreads), 0, stream,
                       reinterpret_cast<const uint64_t *>(B), reinterpret_cast<const uint32_t *>(D),
                       nnz, D1, D2, (uint64_t{1} << pbits) - 1, ntile, slot2,
                       reinterpret_cast<uint32_t *>(C), reinterpret_cast<uint64_t *>(A));
    e = hipGetLastError();
  }
  if (e == hipSuccess)
    e = hipcub::DeviceRadixSort::SortPairs(tmp, tb2, reinterpret_cast<uint32_t *>(C),
                                           reinterpret_cast<uint32_t *>(D),
                                           reinterpret_cast<uint64_t *>(A),
                                           reinterpret_cast<uint64_t *>(B), static_cast<int>(nnz), 0,
                                           tile_bits, stream);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(fill<uint16_t>, dim3(grid_for(nnz)), dim3(kThreads), 0, stream, slot1, nnz,
                       kNoSlot);
    hipLaunchKernelGGL(layout_tile_starts, dim3(grid_for(nnz + 1)), dim3(kThreads), 0, stream,
                       reinterpret_cast<const uint32_t *>(D), nnz, ntile, tstart);
    hipLaunchKernelGGL(layout_tiles, dim3(grid_for(nnz)), dim3(kThreads), 0, stream,
                       reinterpret_cast<const uint32_t *>(D), reinterpret_cast<const uint64_t *>(B),
                       tstart, nnz, D1, ntile, src1, slot1);
    e = hipGetLastError();
  }
  msx_status st = MSX_OK;
  if (e != hipSuccess) st = hip_fail(e, "csr_transpose_layout");
  const hipError_t ef = hipFreeAsync(work, stream);
  if (st == MSX_OK && ef != hipSuccess) st = hip_fail(ef, "csr_transpose_layout scratch release");
  return st;
}

template <class S>
msx_status transpose_permute(int64_t nnz, const void *data, const uint16_t *slot1,
                             const uint32_t *src1, const uint16_t *slot2, bool conjugate,
                             void *scratch, void *t_data, hipStream_t stream) {
  constexpr int D1 = PermSizes<sizeof(S)>::D1, D2 = PermSizes<sizeof(S)>::D2;
  // LDS beyond the default dynamic limit, set for the current device
  MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&perm_tiles<S>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, D1 * sizeof(S)));
  MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&perm_buckets<S>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, D2 * sizeof(S)));
  const int64_t ntile = (nnz + D1 - 1) / D1, nb = (nnz + D2 - 1) / D2;
  const size_t qb = 4 * sizeof(S);  // the quad kernels need every buffer aligned to its quad
  const auto al = [](const void *p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; };
  if (al(data, qb) && al(scratch, qb) && al(t_data, qb) && al(slot1, 8) && al(slot2, 8) &&
      al(src1, 16)) {
    MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&perm_tiles_q<S>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, D1 * sizeof(S)));
    MSX_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void *>(&perm_buckets_q<S>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, D2 * sizeof(S)));
    hipLaunchKernelGGL(perm_tiles_q<S>, dim3(static_cast<uint32_t>(ntile)), dim3(kPermThreads),
                       D1 * sizeof(S), stream, static_cast<const S *>(data), slot1, nnz, conjugate,
                       static_cast<S *>(scratch));
    MSX_HIP_TRY(hipGetLastError());
    hipLaunchKernelGGL(perm_buckets_q<S>, dim3(static_cast<uint32_t>(nb)), dim3(kPermThreads),
                       D2 * sizeof(S), stream, static_cast<const S *>(scratch), src1, slot2, nnz,
                       static_cast<S *>(t_data));
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  }
  hipLaunchKernelGGL(perm_tiles<S>, dim3(static_cast<uint32_t>(ntile)), dim3(kPermThreads),
                     D1 * sizeof(S), stream, static_cast<const S *>(data), slot1, nnz, conjugate,
                     static_cast<S *>(scratch));
  MSX_HIP_TRY(hipGetLastError());
  hipLaunchKernelGGL(perm_buckets<S>, dim3(static_cast<uint32_t>(nb)), dim3(kPermThreads),
                     D2 * sizeof(S), stream, static_cast<const S *>(scratch), src1, slot2, nnz,
                     static_cast<S *>(t_data));
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

msx_status check_csr(const char *op, msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                     int64_t nnz, const void *indices, const void *indptr) {
  if (!valid_itype(it)) return fail(MSX_ETYPE, std::string(op) + " requires int32 or int64 indices.");
  if (!valid_vtype(vt)) return fail(MSX_ETYPE, std::string(op) + " unsupported value dtype.");
  if (n_rows < 0 || n_cols < 0 || nnz < 0)
    return fail(MSX_EINVAL, std::string(op) + " shape dimensions must be non-negative.");
  if (n_rows >= kIntMax || n_cols >= kIntMax)
    return fail(MSX_EINVAL, std::string(op) + " shape dimensions must fit in int32.");
  if (nnz >= kIntMax)
    return fail(MSX_EINVAL, std::string(op) + " supports at most 2^31 - 2 stored values.");
  if (indptr == nullptr) return fail(MSX_EINVAL, std::string(op) + " indptr is NULL.");
  if (nnz > 0 && indices == nullptr)
    return fail(MSX_EINVAL, std::string(op) + " indices must be non-NULL when nnz > 0.");
  return MSX_OK;
}

}  // namespace
}  // namespace msx

using namespace msx;

extern "C" msx_status msx_csr_transpose(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                                        int64_t nnz, const void *data, const void *indices,
                                        const void *indptr, void *t_data, void *t_indices,
                                        void *t_indptr, void *stream) {
  clear_error();
  msx_status st = check_csr("csr_transpose", vt, it, n_rows, n_cols, nnz, indices, indptr);
  if (st != MSX_OK) return st;
  if (t_indptr == nullptr || (nnz > 0 && (data == nullptr || t_data == nullptr || t_indices == nullptr)))
    return fail(MSX_EINVAL, "csr_transpose output buffers must be non-NULL.");
  return dispatch<TransposeOp>(vt, it, n_rows, n_cols, nnz, data, indices, indptr, t_data,
                               t_indices, t_indptr, static_cast<hipStream_t>(stream));
}

extern "C" msx_status msx_csr_transpose_positions(msx_itype it, int64_t n_rows, int64_t n_cols,
                                                  int64_t nnz, const void *indices,
                                                  const void *indptr, int32_t *t_pos,
                                                  void *t_indices, void *t_indptr, void *stream) {
  clear_error();
  msx_status st =
      check_csr("csr_transpose_positions", MSX_F32, it, n_rows, n_cols, nnz, indices, indptr);
  if (st != MSX_OK) return st;
  if (t_indptr == nullptr || (nnz > 0 && (t_pos == nullptr || t_indices == nullptr)))
    return fail(MSX_EINVAL, "csr_transpose_positions output buffers must be non-NULL.");
  auto s = static_cast<hipStream_t>(stream);
  if (nnz == 0) {
    if (it == MSX_I64)
      hipLaunchKernelGGL((fill<int64_t>), dim3(grid_for(n_cols + 1)), dim3(kThreads), 0, s,
                         static_cast<int64_t *>(t_indptr), n_cols + 1, int64_t{0});
    else
      hipLaunchKernelGGL((fill<int32_t>), dim3(grid_for(n_cols + 1)), dim3(kThreads), 0, s,
                         static_cast<int32_t *>(t_indptr), n_cols + 1, int32_t{0});
    MSX_HIP_TRY(hipGetLastError());
    return MSX_OK;
  }
  const int end_bit = bits_for(static_cast<uint64_t>(n_cols));
  return it == MSX_I64
             ? transpose_packed<int32_t, int64_t, true>(n_rows, n_cols, nnz, nullptr, indices,
                                                         indptr, t_pos, t_indices, t_indptr,
                                                         end_bit, s)
             : transpose_packed<int32_t, int32_t, true>(n_rows, n_cols, nnz, nullptr, indices,
                                                         indptr, t_pos, t_indices, t_indptr,
                                                         end_bit, s);
}

extern "C" msx_status msx_csr_transpose_values(msx_vtype vt, int64_t nnz, const void *data,
                                               const int32_t *t_pos, int conjugate, void *t_data,
                                               void *stream) {
  clear_error();
  if (!valid_vtype(vt)) return fail(MSX_ETYPE, "csr_transpose_values unsupported value dtype.");
  if (nnz < 0 || nnz >= kIntMax)
    return fail(MSX_EINVAL, "csr_transpose_values supports 0 to 2^31 - 2 stored values.");
  if (nnz > 0 && (data == nullptr || t_pos == nullptr || t_data == nullptr))
    return fail(MSX_EINVAL, "csr_transpose_values buffers must be non-NULL.");
  if (nnz == 0) return MSX_OK;
  auto s = static_cast<hipStream_t>(stream);
  const bool conj = conjugate != 0 && vt == MSX_C64;
  switch (value_bytes(vt)) {
  case 2:
    hipLaunchKernelGGL((gather_positions<uint16_t>), dim3(grid_for(nnz)), dim3(kThreads), 0, s,
                       static_cast<const uint16_t *>(data), nnz, t_pos, nnz, false,
                       static_cast<uint16_t *>(t_data));
    break;
  case 4:
    hipLaunchKernelGGL((gather_positions<uint32_t>), dim3(grid_for(nnz)), dim3(kThreads), 0, s,
                       static_cast<const uint32_t *>(data), nnz, t_pos, nnz, false,
                       static_cast<uint32_t *>(t_data));
    break;
  default:
    hipLaunchKernelGGL((gather_positions<uint64_t>), dim3(grid_for(nnz)), dim3(kThreads), 0, s,
                       static_cast<const uint64_t *>(data), nnz, t_pos, nnz, conj,
                       static_cast<uint64_t *>(t_data));
    break;
  }
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

extern "C" msx_status msx_csr_transpose_layout(msx_vtype vt, int64_t nnz, const int32_t *t_pos,
                                               uint16_t *slot1, uint32_t *src1, uint16_t *slot2,
                                               void *stream) {
  clear_error();
  if (!valid_vtype(vt)) return fail(MSX_ETYPE, "csr_transpose_layout unsupported value dtype.");
  if (nnz < 0 || nnz >= kIntMax)
    return fail(MSX_EINVAL, "csr_transpose_layout supports 0 to 2^31 - 2 stored values.");
  if (nnz > 0 && (t_pos == nullptr || slot1 == nullptr || src1 == nullptr || slot2 == nullptr))
    return fail(MSX_EINVAL, "csr_transpose_layout buffers must be non-NULL.");
  if (nnz == 0) return MSX_OK;
  auto s = static_cast<hipStream_t>(stream);
  switch (value_bytes(vt)) {
  case 2: return transpose_layout_sized<2>(nnz, t_pos, slot1, src1, slot2, s);
  case 4: return transpose_layout_sized<4>(nnz, t_pos, slot1, src1, slot2, s);
  default: return transpose_layout_sized<8>(nnz, t_pos, slot1, src1, slot2, s);
  }
}

extern "C" msx_status msx_csr_transpose_values_layout(msx_vtype vt, int64_t nnz, const void *data,
                                                      const uint16_t *slot1, const uint32_t *src1,
                                                      const uint16_t *slot2, int conjugate,
                                                      void *scratch, void *t_data, void *stream) {
  clear_error();
  if (!valid_vtype(vt))
    return fail(MSX_ETYPE, "csr_transpose_values_layout unsupported value dtype.");
  if (nnz < 0 || nnz >= kIntMax)
    return fail(MSX_EINVAL, "csr_transpose_values_layout supports 0 to 2^31 - 2 stored values.");
  if (nnz > 0 && (data == nullptr || slot1 == nullptr || src1 == nullptr || slot2 == nullptr ||
                  scratch == nullptr || t_data == nullptr))
    return fail(MSX_EINVAL, "csr_transpose_values_layout buffers must be non-NULL.");
  if (nnz == 0) return MSX_OK;
  auto s = static_cast<hipStream_t>(stream);
  const bool conj = conjugate != 0 && vt == MSX_C64;
  switch (value_bytes(vt)) {
  case 2:
    return transpose_permute<uint16_t>(nnz, data, slot1, src1, slot2, false, scratch, t_data, s);
  case 4:
    return transpose_permute<uint32_t>(nnz, data, slot1, src1, slot2, false, scratch, t_data, s);
  default:
    return transpose_permute<uint64_t>(nnz, data, slot1, src1, slot2, conj, scratch, t_data, s);
  }
}

extern "C" msx_status msx_csr_spmv_transpose(msx_vtype vt, msx_itype it, int64_t n_rows,
                                             int64_t n_cols, int64_t nnz, const void *data,
                                             const void *indices, const void *indptr,
                                             const void *x, void *y, void *stream) {
  clear_error();
  msx_status st = check_csr("csr_matvec_transpose", vt, it, n_rows, n_cols, nnz, indices, indptr);
  if (st != MSX_OK) return st;
  if (n_cols > 0 && y == nullptr) return fail(MSX_EINVAL, "csr_matvec_transpose y is NULL.");
  if (nnz > 0 && (data == nullptr || x == nullptr))
    return fail(MSX_EINVAL, "csr_matvec_transpose data and x must be non-NULL.");
  if (n_cols == 0) return MSX_OK;
  return dispatch<SpmvTransposeOp>(vt, it, n_rows, n_cols, nnz, data, indices, indptr, x, y,
                                   static_cast<float *>(nullptr), static_cast<hipStream_t>(stream));
}

extern "C" msx_status msx_csr_spmv_transpose_noalloc(msx_vtype vt, msx_itype it, int64_t n_rows,
                                                     int64_t n_cols, int64_t nnz, const void *data,
                                                     const void *indices, const void *indptr,
                                                     const void *x, void *y, void *stream) {
  clear_error();
  msx_status st =
      check_csr("csr_matvec_transpose_noalloc", vt, it, n_rows, n_cols, nnz, indices, indptr);
  if (st != MSX_OK) return st;
  if (n_cols > 0 && y == nullptr) return fail(MSX_EINVAL, "csr_matvec_transpose_noalloc y is NULL.");
  if (nnz > 0 && (data == nullptr || x == nullptr))
    return fail(MSX_EINVAL, "csr_matvec_transpose_noalloc data and x must be non-NULL.");
  const bool wide_acc = vt == MSX_F16 || vt == MSX_BF16;  // float32 accumulators in `scratch`
  if (wide_acc && n_cols > kNoAllocAccMax)
    return fail(MSX_EINVAL, "csr_matvec_transpose_noalloc: float16/bfloat16 need n_cols <= " +
                                std::to_string(kNoAllocAccMax) +
                                " (the 32 MiB allocation-free scratch), got " +
                                std::to_string(n_cols) + ".");
  float *fixed = nullptr;
  if (wide_acc) {
    st = noalloc_scratch(&fixed);
    if (st != MSX_OK) return st;
  }
  if (n_cols == 0) return MSX_OK;
  return dispatch<SpmvTransposeOp>(vt, it, n_rows, n_cols, nnz, data, indices, indptr, x, y, fixed,
                                   static_cast<hipStream_t>(stream));
}

extern "C" msx_status msx_csr_spmm_transpose(msx_vtype vt, msx_itype it, int64_t n_rows,
                                             int64_t n_cols, int64_t nnz, const void *data,
                                             const void *indices, const void *indptr, int64_t k,
                                             const void *X, int64_t ldx, void *Y, int64_t ldy,
                                             void *stream) {
  clear_error();
  msx_status st = check_csr("csr_matmul_transpose", vt, it, n_rows, n_cols, nnz, indices, indptr);
  if (st != MSX_OK) return st;
  if (k < 0 || k >= kIntMax) return fail(MSX_EINVAL, "csr_matmul_transpose rhs column count must fit in int32.");
  if (ldx < k || ldy < k)
    return fail(MSX_EINVAL, "csr_matmul_transpose leading dimensions must be at least the column count.");
  if (n_cols > 0 && k > 0 && Y == nullptr) return fail(MSX_EINVAL, "csr_matmul_transpose Y is NULL.");
  if (nnz > 0 && k > 0 && (data == nullptr || X == nullptr))
    return fail(MSX_EINVAL, "csr_matmul_transpose data and X must be non-NULL.");
  if (n_cols == 0 || k == 0) return MSX_OK;
  return dispatch<SpmmTransposeOp>(vt, it, n_rows, n_cols, nnz, data, indices, indptr, k, X, ldx,
                                   Y, ldy, static_cast<hipStream_t>(stream));
}

extern "C" msx_status msx_csr_spmv_data_vjp(msx_vtype vt, msx_itype it, int64_t n_rows,
                                            int64_t n_cols, int64_t nnz, const void *indices,
                                            const void *indptr, const void *x, const void *cot,
                                            void *out, const msx_csr_plan *plan, void *stream) {
  clear_error();
  msx_status st = check_csr("csr_matvec_data_vjp", vt, it, n_rows, n_cols, nnz, indices, indptr);
  if (st != MSX_OK) return st;
  // The gradient does not read the values: a plan bound to this matrix is
  // accepted whatever values it was bound to.
  st = check_plan("csr_matvec_data_vjp", plan, vt, it, n_rows, n_cols, nnz,
                  plan != nullptr ? plan->bound_data : nullptr, indices, indptr);
  if (st != MSX_OK) return st;
  if (nnz > 0 && (out == nullptr || cot == nullptr || (n_cols > 0 && x == nullptr)))
    return fail(MSX_EINVAL, "csr_matvec_data_vjp buffers must be non-NULL.");
  if (nnz == 0 || n_rows == 0) return MSX_OK;
  // A panel plan turns the gather of x into LDS reads (two streaming passes)
  // when its copy holds every value (no invalid column was dropped).
  if (plan != nullptr && plan->bound && plan->vtype == vt && panel_data_vjp_fits(plan))
    return launch_panel_data_vjp(plan, indptr, x, cot, out, static_cast<hipStream_t>(stream));
  return dispatch<SpmvDataVjpOp>(vt, it, n_rows, n_cols, nnz, indices, indptr, x, cot, out,
                                 static_cast<hipStream_t>(stream));
}

extern "C" msx_status msx_csr_spmm_data_vjp(msx_vtype vt, msx_itype it, int64_t n_rows,
                                            int64_t n_cols, int64_t nnz, const void *indices,
                                            const void *indptr, int64_t k, const void *X,
                                            int64_t ldx, const void *cot, int64_t ldc, void *out,
                                            void *stream) {
  clear_error();
  msx_status st = check_csr("csr_matmul_data_vjp", vt, it, n_rows, n_cols, nnz, indices, indptr);
  if (st != MSX_OK) return st;
  if (k < 0 || k >= kIntMax) return fail(MSX_EINVAL, "csr_matmul_data_vjp rhs column count must fit in int32.");
  if (ldx < k || ldc < k)
    return fail(MSX_EINVAL, "csr_matmul_data_vjp leading dimensions must be at least the column count.");
  if (nnz > 0 && (out == nullptr || (k > 0 && (cot == nullptr || (n_cols > 0 && X == nullptr)))))
    return fail(MSX_EINVAL, "csr_matmul_data_vjp buffers must be non-NULL.");
  if (nnz == 0 || n_rows == 0) return MSX_OK;
  return dispatch<SpmmDataVjpOp>(vt, it, n_rows, n_cols, nnz, indices, indptr, k, X, ldx, cot, ldc,
                                 out, static_cast<hipStream_t>(stream));
}
