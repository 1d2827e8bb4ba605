// csr_long_slice.hip - long rows of the SpMV summed per XCD column slice.
//
// Long rows (more than W values) gather x all over its range; on the
// power-law matrix (2 M columns, 8 MB of x) most of those gathers miss the
// 4 MB L2 of the XCD that makes them.  When a long row's columns are sorted
// (canonical CSR), the values whose columns lie in slice s = [s * Wc,
// (s + 1) * Wc), Wc = ceil(n_cols / 8), form one contiguous stretch of the
// row.  A bound plan records those stretches, cut into pieces of at most
// kLongPieceMax values, grouped by slice; the pieces of slice s run on XCD s
// (the hardware hands workgroup g to XCD g % 8), so every XCD gathers from
// its eighth of x, which stays in its L2.  The matrix is read in place: no
// copy.  One wave sums a piece (quads of 4 values per lane, then a
// fixed-order butterfly) into the piece's slot; a fixup sums each row's
// slots with a fixed-order tree.  Results are deterministic.  Like the
// chunked long-row kernel this is not the reference's stored order, so long
// rows match the reference within tolerance.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "msx_device.h"
#include "msx_internal.h"
#include "msx_long_slice.h"

namespace msx {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerGroup = kThreads / kWave;
constexpr uint32_t kMaxGrid = 1u << 20;
// x must be at least this large for the slicing to pay: below it, x fits
// one XCD's L2 anyway.
constexpr int64_t kLongSliceMinX = int64_t{4} << 20;

__device__ inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// One workgroup per long row: whether its columns are sorted (a descent
// anywhere sets *unsorted), and its kSlices + 1 stretch boundaries
// (thread t in 1..7 finds the first position whose column is >= t * Wc).
template <class I>
__global__ void __launch_bounds__(kThreads)
    long_splits(const I *__restrict__ indices, const I *__restrict__ indptr,
                const int32_t *__restrict__ long_rows, int64_t nnz, int64_t slice_width,
                int64_t *__restrict__ splits, unsigned int *__restrict__ unsorted) {
  const int64_t li = blockIdx.x;
  const int64_t row = long_rows[li];
  const int64_t rb = clamp64(static_cast<int64_t>(indptr[row]), 0, nnz);
  const int64_t re = clamp64(static_cast<int64_t>(indptr[row + 1]), rb, nnz);
  const int64_t len = re - rb;
  bool bad = len * static_cast<int64_t>(sizeof(I)) > static_cast<int64_t>(kGatherMaxBytes);
  if (!bad) {
    // four unconditional pairs per thread and step (past the row: masked)
    const auto rr = make_rsrc(indices + rb, static_cast<uint64_t>(len) * sizeof(I));
    for (int64_t b = 0; b + 1 < len; b += 4 * kThreads) {
      I a[4], n[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t off = static_cast<uint32_t>(b + threadIdx.x + u * kThreads);
        a[u] = buffer_index<I>(rr, off * sizeof(I));
        n[u] = buffer_index<I>(rr, (off + 1) * sizeof(I));
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (b + threadIdx.x + u * kThreads + 1 < len && a[u] > n[u]) bad = true;
    }
  }
  if (__syncthreads_or(bad)) {
    if (threadIdx.x == 0) atomicOr(unsorted, 1u);
    return;
  }
  if (threadIdx.x <= static_cast<unsigned>(kSlices)) {
    const int t = static_cast<int>(threadIdx.x);
    int64_t pos = t == 0 ? rb : re;
    if (t > 0 && t < kSlices) {  // lower bound of t * Wc in [rb, re)
      const int64_t key = t * slice_width;
      int64_t lo = rb, hi = re;
      while (lo < hi) {
        const int64_t mid = lo + (hi - lo) / 2;
        if (static_cast<int64_t>(indices[mid]) < key) lo = mid + 1;
        else hi = mid;
      }
      pos = lo;
    }
    splits[li * (kSlices + 1) + t] = pos;
  }
}

template <class V, class I, int AUX>
__global__ void __launch_bounds__(kThreads)
    spmv_long_sliced(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                     const typename V::Storage *__restrict__ x, uint32_t x_bytes, int64_t n_cols,
                     const int64_t *__restrict__ ls_begin, const int32_t *__restrict__ ls_len,
                     const int32_t *__restrict__ ls_slot,
                     const int32_t *__restrict__ ls_slice_begin,
                     typename V::Acc *__restrict__ partial) {
  long_pieces<V, I, AUX>(data, indices, x, x_bytes, n_cols, ls_begin, ls_len, ls_slot,
                         ls_slice_begin, partial, blockIdx.x, gridDim.x);
}

// One wave per long row: its slots in a fixed-order tree.
template <class V>
__global__ void __launch_bounds__(kThreads)
    long_sliced_fixup(typename V::Storage *__restrict__ y, const int32_t *__restrict__ long_rows,
                      const int32_t *__restrict__ ls_row_slot,
                      const typename V::Acc *__restrict__ partial, int64_t n_long) {
  using A = typename V::Acc;
  const int lane = threadIdx.x % kWave;
  const int64_t li = static_cast<int64_t>(blockIdx.x) * kWavesPerGroup + threadIdx.x / kWave;
  if (li >= n_long) return;
  A acc = vzero<A>();
  for (int64_t k = ls_row_slot[li] + lane; k < ls_row_slot[li + 1]; k += kWave)
    acc = vadd(acc, partial[k]);
#pragma unroll
  for (int d = kWave / 2; d >= 1; d >>= 1) acc = vadd(acc, shfl_xor(acc, d));
  if (lane == 0) y[long_rows[li]] = V::narrow(acc);
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

template <class I>
msx_status build_typed(msx_csr_plan *p, const void *indices, const void *indptr,
                       hipStream_t stream) {
  const int64_t n_long = p->n_long;
  const int64_t wc = (p->n_cols + kSlices - 1) / kSlices;
  const size_t b_splits = sizeof(int64_t) * static_cast<size_t>(n_long) * (kSlices + 1);
  char *tmp = nullptr;
  if (hipMallocAsync(reinterpret_cast<void **>(&tmp), b_splits + 256, stream) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MSX_ENOMEM, "msx_csr_plan_create_bound: device allocation of the long-row slices failed.");
  }
  auto *d_splits = reinterpret_cast<int64_t *>(tmp);
  auto *d_flag = reinterpret_cast<unsigned int *>(tmp + b_splits);
  std::vector<int64_t> splits(static_cast<size_t>(n_long) * (kSlices + 1));
  unsigned int flag = 0;
  hipError_t e = hipMemsetAsync(d_flag, 0, sizeof(unsigned int), stream);
  if (e == hipSuccess) {
    hipLaunchKernelGGL((long_splits<I>), dim3(static_cast<uint32_t>(n_long)), dim3(kThreads), 0,
                       stream, static_cast<const I *>(indices), static_cast<const I *>(indptr),
                       p->long_rows, p->nnz, wc, d_splits, d_flag);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(&flag, d_flag, sizeof(flag), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(splits.data(), d_splits, b_splits, hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  (void)hipFreeAsync(tmp, stream);
  if (e != hipSuccess) return hip_fail(e, "long-row slices");
  if (flag != 0) return MSX_OK;  // a long row with unsorted columns: keep the chunked kernel

  // Pieces grouped by slice; slots in (row, slice, piece) order.
  std::vector<std::vector<int64_t>> begin(kSlices);
  std::vector<std::vector<int32_t>> len(kSlices), slot(kSlices);
  std::vector<int32_t> row_slot(static_cast<size_t>(n_long) + 1);
  int64_t n_units = 0;
  for (int64_t li = 0; li < n_long; ++li) {
    row_slot[li] = static_cast<int32_t>(n_units);
    for (int s = 0; s < kSlices; ++s) {
      const int64_t b = splits[li * (kSlices + 1) + s];
      const int64_t e2 = splits[li * (kSlices + 1) + s + 1];
      for (int64_t q = b; q < e2; q += kLongPieceMax) {
        begin[s].push_back(q);
        len[s].push_back(static_cast<int32_t>(std::min<int64_t>(kLongPieceMax, e2 - q)));
        slot[s].push_back(static_cast<int32_t>(n_units++));
        if (n_units >= (int64_t{1} << 31) - 1) return MSX_OK;  // keep the chunked kernel
      }
    }
  }
  row_slot[n_long] = static_cast<int32_t>(n_units);
  if (n_units == 0) return MSX_OK;
  std::vector<int64_t> h_begin;
  std::vector<int32_t> h_len, h_slot, h_slice(kSlices + 1, 0);
  h_begin.reserve(n_units);
  h_len.reserve(n_units);
  h_slot.reserve(n_units);
  int64_t slice_max = 0;
  for (int s = 0; s < kSlices; ++s) {
    h_slice[s] = static_cast<int32_t>(h_begin.size());
    h_begin.insert(h_begin.end(), begin[s].begin(), begin[s].end());
    h_len.insert(h_len.end(), len[s].begin(), len[s].end());
    h_slot.insert(h_slot.end(), slot[s].begin(), slot[s].end());
    slice_max = std::max<int64_t>(slice_max, static_cast<int64_t>(begin[s].size()));
  }
  h_slice[kSlices] = static_cast<int32_t>(h_begin.size());

  const size_t u = static_cast<size_t>(n_units);
  const size_t o_len = align_up(sizeof(int64_t) * u, 256);
  const size_t o_slot = o_len + align_up(sizeof(int32_t) * u, 256);
  const size_t o_slice = o_slot + align_up(sizeof(int32_t) * u, 256);
  const size_t o_row = o_slice + align_up(sizeof(int32_t) * (kSlices + 1), 256);
  const size_t o_part = o_row + align_up(sizeof(int32_t) * (n_long + 1), 256);
  const size_t total = o_part + align_up(8 * u, 256);
  char *base = nullptr;
  if (hipMalloc(&base, total) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MSX_ENOMEM, "msx_csr_plan_create_bound: device allocation of the long-row slices failed.");
  }
  p->ls_base = base;
  p->ls_bytes = total;
  p->ls_begin = reinterpret_cast<int64_t *>(base);
  p->ls_len = reinterpret_cast<int32_t *>(base + o_len);
  p->ls_slot = reinterpret_cast<int32_t *>(base + o_slot);
  p->ls_slice_begin = reinterpret_cast<int32_t *>(base + o_slice);
  p->ls_row_slot = reinterpret_cast<int32_t *>(base + o_row);
  p->ls_partial = base + o_part;
  MSX_HIP_TRY(hipMemcpyAsync(p->ls_begin, h_begin.data(), sizeof(int64_t) * u, hipMemcpyHostToDevice, stream));
  MSX_HIP_TRY(hipMemcpyAsync(p->ls_len, h_len.data(), sizeof(int32_t) * u, hipMemcpyHostToDevice, stream));
  MSX_HIP_TRY(hipMemcpyAsync(p->ls_slot, h_slot.data(), sizeof(int32_t) * u, hipMemcpyHostToDevice, stream));
  MSX_HIP_TRY(hipMemcpyAsync(p->ls_slice_begin, h_slice.data(), sizeof(int32_t) * (kSlices + 1),
                             hipMemcpyHostToDevice, stream));
  MSX_HIP_TRY(hipMemcpyAsync(p->ls_row_slot, row_slot.data(), sizeof(int32_t) * (n_long + 1),
                             hipMemcpyHostToDevice, stream));
  MSX_HIP_TRY(hipStreamSynchronize(stream));  // the host vectors end here
  p->ls_units = n_units;
  p->ls_slice_max = slice_max;
  return MSX_OK;
}

template <class V>
void launch_fixup(const msx_csr_plan *p, void *y, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int64_t groups = (p->n_long + kWavesPerGroup - 1) / kWavesPerGroup;
  hipLaunchKernelGGL((long_sliced_fixup<V>), dim3(static_cast<uint32_t>(groups)), dim3(kThreads), 0,
                     stream, static_cast<S *>(y), p->long_rows, p->ls_row_slot,
                     static_cast<const A *>(p->ls_partial), p->n_long);
}

template <class V, class I>
void launch_typed(const msx_csr_plan *p, const void *data, const void *indices, const void *x,
                  void *y, uint32_t x_bytes, bool stream_nt, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int64_t per_slice = std::min<int64_t>((p->ls_slice_max + kWavesPerGroup - 1) / kWavesPerGroup,
                                              kMaxGrid / kSlices);
  const dim3 grid(static_cast<uint32_t>(std::max<int64_t>(per_slice, 1) * kSlices));
  auto kernel = stream_nt ? spmv_long_sliced<V, I, kCacheStream> : spmv_long_sliced<V, I, kCacheDefault>;
  hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, stream, static_cast<const S *>(data),
                     static_cast<const I *>(indices), static_cast<const S *>(x), x_bytes, p->n_cols,
                     p->ls_begin, p->ls_len, p->ls_slot, p->ls_slice_begin,
                     static_cast<A *>(p->ls_partial));
  launch_fixup<V>(p, y, stream);
}

template <class V>
void launch_v(const msx_csr_plan *p, const void *data, const void *indices, const void *x, void *y,
              uint32_t x_bytes, bool stream_nt, hipStream_t stream) {
  if (p->itype == MSX_I32) launch_typed<V, int32_t>(p, data, indices, x, y, x_bytes, stream_nt, stream);
  else launch_typed<V, int64_t>(p, data, indices, x, y, x_bytes, stream_nt, stream);
}

}  // namespace

msx_status build_long_slices(msx_csr_plan *p, const void *indices, const void *indptr,
                             hipStream_t stream) {
  const int64_t x_bytes = p->n_cols * static_cast<int64_t>(value_bytes(p->vtype));
  if (p->n_long == 0 || x_bytes < kLongSliceMinX || p->n_long >= (int64_t{1} << 31)) return MSX_OK;
  return p->itype == MSX_I32 ? build_typed<int32_t>(p, indices, indptr, stream)
                             : build_typed<int64_t>(p, indices, indptr, stream);
}

msx_status launch_long_sliced(const msx_csr_plan *p, const void *data, const void *indices,
                              const void *x, void *y, uint32_t x_bytes, bool stream_nt,
                              hipStream_t stream) {
  switch (p->vtype) {
  case MSX_F32: launch_v<F32>(p, data, indices, x, y, x_bytes, stream_nt, stream); break;
  case MSX_F16: launch_v<F16>(p, data, indices, x, y, x_bytes, stream_nt, stream); break;
  case MSX_BF16: launch_v<BF16>(p, data, indices, x, y, x_bytes, stream_nt, stream); break;
  case MSX_C64: launch_v<C64>(p, data, indices, x, y, x_bytes, stream_nt, stream); break;
  }
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

msx_status launch_long_sliced_fixup(const msx_csr_plan *p, void *y, hipStream_t stream) {
  switch (p->vtype) {
  case MSX_F32: launch_fixup<F32>(p, y, stream); break;
  case MSX_F16: launch_fixup<F16>(p, y, stream); break;
  case MSX_BF16: launch_fixup<BF16>(p, y, stream); break;
  case MSX_C64: launch_fixup<C64>(p, y, stream); break;
  }
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

}  // namespace msx
