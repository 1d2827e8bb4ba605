// csr_slice.hip - XCD column slicing for SpMV with a scattered x gather.
//
// Why: MI355X has 8 XCDs, each with its own 4 MB L2.  When a matrix's
// columns are scattered over an x larger than that (the 4M-row random
// matrix: x is 16.8 MB), every XCD gathers from all of x, misses L2 on most
// gathers and pulls a whole 128-byte line from the Infinity Cache for each
// 4-byte value - 7.2 GB of fabric traffic for 0.59 GB of matrix.
//
// What: the plan partitions the columns into 8 slices of width Wc and, inside
// every short block, stably reorders the block's values by slice (same
// position range [p0, p1) of the block, so the copy is exactly nnz long).
// Each value's index is packed as (row_in_block << col_bits) | (col - s*Wc).
// The SpMV then runs slice s only on workgroups g with g % 8 == s - the
// hardware hands workgroup g to XCD g % 8 - so XCD s only ever gathers from
// x[s*Wc, (s+1)*Wc), about 2 MB, which stays in its L2.  Each (block, slice)
// wave sums its rows in stored order into partial[s][row]; a merge kernel
// adds the 8 partials in slice order.  Long rows keep the unsliced path.
//
// Summation order therefore differs from the reference's (per row: 8 slice
// sums, each in stored order, added in slice order); results agree within
// the path's tolerance and are identical from call to call.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "msx_device.h"
#include "msx_internal.h"

namespace msx {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerGroup = kThreads / kWave;
constexpr int kRows = 256;  // rows per short block at most (plan R)
constexpr uint32_t kMaxGrid = 1u << 20;
constexpr uint32_t kLongFlag = 0x80000000u;

__device__ inline int64_t clamp64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline uint64_t lanemask_lt(int lane) {
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

struct BlockRange {
  bool valid;
  int64_t r0, p0, p1;
  int m;
};

// The short block of bounds entry b, clamped as the SpMV kernel clamps it.
template <int W>
__device__ inline BlockRange block_range(const int32_t *bounds, const int64_t *bounds_nnz, int64_t b,
                                         int64_t nnz) {
  BlockRange br{};
  const uint32_t e0 = static_cast<uint32_t>(bounds[b]);
  if (e0 & kLongFlag) return br;
  br.valid = true;
  br.r0 = e0;
  const int64_t r1 = static_cast<uint32_t>(bounds[b + 1]) & ~kLongFlag;
  br.m = static_cast<int>(std::min<int64_t>(r1 - br.r0, kRows));
  br.p0 = clamp64(bounds_nnz[b], 0, nnz);
  br.p1 = clamp64(bounds_nnz[b + 1], br.p0, std::min<int64_t>(nnz, br.p0 + 2 * W - 1));
  return br;
}

// ---------------------------------------------------------------------------
// Probe: count short blocks whose valid columns span more than n_cols / 4.
template <class I, int W>
__global__ void __launch_bounds__(kThreads)
    slice_probe(const I *__restrict__ indices, const int32_t *__restrict__ bounds,
                const int64_t *__restrict__ bounds_nnz, int64_t n_bounds, int64_t nnz,
                int64_t n_cols, unsigned long long *__restrict__ scattered) {
  const int lane = threadIdx.x % kWave;
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kWavesPerGroup + threadIdx.x / kWave;
  if (b >= n_bounds) return;
  const BlockRange br = block_range<W>(bounds, bounds_nnz, b, nnz);
  if (!br.valid || br.p1 <= br.p0) return;
  int64_t lo = INT64_MAX, hi = -1;
  for (int64_t p = br.p0 + lane; p < br.p1; p += kWave) {
    const int64_t c = static_cast<int64_t>(indices[p]);
    if (static_cast<uint64_t>(c) < static_cast<uint64_t>(n_cols)) {
      lo = c < lo ? c : lo;
      hi = c > hi ? c : hi;
    }
  }
  for (int d = kWave / 2; d >= 1; d >>= 1) {
    const int64_t ol = __shfl_xor(lo, d, kWave);
    const int64_t oh = __shfl_xor(hi, d, kWave);
    lo = ol < lo ? ol : lo;
    hi = oh > hi ? oh : hi;
  }
  if (lane == 0 && hi >= lo && hi - lo > n_cols / 4) atomicAdd(scattered, 1ull);
}

// ---------------------------------------------------------------------------
// Build: per short block (one wave), count values per slice, then scatter
// them stably to [p0 + seg[s], p0 + seg[s+1]).  Values with a column outside
// [0, n_cols) are dropped (they add nothing to y).
template <class V, class I, int W>
__global__ void __launch_bounds__(kThreads)
    slice_build(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                const I *__restrict__ indptr, const int32_t *__restrict__ bounds,
                const int64_t *__restrict__ bounds_nnz, int64_t n_bounds, int64_t nnz,
                int64_t n_cols, int64_t slice_width, int col_bits,
                typename V::Storage *__restrict__ s_data, uint32_t *__restrict__ s_col,
                uint16_t *__restrict__ s_seg) {
  __shared__ int32_t lds_rp[kWavesPerGroup][kRows + 1];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  int32_t *rp = lds_rp[wave];
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kWavesPerGroup + wave;
  if (b >= n_bounds) return;
  uint16_t *seg = s_seg + b * (kSlices + 1);
  const BlockRange br = block_range<W>(bounds, bounds_nnz, b, nnz);
  if (!br.valid) {
    if (lane <= kSlices) seg[lane] = 0;
    return;
  }
  for (int i = lane; i <= br.m; i += kWave)
    rp[i] = static_cast<int32_t>(clamp64(static_cast<int64_t>(indptr[br.r0 + i]), br.p0, br.p1) - br.p0);
  wave_lds_sync();
  const int n = static_cast<int>(br.p1 - br.p0);
  auto slice_of = [&](int e, int64_t &col) -> int {
    col = static_cast<int64_t>(indices[br.p0 + e]);
    if (static_cast<uint64_t>(col) >= static_cast<uint64_t>(n_cols)) return kSlices;
    return static_cast<int>(col / slice_width);
  };
  // pass 1: counts per slice
  int count[kSlices];
#pragma unroll
  for (int s = 0; s < kSlices; ++s) count[s] = 0;
  for (int c0 = 0; c0 < n; c0 += kWave) {
    const int e = c0 + lane;
    int64_t col = 0;
    const int sl = e < n ? slice_of(e, col) : kSlices;
#pragma unroll
    for (int s = 0; s < kSlices; ++s) count[s] += __popcll(__ballot(sl == s));
  }
  int start[kSlices + 1];
  start[0] = 0;
#pragma unroll
  for (int s = 0; s < kSlices; ++s) start[s + 1] = start[s] + count[s];
  if (lane <= kSlices) {
    int v = 0;
#pragma unroll
    for (int s = 0; s <= kSlices; ++s) v = lane == s ? start[s] : v;
    seg[lane] = static_cast<uint16_t>(v);
  }
  // pass 2: stable scatter
  int run[kSlices];
#pragma unroll
  for (int s = 0; s < kSlices; ++s) run[s] = start[s];
  const uint64_t lt = lanemask_lt(lane);
  for (int c0 = 0; c0 < n; c0 += kWave) {
    const int e = c0 + lane;
    int64_t col = 0;
    const int sl = e < n ? slice_of(e, col) : kSlices;
    int dest = -1;
#pragma unroll
    for (int s = 0; s < kSlices; ++s) {
      const uint64_t mask = __ballot(sl == s);
      if (sl == s) dest = run[s] + __popcll(mask & lt);
      run[s] += __popcll(mask);
    }
    if (dest >= 0) {
      // row of element e: last row whose start is <= e
      int lo = 0, hi = br.m;  // rp[lo] <= e < rp[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (rp[mid] <= e) lo = mid;
        else hi = mid;
      }
      const int64_t q = br.p0 + dest;
      s_data[q] = data[br.p0 + e];
      s_col[q] = (static_cast<uint32_t>(lo) << col_bits) |
                 static_cast<uint32_t>(col - static_cast<int64_t>(sl) * slice_width);
    }
  }
}

// ---------------------------------------------------------------------------
// SpMV over one (short block, slice) per wave; workgroup g serves slice g % 8.
template <class V, int W>
__global__ void __launch_bounds__(kThreads)
    spmv_sliced(const typename V::Storage *__restrict__ s_data, const uint32_t *__restrict__ s_col,
                const uint16_t *__restrict__ s_seg, const typename V::Storage *__restrict__ x,
                typename V::Acc *__restrict__ partial, const int32_t *__restrict__ bounds,
                const int64_t *__restrict__ bounds_nnz, int64_t n_bounds, int64_t n_rows,
                int64_t nnz, int64_t slice_width, int col_bits) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  constexpr int kQuads = W / 2 + 1;
  constexpr int QPL = (kQuads + kWave - 1) / kWave;
  constexpr int kCap = 4 * kQuads;
  __shared__ A lds_prod[kWavesPerGroup][kCap];
  __shared__ uint8_t lds_row[kWavesPerGroup][kCap];
  __shared__ uint16_t lds_rs[kWavesPerGroup][kRows];
  __shared__ uint16_t lds_re[kWavesPerGroup][kRows];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  A *prod = lds_prod[wave];
  uint8_t *rowid = lds_row[wave];
  uint16_t *rs = lds_rs[wave];
  uint16_t *re = lds_re[wave];
  const uint32_t col_mask = (1u << col_bits) - 1u;
  const int s = static_cast<int>(blockIdx.x % kSlices);
  const S *xs = x + static_cast<int64_t>(s) * slice_width;
  A *part = partial + static_cast<int64_t>(s) * n_rows;

  for (int64_t g = blockIdx.x / kSlices; g * kWavesPerGroup < n_bounds; g += gridDim.x / kSlices) {
    const int64_t b = g * kWavesPerGroup + wave;
    if (b >= n_bounds) break;
    const BlockRange br = block_range<W>(bounds, bounds_nnz, b, nnz);
    if (!br.valid) continue;
    const uint16_t *seg = s_seg + b * (kSlices + 1);
    const int64_t lo = br.p0 + seg[s];
    const int64_t hi = std::min<int64_t>(br.p0 + seg[s + 1], br.p1);
    const int cnt = static_cast<int>(hi > lo ? hi - lo : 0);
    const int64_t a0 = lo & ~int64_t{3};
    const int nq = static_cast<int>((hi - a0 + 3) >> 2);
    for (int i = lane; i < br.m; i += kWave) {
      rs[i] = 0;
      re[i] = 0;
    }
    const auto rc = make_rsrc(s_col + a0, static_cast<uint64_t>(nnz - a0) * sizeof(uint32_t));
    const auto rd = make_rsrc(s_data + a0, static_cast<uint64_t>(nnz - a0) * sizeof(S));
    Quad<uint32_t> cq[QPL];
    Quad<S> dq[QPL];
#pragma unroll
    for (int k = 0; k < QPL; ++k) {
      const int q = lane + k * kWave;
      if (q < nq) {
        cq[k] = load_quad<uint32_t>(rc, static_cast<uint32_t>(q) * 16u);
        dq[k] = load_quad<S>(rd, static_cast<uint32_t>(q) * 4u * sizeof(S));
      }
    }
    S xv[QPL][4];
#pragma unroll
    for (int k = 0; k < QPL; ++k) {
      const int q = lane + k * kWave;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t pos = a0 + 4 * q + e;
        xv[k][e] = S{};
        if (q < nq && pos >= lo && pos < hi) xv[k][e] = xs[cq[k].v[e] & col_mask];
      }
    }
#pragma unroll
    for (int k = 0; k < QPL; ++k) {
      const int q = lane + k * kWave;
      if (q < nq) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t pos = a0 + 4 * q + e;
          if (pos >= lo && pos < hi) {
            const int t = static_cast<int>(pos - lo);
            prod[t] = vmul<V>(dq[k].v[e], xv[k][e]);
            rowid[t] = static_cast<uint8_t>(cq[k].v[e] >> col_bits);
          }
        }
      }
    }
    wave_lds_sync();
    // run boundaries of each row inside the slice segment (rows ascend)
    for (int t = lane; t < cnt; t += kWave) {
      const int r = rowid[t];
      if (t == 0 || rowid[t - 1] != r) rs[r] = static_cast<uint16_t>(t);
      if (t == cnt - 1 || rowid[t + 1] != r) re[r] = static_cast<uint16_t>(t + 1);
    }
    wave_lds_sync();
    for (int i = lane; i < br.m; i += kWave) {
      A acc = vzero<A>();
      for (int t = rs[i]; t < re[i]; ++t) acc = vadd(acc, prod[t]);
      part[br.r0 + i] = acc;
    }
    wave_lds_sync();
  }
}

// y[r] = partial[0][r] + ... + partial[7][r], in slice order.
template <class V>
__global__ void __launch_bounds__(kThreads)
    slice_merge(const typename V::Acc *__restrict__ partial, typename V::Storage *__restrict__ y,
                int64_t n_rows) {
  using A = typename V::Acc;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; r < n_rows;
       r += static_cast<int64_t>(gridDim.x) * kThreads) {
    A acc = partial[r];
#pragma unroll
    for (int s = 1; s < kSlices; ++s) acc = vadd(acc, partial[static_cast<int64_t>(s) * n_rows + r]);
    y[r] = V::narrow(acc);
  }
}

int bits_for(int64_t v) {  // smallest b with v <= 2^b
  int b = 0;
  while ((int64_t{1} << b) < v) ++b;
  return b;
}

template <class V, class I, int W>
msx_status build_typed(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                       hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int64_t groups = (p->n_bounds + kWavesPerGroup - 1) / kWavesPerGroup;
  if (p->slice_mode == MSX_SLICE_AUTO) {
    if (p->n_cols * static_cast<int64_t>(sizeof(S)) < (int64_t{8} << 20) || groups == 0) return MSX_OK;
    unsigned long long *counter = nullptr;
    MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&counter), sizeof(*counter), stream));
    MSX_HIP_TRY(hipMemsetAsync(counter, 0, sizeof(*counter), stream));
    hipLaunchKernelGGL((slice_probe<I, W>), dim3(static_cast<uint32_t>(groups)), dim3(kThreads), 0,
                       stream, static_cast<const I *>(indices), p->bounds, p->bounds_nnz,
                       p->n_bounds, p->nnz, p->n_cols, counter);
    unsigned long long scattered = 0;
    hipError_t e = hipGetLastError();
    if (e == hipSuccess)
      e = hipMemcpyAsync(&scattered, counter, sizeof(scattered), hipMemcpyDeviceToHost, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    (void)hipFreeAsync(counter, stream);
    if (e != hipSuccess) return hip_fail(e, "slice probe");
    if (2 * static_cast<int64_t>(scattered) <= p->n_blocks) return MSX_OK;  // mostly local
  }
  const int64_t width = ((p->n_cols + kSlices - 1) / kSlices + 31) / 32 * 32;
  const int col_bits = std::max(1, bits_for(width));
  if (col_bits > 24 || groups == 0) return MSX_OK;  // needs 8 bits for the row in block
  const size_t b_data = ((static_cast<size_t>(p->nnz) * sizeof(S) + 255) / 256) * 256;
  const size_t b_col = ((static_cast<size_t>(p->nnz) * 4 + 255) / 256) * 256;
  const size_t b_seg = ((static_cast<size_t>(p->n_bounds) * (kSlices + 1) * 2 + 255) / 256) * 256;
  const size_t b_part = static_cast<size_t>(kSlices) * p->n_rows * sizeof(A);
  char *base = nullptr;
  if (hipMalloc(&base, b_data + b_col + b_seg + b_part) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MSX_ENOMEM, "msx_csr_plan_create_bound: device allocation of the sliced copy failed.");
  }
  p->s_base = base;
  p->s_data = base;
  p->s_col = reinterpret_cast<uint32_t *>(base + b_data);
  p->s_seg = reinterpret_cast<uint16_t *>(base + b_data + b_col);
  p->s_partial = base + b_data + b_col + b_seg;
  p->s_bytes = b_data + b_col + b_seg + b_part;
  p->slice_width = width;
  p->col_bits = col_bits;
  hipLaunchKernelGGL((slice_build<V, I, W>), dim3(static_cast<uint32_t>(groups)), dim3(kThreads), 0,
                     stream, static_cast<const S *>(data), static_cast<const I *>(indices),
                     static_cast<const I *>(indptr), p->bounds, p->bounds_nnz, p->n_bounds, p->nnz,
                     p->n_cols, width, col_bits, static_cast<S *>(p->s_data), p->s_col, p->s_seg);
  MSX_HIP_TRY(hipGetLastError());
  MSX_HIP_TRY(hipStreamSynchronize(stream));
  p->n_slices = kSlices;
  return MSX_OK;
}

template <class V, class I>
msx_status build_w(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                   hipStream_t stream) {
  switch (p->block_nnz) {
  case 64: return build_typed<V, I, 64>(p, data, indices, indptr, stream);
  case 128: return build_typed<V, I, 128>(p, data, indices, indptr, stream);
  case 256: return build_typed<V, I, 256>(p, data, indices, indptr, stream);
  case 512: return build_typed<V, I, 512>(p, data, indices, indptr, stream);
  default: return build_typed<V, I, 1024>(p, data, indices, indptr, stream);
  }
}

template <class V>
msx_status build_v(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                   hipStream_t stream) {
  return p->itype == MSX_I32 ? build_w<V, int32_t>(p, data, indices, indptr, stream)
                             : build_w<V, int64_t>(p, data, indices, indptr, stream);
}

template <class V, int W>
void launch_w(const msx_csr_plan *p, const void *x, void *y, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int64_t groups = (p->n_bounds + kWavesPerGroup - 1) / kWavesPerGroup;
  const int64_t total = groups * kSlices;
  const uint32_t grid = static_cast<uint32_t>(std::min<int64_t>(total, kMaxGrid / kSlices * kSlices));
  hipLaunchKernelGGL((spmv_sliced<V, W>), dim3(grid), dim3(kThreads), 0, stream,
                     static_cast<const S *>(p->s_data), p->s_col, p->s_seg, static_cast<const S *>(x),
                     static_cast<A *>(p->s_partial), p->bounds, p->bounds_nnz, p->n_bounds,
                     p->n_rows, p->nnz, p->slice_width, p->col_bits);
  const uint32_t mgrid = static_cast<uint32_t>(
      std::max<int64_t>(1, std::min<int64_t>((p->n_rows + kThreads - 1) / kThreads, kMaxGrid)));
  hipLaunchKernelGGL((slice_merge<V>), dim3(mgrid), dim3(kThreads), 0, stream,
                     static_cast<const A *>(p->s_partial), static_cast<S *>(y), p->n_rows);
}

template <class V>
void launch_v(const msx_csr_plan *p, const void *x, void *y, hipStream_t stream) {
  switch (p->block_nnz) {
  case 64: return launch_w<V, 64>(p, x, y, stream);
  case 128: return launch_w<V, 128>(p, x, y, stream);
  case 256: return launch_w<V, 256>(p, x, y, stream);
  case 512: return launch_w<V, 512>(p, x, y, stream);
  default: return launch_w<V, 1024>(p, x, y, stream);
  }
}

}  // namespace

msx_status build_slices(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                        hipStream_t stream) {
  switch (p->vtype) {
  case MSX_F32: return build_v<F32>(p, data, indices, indptr, stream);
  case MSX_F16: return build_v<F16>(p, data, indices, indptr, stream);
  case MSX_BF16: return build_v<BF16>(p, data, indices, indptr, stream);
  case MSX_C64: return build_v<C64>(p, data, indices, indptr, stream);
  }
  return fail(MSX_ETYPE, "msx_csr_plan_create_bound unsupported value dtype.");
}

msx_status launch_spmv_sliced(const msx_csr_plan *p, const void *x, void *y, hipStream_t stream) {
  switch (p->vtype) {
  case MSX_F32: launch_v<F32>(p, x, y, stream); break;
  case MSX_F16: launch_v<F16>(p, x, y, stream); break;
  case MSX_BF16: launch_v<BF16>(p, x, y, stream); break;
  case MSX_C64: launch_v<C64>(p, x, y, stream); break;
  }
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

}  // namespace msx
