// csr_slice.hip - XCD column slicing for SpMV with a scattered x gather.
//
// Why: MI355X has 8 XCDs, each with its own 4 MB L2.  When a matrix's
// columns are scattered over an x larger than that (the 4M-row random
// matrix: x is 16.8 MB), every XCD gathers from all of x, misses L2 on most
// gathers and pulls a whole 128-byte line from the Infinity Cache for each
// 4-byte value - 7.2 GB of fabric traffic for 0.59 GB of matrix.
//
// What: the plan partitions the columns into 8 slices of width Wc and, inside
// every 256-row super-block, stably reorders the block's values by slice
// (same position range of the block, so the copy is exactly nnz long).  Each
// value's index is packed as (row_in_block << col_bits) | (col - s*Wc).  The
// SpMV then runs slice s only on workgroups g with g % 8 == s - the hardware
// hands workgroup g to XCD g % 8 - so XCD s only ever gathers from
// x[s*Wc, (s+1)*Wc), about 2 MB for the 16.8 MB x, which stays in its L2.
// Each (super-block, slice) wave sums its rows in stored order into
// partial[s][row]; a merge kernel adds the 8 partials in slice order.  Long
// rows keep the unsliced path.
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
// Probe: count short blocks whose valid columns span more than n_cols / 4
// (counter[0]) and the values of all short blocks (counter[1]).
template <class I, int W>
__global__ void __launch_bounds__(kThreads)
    slice_probe(const I *__restrict__ indices, const int32_t *__restrict__ bounds,
                const int64_t *__restrict__ bounds_nnz, int64_t n_bounds, int64_t nnz,
                int64_t n_cols, unsigned long long *__restrict__ counter) {
  // Each wave walks blocks with a stride of the grid and keeps its counts in
  // registers; one atomic per counter and workgroup (an atomic per block
  // serialises hundreds of thousands of them on two addresses).
  __shared__ unsigned long long wg_count[2][kWavesPerGroup];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  unsigned long long scattered = 0, values = 0;
  for (int64_t b = static_cast<int64_t>(blockIdx.x) * kWavesPerGroup + wave; b < n_bounds;
       b += static_cast<int64_t>(gridDim.x) * kWavesPerGroup) {
    const BlockRange br = block_range<W>(bounds, bounds_nnz, b, nnz);
    if (!br.valid || br.p1 <= br.p0) continue;
    values += static_cast<unsigned long long>(br.p1 - br.p0);
    int64_t lo = INT64_MAX, hi = -1;
    // a block holds < 2W values: four unconditional loads per lane and step
    const auto rr = make_rsrc(indices + br.p0, static_cast<uint64_t>(br.p1 - br.p0) * sizeof(I));
    for (int64_t q = 0; q < br.p1 - br.p0; q += 4 * kWave) {
      I c[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        c[u] = buffer_index<I>(rr, static_cast<uint32_t>(q + lane + u * kWave) * sizeof(I));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = static_cast<int64_t>(c[u]);
        if (q + lane + u * kWave < br.p1 - br.p0 &&
            static_cast<uint64_t>(v) < static_cast<uint64_t>(n_cols)) {
          lo = v < lo ? v : lo;
          hi = v > hi ? v : hi;
        }
      }
    }
    for (int d = kWave / 2; d >= 1; d >>= 1) {
      const int64_t ol = __shfl_xor(lo, d, kWave);
      const int64_t oh = __shfl_xor(hi, d, kWave);
      lo = ol < lo ? ol : lo;
      hi = oh > hi ? oh : hi;
    }
    if (hi >= lo && hi - lo > n_cols / 4) ++scattered;
  }
  if (lane == 0) {
    wg_count[0][wave] = scattered;
    wg_count[1][wave] = values;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long a = 0, v = 0;
    for (int w = 0; w < kWavesPerGroup; ++w) {
      a += wg_count[0][w];
      v += wg_count[1][w];
    }
    if (a > 0) atomicAdd(counter, a);
    if (v > 0) atomicAdd(counter + 1, v);
  }
}

// ---------------------------------------------------------------------------
// Build.  Super-block k is the row window [256k, 256k + 256); its values keep
// their position range [P0, P1) = [indptr[256k], indptr[256k + 256]) and are
// stably reordered there by slice, seg[k][s] .. seg[k][s+1] relative to P0.
// Dropped: values of long rows (summed by spmv_long on the caller's arrays)
// and values whose column is outside [0, n_cols) (they add nothing).  One
// wave per super-block: a counting pass, then a stable scatter.  With
// `values_only` (a refresh after the values changed: same indices and
// indptr, so the same order) only s_data is written.
template <class V, class I>
__global__ void __launch_bounds__(kThreads)
    slice_build(const typename V::Storage *__restrict__ data, const I *__restrict__ indices,
                const I *__restrict__ indptr, int64_t n_rows, int64_t nnz, int64_t n_cols,
                int64_t long_len, int64_t slice_width, int col_bits,
                typename V::Storage *__restrict__ s_data, uint32_t *__restrict__ s_col,
                uint32_t *__restrict__ s_seg, bool values_only) {
  __shared__ int64_t lds_rp[kWavesPerGroup][kRows + 1];
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  int64_t *rp = lds_rp[wave];
  const int64_t k = static_cast<int64_t>(blockIdx.x) * kWavesPerGroup + wave;
  const int64_t n_super = (n_rows + kRows - 1) / kRows;
  if (k >= n_super) return;
  uint32_t *seg = s_seg + k * (kSlices + 1);
  const int64_t r0 = k * kRows;
  const int m = static_cast<int>(std::min<int64_t>(kRows, n_rows - r0));
  const int64_t P0 = clamp64(static_cast<int64_t>(indptr[r0]), 0, nnz);
  for (int i = lane; i <= m; i += kWave)
    rp[i] = clamp64(static_cast<int64_t>(indptr[r0 + i]), P0, nnz);
  wave_lds_sync();
  const int64_t P1 = rp[m];
  const int64_t n = P1 - P0;
  // classify element e: slice, or kSlices when dropped; also its row
  auto classify = [&](int64_t e, int64_t &col, int &row) -> int {
    int lo = 0, hi = m;  // rp[lo] <= P0 + e < rp[hi]
    const int64_t pos = P0 + e;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (rp[mid] <= pos) lo = mid;
      else hi = mid;
    }
    row = lo;
    if (rp[lo + 1] - rp[lo] > long_len) return kSlices;
    col = static_cast<int64_t>(indices[pos]);
    if (static_cast<uint64_t>(col) >= static_cast<uint64_t>(n_cols)) return kSlices;
    return static_cast<int>(col / slice_width);
  };
  int64_t count[kSlices];
#pragma unroll
  for (int s = 0; s < kSlices; ++s) count[s] = 0;
  for (int64_t c0 = 0; c0 < n; c0 += kWave) {
    const int64_t e = c0 + lane;
    int64_t col = 0;
    int row = 0;
    const int sl = e < n ? classify(e, col, row) : kSlices;
#pragma unroll
    for (int s = 0; s < kSlices; ++s) count[s] += __popcll(__ballot(sl == s));
  }
  int64_t start[kSlices + 1];
  start[0] = 0;
#pragma unroll
  for (int s = 0; s < kSlices; ++s) start[s + 1] = start[s] + count[s];
  if (lane <= kSlices && !values_only) {
    int64_t v = 0;
#pragma unroll
    for (int s = 0; s <= kSlices; ++s) v = lane == s ? start[s] : v;
    seg[lane] = static_cast<uint32_t>(v);
  }
  int64_t run[kSlices];
#pragma unroll
  for (int s = 0; s < kSlices; ++s) run[s] = start[s];
  const uint64_t lt = lanemask_lt(lane);
  for (int64_t c0 = 0; c0 < n; c0 += kWave) {
    const int64_t e = c0 + lane;
    int64_t col = 0;
    int row = 0;
    const int sl = e < n ? classify(e, col, row) : kSlices;
    int64_t dest = -1;
#pragma unroll
    for (int s = 0; s < kSlices; ++s) {
      const uint64_t mask = __ballot(sl == s);
      if (sl == s) dest = run[s] + __popcll(mask & lt);
      run[s] += __popcll(mask);
    }
    if (dest >= 0) {
      s_data[P0 + dest] = data[P0 + e];
      if (!values_only)
        s_col[P0 + dest] = (static_cast<uint32_t>(row) << col_bits) |
                           static_cast<uint32_t>(col - static_cast<int64_t>(sl) * slice_width);
    }
  }
}

// ---------------------------------------------------------------------------
// SpMV over one (super-block, slice) per wave; workgroup g serves slice g % 8,
// which the hardware runs on XCD g % 8.  The slice segment is consumed in
// chunks of kChunk values (all loads of a chunk issued before any use);
// within a chunk each row's run is summed in stored order by one lane and
// added to the row's running sum, so segments of any length fit LDS.
template <class V, int AUX>
__global__ void __launch_bounds__(kThreads)
    spmv_sliced(const typename V::Storage *__restrict__ s_data, const uint32_t *__restrict__ s_col,
                const uint32_t *__restrict__ s_seg, const typename V::Storage *__restrict__ x,
                typename V::Acc *__restrict__ partial, int64_t n_rows, int64_t nnz,
                const void *__restrict__ indptr_v, int index_bytes, int64_t slice_width,
                int col_bits, uint64_t x_bytes_total) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  constexpr int QPL = 4;
  constexpr int kChunk = 4 * QPL * kWave;  // values per chunk
  __shared__ A lds_prod[kWavesPerGroup][kChunk];
  __shared__ uint8_t lds_row[kWavesPerGroup][kChunk];
  __shared__ uint16_t lds_rs[kWavesPerGroup][kRows];
  __shared__ uint16_t lds_re[kWavesPerGroup][kRows];
  __shared__ A lds_acc[kWavesPerGroup][kRows];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  A *prod = lds_prod[wave];
  uint8_t *rowid = lds_row[wave];
  uint16_t *rs = lds_rs[wave];
  uint16_t *re = lds_re[wave];
  A *racc = lds_acc[wave];
  const uint32_t col_mask = (1u << col_bits) - 1u;
  const int s = static_cast<int>(blockIdx.x % kSlices);
  const S *xs = x + static_cast<int64_t>(s) * slice_width;
  A *part = partial + static_cast<int64_t>(s) * n_rows;
  // This slice of x through a descriptor (x_bytes_total == 0: x is not
  // dword-aligned or too large for one, and the gathers are plain loads).
  const uint64_t s_off = static_cast<uint64_t>(s) * slice_width * sizeof(S);
  const uint64_t s_len = x_bytes_total > s_off
      ? std::min<uint64_t>(slice_width * sizeof(S), x_bytes_total - s_off) : 0;
  const uint32_t xs_bytes = static_cast<uint32_t>((s_len + 3) & ~uint64_t{3});
  const auto rxs = make_rsrc(xs, xs_bytes);
  const int64_t n_super = (n_rows + kRows - 1) / kRows;

  for (int64_t g = blockIdx.x / kSlices; g * kWavesPerGroup < n_super; g += gridDim.x / kSlices) {
    const int64_t k = g * kWavesPerGroup + wave;
    if (k >= n_super) break;
    const int64_t r0 = k * kRows;
    const int m = static_cast<int>(std::min<int64_t>(kRows, n_rows - r0));
    const int64_t P0 = clamp64(index_bytes == 8 ? static_cast<const int64_t *>(indptr_v)[r0]
                                                : static_cast<const int32_t *>(indptr_v)[r0],
                               0, nnz);
    const uint32_t *seg = s_seg + k * (kSlices + 1);
    const int64_t lo = std::min<int64_t>(P0 + seg[s], nnz);
    const int64_t hi = std::min<int64_t>(P0 + seg[s + 1], nnz);
    // Invariant at each chunk start: rs/re are zero for every row.
    for (int i = lane; i < kRows; i += kWave) {
      racc[i] = vzero<A>();
      rs[i] = 0;
      re[i] = 0;
    }
    wave_lds_sync();
    // Chunks start on quad boundaries, so a chunk is at most QPL quads per
    // lane; the descriptors end at the chunk's last value, so every load is
    // unconditional (lanes past it read zero) and a wave issues all of its
    // loads before it waits on any.
    for (int64_t a0 = lo & ~int64_t{3}; a0 < hi; a0 += kChunk) {
      const int64_t c_lo = std::max(lo, a0);
      const int64_t c_hi = std::min<int64_t>(a0 + kChunk, hi);
      const int cnt = static_cast<int>(c_hi - c_lo);
      const auto rc = make_rsrc(s_col + a0, static_cast<uint64_t>(c_hi - a0) * sizeof(uint32_t));
      const auto rd = make_rsrc(s_data + a0, static_cast<uint64_t>(c_hi - a0) * sizeof(S));
      Quad<uint32_t> cq[QPL];
      Quad<S> dq[QPL];
#pragma unroll
      for (int j = 0; j < QPL; ++j) {
        const uint32_t q = static_cast<uint32_t>(lane + j * kWave);
        cq[j] = load_quad<uint32_t, AUX>(rc, q * 16u);
        dq[j] = load_quad<S, AUX>(rd, q * 4u * sizeof(S));
      }
      A xv[QPL][4];
      if (x_bytes_total != 0) {
        GatherRaw<S> raw[QPL][4];
#pragma unroll
        for (int j = 0; j < QPL; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t pos = a0 + 4 * (lane + j * kWave) + e;
            raw[j][e] = gather_raw<S>(rxs, xs_bytes, cq[j].v[e] & col_mask, pos >= c_lo && pos < c_hi);
          }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < QPL; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) xv[j][e] = gather_widen<V>(raw[j][e], cq[j].v[e] & col_mask);
      } else {
#pragma unroll
        for (int j = 0; j < QPL; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int64_t pos = a0 + 4 * (lane + j * kWave) + e;
            xv[j][e] = vzero<A>();
            if (pos >= c_lo && pos < c_hi) xv[j][e] = V::widen(xs[cq[j].v[e] & col_mask]);
          }
      }
      // rows of this chunk: rowid[0] .. rowid[cnt-1] (ascending)
#pragma unroll
      for (int j = 0; j < QPL; ++j) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int64_t pos = a0 + 4 * (lane + j * kWave) + e;
          if (pos >= c_lo && pos < c_hi) {
            const int t = static_cast<int>(pos - c_lo);
            prod[t] = vmul_acc<V>(xv[j][e], dq[j].v[e]);
            rowid[t] = static_cast<uint8_t>((cq[j].v[e] >> col_bits) & (kRows - 1));
          }
        }
      }
      wave_lds_sync();
      for (int t = lane; t < cnt; t += kWave) {
        const int r = rowid[t];
        if (t == 0 || rowid[t - 1] != r) rs[r] = static_cast<uint16_t>(t);
        if (t == cnt - 1 || rowid[t + 1] != r) re[r] = static_cast<uint16_t>(t + 1);
      }
      wave_lds_sync();
      const int first = rowid[0];
      const int last = rowid[cnt - 1];
      for (int r = first + lane; r <= last; r += kWave) {
        const int t0 = rs[r], t1 = re[r];
        if (t1 > t0) {
          A acc = vzero<A>();
          for (int t = t0; t < t1; ++t) acc = vadd(acc, prod[t]);
          racc[r] = vadd(racc[r], acc);
        }
        rs[r] = 0;  // restore the invariant for the next chunk
        re[r] = 0;
      }
      wave_lds_sync();
    }
    for (int i = lane; i < m; i += kWave) part[r0 + i] = racc[i];
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

template <class I, int W>
msx_status probe_typed(const msx_csr_plan *p, const void *indices, hipStream_t stream,
                       bool *scattered, int64_t *short_values) {
  const int64_t groups = std::min<int64_t>((p->n_bounds + kWavesPerGroup - 1) / kWavesPerGroup, 2048);
  unsigned long long *counter = nullptr;
  MSX_HIP_TRY(hipMallocAsync(reinterpret_cast<void **>(&counter), 2 * sizeof(*counter), stream));
  MSX_HIP_TRY(hipMemsetAsync(counter, 0, 2 * sizeof(*counter), stream));
  hipLaunchKernelGGL((slice_probe<I, W>), dim3(static_cast<uint32_t>(groups)), dim3(kThreads), 0,
                     stream, static_cast<const I *>(indices), p->bounds, p->bounds_nnz,
                     p->n_bounds, p->nnz, p->n_cols, counter);
  unsigned long long count[2] = {0, 0};
  hipError_t e = hipGetLastError();
  if (e == hipSuccess)
    e = hipMemcpyAsync(count, counter, sizeof(count), hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  (void)hipFreeAsync(counter, stream);
  if (e != hipSuccess) return hip_fail(e, "slice probe");
  *scattered = 2 * static_cast<int64_t>(count[0]) > p->n_blocks;  // else mostly local
  *short_values = static_cast<int64_t>(count[1]);
  return MSX_OK;
}

template <class I>
msx_status probe_w(const msx_csr_plan *p, const void *indices, hipStream_t stream,
                   bool *scattered, int64_t *short_values) {
  switch (p->block_nnz) {
  case 64: return probe_typed<I, 64>(p, indices, stream, scattered, short_values);
  case 128: return probe_typed<I, 128>(p, indices, stream, scattered, short_values);
  case 256: return probe_typed<I, 256>(p, indices, stream, scattered, short_values);
  case 512: return probe_typed<I, 512>(p, indices, stream, scattered, short_values);
  default: return probe_typed<I, 1024>(p, indices, stream, scattered, short_values);
  }
}

template <class V, class I>
msx_status build_typed(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                       hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int64_t width = ((p->n_cols + kSlices - 1) / kSlices + 31) / 32 * 32;
  const int col_bits = std::max(1, bits_for(width));
  const int64_t n_super = (p->n_rows + kRows - 1) / kRows;
  if (col_bits > 24 || n_super == 0 || p->nnz >= (int64_t{1} << 32)) return MSX_OK;
  const size_t b_data = ((static_cast<size_t>(p->nnz) * sizeof(S) + 255) / 256) * 256;
  const size_t b_col = ((static_cast<size_t>(p->nnz) * 4 + 255) / 256) * 256;
  const size_t b_seg = ((static_cast<size_t>(n_super) * (kSlices + 1) * 4 + 255) / 256) * 256;
  const size_t b_part = static_cast<size_t>(kSlices) * p->n_rows * sizeof(A);
  char *base = nullptr;
  if (hipMalloc(&base, b_data + b_col + b_seg + b_part) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MSX_ENOMEM, "msx_csr_plan_create_bound: device allocation of the sliced copy failed.");
  }
  p->s_base = base;
  p->s_data = base;
  p->s_col = reinterpret_cast<uint32_t *>(base + b_data);
  p->s_seg = reinterpret_cast<uint32_t *>(base + b_data + b_col);
  p->s_partial = base + b_data + b_col + b_seg;
  p->s_bytes = b_data + b_col + b_seg + b_part;
  p->slice_width = width;
  p->col_bits = col_bits;
  const int64_t bgroups = (n_super + kWavesPerGroup - 1) / kWavesPerGroup;
  hipLaunchKernelGGL((slice_build<V, I>), dim3(static_cast<uint32_t>(bgroups)), dim3(kThreads), 0,
                     stream, static_cast<const S *>(data), static_cast<const I *>(indices),
                     static_cast<const I *>(indptr), p->n_rows, p->nnz, p->n_cols, p->block_nnz,
                     width, col_bits, static_cast<S *>(p->s_data), p->s_col, p->s_seg, false);
  MSX_HIP_TRY(hipGetLastError());
  MSX_HIP_TRY(hipStreamSynchronize(stream));
  p->n_slices = kSlices;
  p->s_indptr = indptr;
  return MSX_OK;
}

template <class V, class I>
msx_status refresh_typed(msx_csr_plan *p, const void *data, hipStream_t stream) {
  using S = typename V::Storage;
  const int64_t n_super = (p->n_rows + kRows - 1) / kRows;
  const int64_t bgroups = (n_super + kWavesPerGroup - 1) / kWavesPerGroup;
  hipLaunchKernelGGL((slice_build<V, I>), dim3(static_cast<uint32_t>(bgroups)), dim3(kThreads), 0,
                     stream, static_cast<const S *>(data), static_cast<const I *>(p->bound_indices),
                     static_cast<const I *>(p->s_indptr), p->n_rows, p->nnz, p->n_cols,
                     p->block_nnz, p->slice_width, p->col_bits, static_cast<S *>(p->s_data),
                     p->s_col, p->s_seg, true);
  MSX_HIP_TRY(hipGetLastError());
  return MSX_OK;
}

template <class V>
msx_status refresh_v(msx_csr_plan *p, const void *data, hipStream_t stream) {
  return p->itype == MSX_I32 ? refresh_typed<V, int32_t>(p, data, stream)
                             : refresh_typed<V, int64_t>(p, data, stream);
}

template <class V>
msx_status build_v(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                   hipStream_t stream) {
  return p->itype == MSX_I32 ? build_typed<V, int32_t>(p, data, indices, indptr, stream)
                             : build_typed<V, int64_t>(p, data, indices, indptr, stream);
}

template <class V>
void launch_v(const msx_csr_plan *p, const void *x, void *y, hipStream_t stream) {
  using S = typename V::Storage;
  using A = typename V::Acc;
  const int64_t n_super = (p->n_rows + kRows - 1) / kRows;
  const int64_t total = (n_super + kWavesPerGroup - 1) / kWavesPerGroup * kSlices;
  const uint32_t grid = static_cast<uint32_t>(std::min<int64_t>(total, kMaxGrid / kSlices * kSlices));
  // Copies that cannot stay in the Infinity Cache are streamed non-temporally.
  const bool stream_nt =
      static_cast<uint64_t>(p->nnz) * (sizeof(S) + sizeof(uint32_t)) > kStreamNtBytes;
  auto kernel = stream_nt ? spmv_sliced<V, kCacheStream> : spmv_sliced<V, kCacheDefault>;
  // Each slice's descriptor must reach its last byte: x below 4 GB, dword-aligned.
  const uint64_t xb = static_cast<uint64_t>(p->n_cols) * sizeof(S);
  const uint64_t x_bytes =
      xb <= kGatherMaxBytes && reinterpret_cast<uintptr_t>(x) % 4 == 0 ? xb : 0;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(kThreads), 0, stream,
                     static_cast<const S *>(p->s_data), p->s_col, p->s_seg, static_cast<const S *>(x),
                     static_cast<A *>(p->s_partial), p->n_rows, p->nnz, p->s_indptr,
                     p->itype == MSX_I64 ? 8 : 4, p->slice_width, p->col_bits, x_bytes);
  const uint32_t mgrid = static_cast<uint32_t>(
      std::max<int64_t>(1, std::min<int64_t>((p->n_rows + kThreads - 1) / kThreads, kMaxGrid)));
  hipLaunchKernelGGL((slice_merge<V>), dim3(mgrid), dim3(kThreads), 0, stream,
                     static_cast<const A *>(p->s_partial), static_cast<S *>(y), p->n_rows);
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

msx_status refresh_slices(msx_csr_plan *p, const void *data, hipStream_t stream) {
  if (p->n_slices == 0) return MSX_OK;
  switch (p->vtype) {
  case MSX_F32: return refresh_v<F32>(p, data, stream);
  case MSX_F16: return refresh_v<F16>(p, data, stream);
  case MSX_BF16: return refresh_v<BF16>(p, data, stream);
  case MSX_C64: return refresh_v<C64>(p, data, stream);
  }
  return fail(MSX_ETYPE, "msx_csr_plan_refresh unsupported value dtype.");
}

msx_status probe_scattered(const msx_csr_plan *p, const void *indices, hipStream_t stream,
                           bool *scattered, int64_t *short_values) {
  *scattered = false;
  *short_values = 0;
  const int64_t x_bytes = p->n_cols * static_cast<int64_t>(value_bytes(p->vtype));
  if (x_bytes < (int64_t{8} << 20) || p->n_bounds == 0 || p->n_blocks == 0) return MSX_OK;
  return p->itype == MSX_I32 ? probe_w<int32_t>(p, indices, stream, scattered, short_values)
                             : probe_w<int64_t>(p, indices, stream, scattered, short_values);
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
