// csr_plan.hip - row-block plans built on the device from `indptr`.
//
// A plan sorts the rows of a CSR matrix into two kinds of work:
//
//   short blocks - runs of consecutive rows processed by one wavefront.  Row r
//                  (not long) starts a new block when r == 0, r % R == 0, row
//                  r-1 is long, or indptr[r] / W != indptr[r-1] / W.  All row
//                  starts of a block then fall in one W-wide window of the
//                  nnz range and every row holds <= W values, so a block holds
//                  fewer than 2W values and at most R rows.
//   long rows    - rows with more than W values, cut into ceil(len / C)
//                  chunks; each chunk is summed by one workgroup and the chunk
//                  sums of a row are added in chunk order.
//
// Storage: `bounds` lists, in row order, every row that starts a short block
// or is long (long rows flagged in bit 31), then the sentinel n_rows; a short
// block runs from its entry to the next entry, so it never contains a long
// row.  `bounds_nnz` holds indptr at each entry (int64), which saves the
// kernels one dependent load.  Long rows also get a chunk list.
//
// This replaces the reference's single per-launch choice between a
// one-thread-per-row and a 128-lane-per-row kernel from the matrix average
// `nnz >= 32 * n_rows` (reference: src/sparse/csr_matvec/csr_matvec.cpp:40-41,
// 291-296), which runs a 200,000-value row of a power-law matrix on a single
// thread.
//
// Construction is three kernels: count flags per 4096-row tile, scan the tile
// counts in one workgroup, scatter row ids to their ranks.  The only host
// synchronisation reads the three totals to size the arrays.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "msx_device.h"
#include "msx_internal.h"

namespace msx {
namespace {

constexpr int kPlanThreads = 256;
constexpr int kRowsPerThread = 16;
constexpr int64_t kTileRows = static_cast<int64_t>(kPlanThreads) * kRowsPerThread;
constexpr uint32_t kLongFlag = 0x80000000u;

struct Counts {
  int64_t bounds;  // rows that start a short block or are long
  int64_t longs;
  int64_t chunks;
};

struct RowClass {
  bool start;
  bool is_long;
  int64_t chunks;
};

template <class I>
__device__ inline RowClass classify(const I *__restrict__ indptr, int64_t r, int64_t W, int64_t R,
                                    int64_t C) {
  const int64_t b = static_cast<int64_t>(indptr[r]);
  const int64_t e = static_cast<int64_t>(indptr[r + 1]);
  const int64_t len = e - b;
  RowClass c;
  c.is_long = len > W;
  c.chunks = c.is_long ? (len + C - 1) / C : 0;
  if (c.is_long) {
    c.start = false;
  } else if (r == 0 || (r % R) == 0) {
    c.start = true;
  } else {
    const int64_t pb = static_cast<int64_t>(indptr[r - 1]);
    const bool prev_long = (b - pb) > W;
    // floor division so malformed (negative) offsets still classify
    const int64_t wb = b >= 0 ? b / W : -((-b + W - 1) / W);
    const int64_t wp = pb >= 0 ? pb / W : -((-pb + W - 1) / W);
    c.start = prev_long || wb != wp;
  }
  return c;
}

// Inclusive scan of one int64 per thread across a 256-thread workgroup.
__device__ inline int64_t block_inclusive_scan(int64_t v, int64_t *lds_waves) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int64_t u = __shfl_up(v, d, kWave);
    if (lane >= d) v += u;
  }
  if (lane == kWave - 1) lds_waves[wave] = v;
  __syncthreads();
  int64_t off = 0;
  for (int w = 0; w < wave; ++w) off += lds_waves[w];
  __syncthreads();
  return v + off;
}

template <class I>
__global__ void __launch_bounds__(kPlanThreads)
    plan_count(const I *__restrict__ indptr, int64_t n, int64_t W, int64_t R, int64_t C,
               Counts *__restrict__ tile_counts) {
  __shared__ int64_t lds[3][kPlanThreads / kWave];
  const int64_t tile = blockIdx.x;
  const int64_t r0 = tile * kTileRows + static_cast<int64_t>(threadIdx.x) * kRowsPerThread;
  Counts c{0, 0, 0};
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int64_t r = r0 + i;
    if (r >= n) break;
    const RowClass rc = classify(indptr, r, W, R, C);
    c.bounds += rc.start || rc.is_long;
    c.longs += rc.is_long;
    c.chunks += rc.chunks;
  }
  const int64_t s = block_inclusive_scan(c.bounds, lds[0]);
  const int64_t l = block_inclusive_scan(c.longs, lds[1]);
  const int64_t k = block_inclusive_scan(c.chunks, lds[2]);
  if (threadIdx.x == kPlanThreads - 1) tile_counts[tile] = Counts{s, l, k};
}

// Exclusive scan of the tile counts in place; totals land in `totals`.
__global__ void __launch_bounds__(kPlanThreads)
    plan_scan(Counts *__restrict__ tile_counts, int64_t n_tiles, Counts *__restrict__ totals) {
  __shared__ int64_t lds[3][kPlanThreads / kWave];
  Counts carry{0, 0, 0};
  for (int64_t base = 0; base < n_tiles; base += kPlanThreads) {
    const int64_t t = base + threadIdx.x;
    const Counts v = t < n_tiles ? tile_counts[t] : Counts{0, 0, 0};
    const int64_t s = block_inclusive_scan(v.bounds, lds[0]);
    const int64_t l = block_inclusive_scan(v.longs, lds[1]);
    const int64_t k = block_inclusive_scan(v.chunks, lds[2]);
    if (t < n_tiles)
      tile_counts[t] = Counts{carry.bounds + s - v.bounds, carry.longs + l - v.longs,
                              carry.chunks + k - v.chunks};
    // the last thread holds the batch total; broadcast through LDS
    __shared__ Counts batch_total;
    if (threadIdx.x == kPlanThreads - 1) batch_total = Counts{s, l, k};
    __syncthreads();
    carry.bounds += batch_total.bounds;
    carry.longs += batch_total.longs;
    carry.chunks += batch_total.chunks;
    __syncthreads();
  }
  if (threadIdx.x == 0) *totals = carry;
}

template <class I>
__global__ void __launch_bounds__(kPlanThreads)
    plan_scatter(const I *__restrict__ indptr, int64_t n, int64_t W, int64_t R, int64_t C,
                 const Counts *__restrict__ tile_offsets, int64_t n_bounds, int64_t n_long,
                 int64_t n_chunks, int32_t *__restrict__ bounds, int64_t *__restrict__ bounds_nnz,
                 int32_t *__restrict__ long_rows, int32_t *__restrict__ long_chunk_begin,
                 int32_t *__restrict__ chunk_row) {
  __shared__ int64_t lds[3][kPlanThreads / kWave];
  const int64_t tile = blockIdx.x;
  const int64_t r0 = tile * kTileRows + static_cast<int64_t>(threadIdx.x) * kRowsPerThread;
  Counts c{0, 0, 0};
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int64_t r = r0 + i;
    if (r >= n) break;
    const RowClass rc = classify(indptr, r, W, R, C);
    c.bounds += rc.start || rc.is_long;
    c.longs += rc.is_long;
    c.chunks += rc.chunks;
  }
  const Counts base = tile_offsets[tile];
  int64_t s = base.bounds + block_inclusive_scan(c.bounds, lds[0]) - c.bounds;
  int64_t l = base.longs + block_inclusive_scan(c.longs, lds[1]) - c.longs;
  int64_t k = base.chunks + block_inclusive_scan(c.chunks, lds[2]) - c.chunks;
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int64_t r = r0 + i;
    if (r >= n) break;
    const RowClass rc = classify(indptr, r, W, R, C);
    if (rc.start || rc.is_long) {
      bounds[s] = static_cast<int32_t>(static_cast<uint32_t>(r) | (rc.is_long ? kLongFlag : 0u));
      bounds_nnz[s] = static_cast<int64_t>(indptr[r]);
      ++s;
    }
    if (rc.is_long) {
      long_rows[l] = static_cast<int32_t>(r);
      long_chunk_begin[l] = static_cast<int32_t>(k);
      for (int64_t j = 0; j < rc.chunks; ++j) chunk_row[k + j] = static_cast<int32_t>(l);
      k += rc.chunks;
      ++l;
    }
  }
  if (tile == 0 && threadIdx.x == 0) {
    bounds[n_bounds] = static_cast<int32_t>(n);
    bounds_nnz[n_bounds] = static_cast<int64_t>(indptr[n]);
    long_chunk_begin[n_long] = static_cast<int32_t>(n_chunks);
  }
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

template <class I>
msx_status build_plan(msx_csr_plan *p, const I *indptr, hipStream_t stream) {
  const int64_t n = p->n_rows;
  const int64_t n_tiles = (n + kTileRows - 1) / kTileRows;
  Counts *tmp = nullptr;
  if (n_tiles > 0) {
    MSX_HIP_TRY(hipMalloc(&tmp, sizeof(Counts) * (n_tiles + 1)));
    hipLaunchKernelGGL(plan_count<I>, dim3(static_cast<uint32_t>(n_tiles)), dim3(kPlanThreads), 0,
                       stream, indptr, n, p->block_nnz, p->block_rows, p->chunk_nnz, tmp);
    hipLaunchKernelGGL(plan_scan, dim3(1), dim3(kPlanThreads), 0, stream, tmp, n_tiles,
                       tmp + n_tiles);
    Counts totals{0, 0, 0};
    hipError_t e = hipMemcpyAsync(&totals, tmp + n_tiles, sizeof(Counts), hipMemcpyDeviceToHost,
                                  stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) {
      (void)hipFree(tmp);
      return hip_fail(e, "plan count");
    }
    p->n_bounds = totals.bounds;
    p->n_long = totals.longs;
    p->n_chunks = totals.chunks;
    p->n_blocks = p->n_bounds - p->n_long;
  } else {
    p->n_bounds = p->n_blocks = p->n_long = p->n_chunks = 0;
  }
  if (p->n_chunks >= (int64_t{1} << 31) || p->n_bounds >= (int64_t{1} << 31)) {
    if (tmp) (void)hipFree(tmp);
    return fail(MSX_EINVAL, "msx_csr_plan_create: matrix too large for an int32 plan.");
  }
  // One allocation: int32 bounds, int64 bounds_nnz, three int32 long-row
  // arrays, then 8-byte chunk partial sums.
  const size_t a0 = align_up(sizeof(int32_t) * (p->n_bounds + 1), 256);
  const size_t a1 = align_up(sizeof(int64_t) * (p->n_bounds + 1), 256);
  const size_t a2 = align_up(sizeof(int32_t) * std::max<int64_t>(p->n_long, 1), 256);
  const size_t a3 = align_up(sizeof(int32_t) * (p->n_long + 1), 256);
  const size_t a4 = align_up(sizeof(int32_t) * std::max<int64_t>(p->n_chunks, 1), 256);
  const size_t a5 = align_up(8 * std::max<int64_t>(p->n_chunks, 1), 256);
  p->bytes = a0 + a1 + a2 + a3 + a4 + a5;
  char *base = nullptr;
  hipError_t e = hipMalloc(&base, p->bytes);
  if (e != hipSuccess) {
    if (tmp) (void)hipFree(tmp);
    (void)hipGetLastError();
    return fail(MSX_ENOMEM, "msx_csr_plan_create: device allocation of the plan failed.");
  }
  p->base = base;
  p->bounds = reinterpret_cast<int32_t *>(base);
  p->bounds_nnz = reinterpret_cast<int64_t *>(base + a0);
  p->long_rows = reinterpret_cast<int32_t *>(base + a0 + a1);
  p->long_chunk_begin = reinterpret_cast<int32_t *>(base + a0 + a1 + a2);
  p->chunk_row = reinterpret_cast<int32_t *>(base + a0 + a1 + a2 + a3);
  p->partials = base + a0 + a1 + a2 + a3 + a4;
  if (n_tiles > 0) {
    hipLaunchKernelGGL(plan_scatter<I>, dim3(static_cast<uint32_t>(n_tiles)), dim3(kPlanThreads), 0,
                       stream, indptr, n, p->block_nnz, p->block_rows, p->chunk_nnz, tmp,
                       p->n_bounds, p->n_long, p->n_chunks, p->bounds, p->bounds_nnz,
                       p->long_rows, p->long_chunk_begin, p->chunk_row);
    e = hipGetLastError();
    // tmp is read by the scatter kernel: release only after it has run.
    hipError_t e2 = hipStreamSynchronize(stream);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(e, "plan_scatter launch");
    if (e2 != hipSuccess) return hip_fail(e2, "plan_scatter");
  } else {
    // n == 0: sentinels only (row 0, nnz offset 0, chunk 0)
    const int64_t zeros[2] = {0, 0};
    MSX_HIP_TRY(hipMemcpy(p->bounds, zeros, sizeof(int32_t), hipMemcpyHostToDevice));
    MSX_HIP_TRY(hipMemcpy(p->bounds_nnz, zeros, sizeof(int64_t), hipMemcpyHostToDevice));
    MSX_HIP_TRY(hipMemcpy(p->long_chunk_begin, zeros, sizeof(int32_t), hipMemcpyHostToDevice));
  }
  return MSX_OK;
}

}  // namespace
}  // namespace msx

using namespace msx;

namespace {

msx_status create_plan(msx_itype it, int64_t n_rows, int64_t nnz, const void *indptr,
                       int64_t block_nnz, void *stream, msx_csr_plan **out) {
  if (out == nullptr) return fail(MSX_EINVAL, "msx_csr_plan_create: out is NULL.");
  *out = nullptr;
  if (!valid_itype(it))
    return fail(MSX_ETYPE, "msx_csr_plan_create requires int32 or int64 indices.");
  if (n_rows < 0 || nnz < 0)
    return fail(MSX_EINVAL, "msx_csr_plan_create shape dimensions must be non-negative.");
  if (n_rows >= (int64_t{1} << 31) - 1)
    return fail(MSX_EINVAL, "msx_csr_plan_create: n_rows must be below 2^31 - 1.");
  if (indptr == nullptr) return fail(MSX_EINVAL, "msx_csr_plan_create: indptr is NULL.");
  if (block_nnz == 0)
    block_nnz = nnz >= kWideBlockMean * n_rows && n_rows > 0 ? kWideBlockNnz : kDefaultBlockNnz;
  if (block_nnz < 64 || block_nnz > 1024 || (block_nnz & (block_nnz - 1)) != 0)
    return fail(MSX_EINVAL, "msx_csr_plan_create: block_nnz must be a power of two in [64, 1024].");
  auto *p = new (std::nothrow) msx_csr_plan{};
  if (p == nullptr) return fail(MSX_ENOMEM, "msx_csr_plan_create: host allocation failed.");
  p->itype = it;
  p->n_rows = n_rows;
  p->nnz = nnz;
  p->block_nnz = block_nnz;
  p->block_rows = kBlockRows;
  p->chunk_nnz = kChunkNnz;
  p->slice_mode = MSX_SLICE_OFF;
  p->indptr = indptr;
  hipError_t e = hipGetDevice(&p->device);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "hipGetDevice");
  }
  auto s = static_cast<hipStream_t>(stream);
  msx_status st = it == MSX_I32 ? build_plan(p, static_cast<const int32_t *>(indptr), s)
                                : build_plan(p, static_cast<const int64_t *>(indptr), s);
  if (st != MSX_OK) {
    if (p->base) (void)hipFree(p->base);
    delete p;
    return st;
  }
  *out = p;
  return MSX_OK;
}

void release(msx_csr_plan *p) {
  if (p->base) (void)hipFree(p->base);
  if (p->s_base) (void)hipFree(p->s_base);
  if (p->pn_base) (void)hipFree(p->pn_base);
  if (p->pn_meta) (void)hipFree(p->pn_meta);
  if (p->pn_vmeta) (void)hipFree(p->pn_vmeta);
  if (p->win) (void)hipFree(p->win);
  if (p->ls_base) (void)hipFree(p->ls_base);
  delete p;
}

}  // namespace

extern "C" msx_status msx_csr_plan_create(msx_itype it, int64_t n_rows, int64_t nnz,
                                          const void *indptr, int64_t block_nnz, void *stream,
                                          msx_csr_plan **out) {
  clear_error();
  return create_plan(it, n_rows, nnz, indptr, block_nnz, stream, out);
}

extern "C" msx_status msx_csr_plan_create_bound(msx_vtype vt, msx_itype it, int64_t n_rows,
                                                int64_t n_cols, int64_t nnz, const void *data,
                                                const void *indices, const void *indptr,
                                                const msx_plan_options *opts, void *stream,
                                                msx_csr_plan **out) {
  clear_error();
  if (!valid_vtype(vt))
    return fail(MSX_ETYPE, "msx_csr_plan_create_bound unsupported value dtype.");
  if (n_cols < 0 || n_cols > 2147483647)
    return fail(MSX_EINVAL, "msx_csr_plan_create_bound: n_cols must be in [0, 2^31).");
  if (nnz > 0 && (data == nullptr || indices == nullptr))
    return fail(MSX_EINVAL, "msx_csr_plan_create_bound: data and indices must be non-NULL.");
  const msx_plan_options defaults{0, MSX_SLICE_AUTO, 0};
  if (opts == nullptr) opts = &defaults;
  if (opts->slice_mode < MSX_SLICE_AUTO || opts->slice_mode > MSX_SLICE_PANELS || opts->reserved != 0)
    return fail(MSX_EINVAL, "msx_csr_plan_create_bound: invalid options.");
  // complex64 keeps the narrow default: a 512-value block holds twice the
  // registers for its 8-byte values, which halves occupancy (banded matrix,
  // 42.6 values per row: 171 us at W = 256, 197 us at 512).
  const int64_t w = opts->block_nnz == 0 && vt == MSX_C64 ? kDefaultBlockNnz : opts->block_nnz;
  msx_csr_plan *p = nullptr;
  msx_status st = create_plan(it, n_rows, nnz, indptr, w, stream, &p);
  if (st != MSX_OK) return st;
  p->vtype = vt;
  p->n_cols = n_cols;
  p->slice_mode = opts->slice_mode;
  p->bound = true;
  p->bound_data = data;
  p->bound_indices = indices;
  auto s = static_cast<hipStream_t>(stream);
  int mode = opts->slice_mode;
  if (mode == MSX_SLICE_AUTO) {
    // Scattered short rows over a large x: LDS panels (long rows ride in
    // them as 64-value virtual rows) when the matrix holds enough values to
    // give every compute unit a pass-1 chunk - the 4M-row random matrix:
    // 221 us against 930 us in row blocks; the power-law matrix (x 8.4 MB,
    // about half of its values in long rows): 92 us against 157 us; XCD
    // slices when x is 16 MB or more and panels are not possible.
    bool scattered = false;
    int64_t short_values = 0;
    st = probe_scattered(p, indices, s, &scattered, &short_values);
    const int64_t x_bytes = n_cols * static_cast<int64_t>(value_bytes(vt));
    mode = MSX_SLICE_OFF;
    if (scattered && panels_eligible(p) && p->nnz >= panels_min_values(p->device))
      mode = MSX_SLICE_PANELS;
    else if (scattered && x_bytes >= (int64_t{16} << 20))
      mode = MSX_SLICE_ON;
  }
  if (st == MSX_OK && mode == MSX_SLICE_PANELS && p->n_blocks > 0) {
    if (!panels_eligible(p))
      st = fail(MSX_EINVAL,
                "msx_csr_plan_create_bound: panels need nnz < 2^31, n_cols >= 1 and at most "
                "2048 panels of x.");
    else
      st = build_panels(p, data, indices, indptr, s);
  } else if (st == MSX_OK && mode == MSX_SLICE_ON && p->n_blocks > 0) {
    st = build_slices(p, data, indices, indptr, s);
  }
  if (st == MSX_OK) st = build_windows(p, indices, indptr, s);
  // long rows in a panel layout need no sliced pieces
  if (st == MSX_OK && p->pn_vstart == nullptr) st = build_long_slices(p, indices, indptr, s);
  if (st != MSX_OK) {
    release(p);
    return st;
  }
  *out = p;
  return MSX_OK;
}

extern "C" msx_status msx_csr_plan_refresh(msx_csr_plan *plan, const void *data, void *stream) {
  clear_error();
  if (plan == nullptr) return fail(MSX_EINVAL, "msx_csr_plan_refresh: plan is NULL.");
  if (!plan->bound) return MSX_OK;  // row blocks hold no values
  if (plan->nnz > 0 && data == nullptr)
    return fail(MSX_EINVAL, "msx_csr_plan_refresh: data is NULL.");
  int dev = -1;
  MSX_HIP_TRY(hipGetDevice(&dev));
  if (dev != plan->device)
    return fail(MSX_EINVAL, "msx_csr_plan_refresh: plan lives on another device.");
  auto s = static_cast<hipStream_t>(stream);
  msx_status st = refresh_slices(plan, data, s);
  if (st == MSX_OK && plan->n_panels > 0) st = refresh_panels(plan, data, s);
  if (st == MSX_OK) plan->bound_data = data;
  return st;
}

extern "C" msx_status msx_csr_plan_destroy(msx_csr_plan *plan) {
  clear_error();
  if (plan == nullptr) return MSX_OK;
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(plan->device);
  hipError_t e = hipDeviceSynchronize();
  release(plan);
  (void)hipSetDevice(prev);
  if (e != hipSuccess) return hip_fail(e, "msx_csr_plan_destroy");
  return MSX_OK;
}

extern "C" msx_status msx_csr_plan_info(const msx_csr_plan *plan, msx_plan_info *info) {
  clear_error();
  if (plan == nullptr || info == nullptr)
    return fail(MSX_EINVAL, "msx_csr_plan_info: plan and info must be non-NULL.");
  info->n_rows = plan->n_rows;
  info->nnz = plan->nnz;
  info->block_nnz = plan->block_nnz;
  info->block_rows = plan->block_rows;
  info->chunk_nnz = plan->chunk_nnz;
  info->n_blocks = plan->n_blocks;
  info->n_bounds = plan->n_bounds;
  info->n_long_rows = plan->n_long;
  info->n_chunks = plan->n_chunks;
  info->device = plan->device;
  info->plan_bytes =
      static_cast<int64_t>(plan->bytes + plan->s_bytes + plan->pn_bytes + plan->win_bytes +
                           plan->ls_bytes);
  info->n_slices = plan->n_slices;
  info->slice_width = plan->slice_width;
  info->slice_bytes = static_cast<int64_t>(plan->s_bytes);
  info->n_panels = plan->n_panels;
  info->panel_width = plan->panel_width;
  info->n_tiles = plan->n_tiles;
  info->panel_values = plan->pn_values;
  info->panel_bytes = static_cast<int64_t>(plan->pn_bytes);
  info->window_rows = plan->win_rows_max;
  return MSX_OK;
}

namespace {
// Device int32 array -> host int64.  `as_unsigned` zero-extends (the bounds
// list carries a flag in bit 31).
msx_status export_i32(const int32_t *src, int64_t count, int64_t *dst, bool as_unsigned = false) {
  if (dst == nullptr || count <= 0) return MSX_OK;
  int32_t *tmp = new (std::nothrow) int32_t[count];
  if (tmp == nullptr) return fail(MSX_ENOMEM, "msx_csr_plan_export: host allocation failed.");
  hipError_t e = hipMemcpy(tmp, src, sizeof(int32_t) * count, hipMemcpyDeviceToHost);
  if (e == hipSuccess)
    for (int64_t i = 0; i < count; ++i)
      dst[i] = as_unsigned ? static_cast<int64_t>(static_cast<uint32_t>(tmp[i])) : tmp[i];
  delete[] tmp;
  if (e != hipSuccess) return hip_fail(e, "msx_csr_plan_export");
  return MSX_OK;
}
}  // namespace

extern "C" msx_status msx_csr_plan_export(const msx_csr_plan *plan, int64_t *bounds,
                                          int64_t *long_rows, int64_t *long_chunk_begin) {
  clear_error();
  if (plan == nullptr) return fail(MSX_EINVAL, "msx_csr_plan_export: plan is NULL.");
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(plan->device);
  msx_status st = export_i32(plan->bounds, plan->n_bounds + 1, bounds, true);
  if (st == MSX_OK) st = export_i32(plan->long_rows, plan->n_long, long_rows);
  if (st == MSX_OK) st = export_i32(plan->long_chunk_begin, plan->n_long + 1, long_chunk_begin);
  (void)hipSetDevice(prev);
  return st;
}

extern "C" msx_status msx_csr_plan_export_panels(const msx_csr_plan *plan, int64_t *tile_begin,
                                                 int64_t *tile_end, int64_t *seg_begin) {
  clear_error();
  if (plan == nullptr) return fail(MSX_EINVAL, "msx_csr_plan_export_panels: plan is NULL.");
  if (plan->n_panels == 0)
    return fail(MSX_EINVAL, "msx_csr_plan_export_panels: the plan has no panels.");
  int prev = 0;
  (void)hipGetDevice(&prev);
  (void)hipSetDevice(plan->device);
  msx_status st = export_i32(plan->pn_tile_begin, plan->n_tiles, tile_begin);
  if (st == MSX_OK) st = export_i32(plan->pn_tile_end, plan->n_tiles, tile_end);
  if (st == MSX_OK)
    st = export_i32(reinterpret_cast<const int32_t *>(plan->pn_seg),
                    plan->n_panels * plan->n_tiles + 1, seg_begin, true);
  (void)hipSetDevice(prev);
  return st;
}
